/*
 * Kernel argument blocks, shared verbatim by the host runtime (runtime.cpp)
 * and the device code objects (*.hip). Each kernel takes exactly one of these
 * structs by value; the host passes it through hipModuleLaunchKernel.
 * Plain C: fixed-width integers and raw device pointers only.
 */
#ifndef MTK_KARGS_H
#define MTK_KARGS_H

#include <stdint.h>

#define MTK_KARGS_VERSION 11

/* In-workgroup split-K: bytes of workspace slot per output tile of BM x BM (256 or 128). Each
 * wavefront keeps these accumulator blocks (32 x 32 fp32, 4 KB) of its running sum in the slot,
 * the others in registers and LDS: 256x256 tiles, 8 wavefronts x 4 blocks; 128x128 tiles,
 * 4 wavefronts x 1 block. */
#define MTK_SERIAL_SLOT_BYTES(BM) ((BM) == 256 ? 8 * 4 * 4096 : 4 * 1 * 4096)

/* Tile-GEMM kernels: plain GEMM (A [M][K] . B, B either [N][K] or [K][N]) and
 * implicit-GEMM convolution (A = im2col of an NDHWC activation, B = DHWIO
 * weights viewed as [K][O]), one template. */
typedef struct {
  const void *A;    /* GEMM: [M][lda] ; conv: activation NDHWC */
  const void *B;    /* [N][ldb] (NK) or [K][ldb] (KN) */
  const void *bias; /* [N] or NULL */
  void *C;          /* [M][ldc] output (f16/bf16), or NULL when writing partials */
  float *partial;   /* two-pass split-K: [split_k][M][N] fp32 partials (C NULL);
                       in-workgroup split-K (*_s kernels): [tiles][MTK_SERIAL_SLOT_BYTES(BM)]
                       the part of each tile's running sum kept in the workspace (C set);
                       else NULL */
  int32_t M, N, K;
  int32_t lda, ldb, ldc;
  uint32_t a_bytes, b_bytes; /* buffer-resource ranges: loads at or past these byte offsets return 0 */
  int32_t tiles_m, tiles_n;
  int32_t k_tiles;          /* ceil(K / 64) */
  int32_t k_tiles_per_split;
  int32_t split_k;
  int32_t has_bias;
  /* Split-K partition boundaries of output tile t: s * k_tiles_per_split + (t % k_stagger) -
     k_stagger / 2 for 0 < s < split_k (0 when k_stagger < 2). Staggering spreads the tiles'
     partition ends over several K-tiles while every tile still walks K in the same order. */
  int32_t k_stagger;
  /* implicit-GEMM convolution geometry (unused by plain GEMM) */
  int32_t cN, cD, cH, cW, cC;
  int32_t cKD, cKH, cKW;
  int32_t cSZ, cSY, cSX;
  int32_t cDZ, cDY, cDX;
  int32_t cPF, cPT, cPL;
  int32_t cOD, cOH, cOW;
} mtk_tile_args;

/* Second pass of split-K: out[m][n] = sum_s partial[s][m][n] + bias[n]. */
typedef struct {
  const float *partial;
  const void *bias;
  void *C;
  int32_t M, N, ldc;
  int32_t split_k;
  int32_t has_bias;
  int32_t vec4; /* 1: N, ldc multiple of 4 and C, bias 8-byte aligned -> 4-wide path */
} mtk_reduce_args;

/* 16-bit fill (zeroing workspaces inside a plan; graph-capturable, unlike hipMemsetAsync). */
typedef struct {
  void *p;
  uint64_t n; /* elements */
  uint32_t v;
} mtk_fill_args;

/* Skinny (decode-shaped) GEMM: A [M <= 16][lda] (M <= 32 for the partial-writing kernel), B [N][ldb] (NK);
   partial: that kernel's output, [split_k][M][N] fp32. */
typedef struct {
  const void *A;
  const void *B;
  const void *bias;
  void *C;
  float *partial;
  int32_t M, N, K;
  int32_t lda, ldb, ldc;
  uint32_t a_bytes, b_bytes;
  int32_t split_k;
  int32_t k_per_split; /* multiple of the kernel's K step */
  int32_t has_bias;
} mtk_skinny_args;

/* Flash-attention forward, Q/K/V/O laid out [B][S][H][D]; the kernel is compiled for a padded head
   dimension (64, 128 or 256) and runs any D up to it. */
typedef struct {
  const void *Q;
  const void *K;
  const void *V;
  void *O;
  int32_t B, H, S_q, S_kv;
  int32_t q_blocks;  /* ceil(S_q / query rows per workgroup) */
  int32_t causal;
  float scale_log2; /* log2(e) / sqrt(D) */
  uint32_t q_bytes, kv_bytes;
  float *lse; /* [B][H][S_q] natural-log row log-sum-exp of the scaled scores, or NULL */
  int32_t H_kv; /* K/V heads (divides H): query head h reads K/V head h / (H / H_kv) */
  int32_t D;    /* head dimension */
} mtk_attn_kargs;

/* Flash-attention backward (all three kernels of the plan take this block). */
typedef struct {
  const void *Q, *K, *V, *O, *dO;
  const float *lse; /* [B][H][S_q] from the forward */
  float *Dt;        /* [B][H][S_q] workspace: rowsum(dO * O) * scale */
  void *dQ, *dK, *dV;
  int32_t B, H, S_q, S_kv;
  int32_t H_kv;     /* K/V heads (divides H); dK, dV sum over the H / H_kv query heads of a group */
  int32_t q_blocks; /* ceil(S_q / 256): dQ workgroups per (batch, head) */
  int32_t k_blocks; /* ceil(S_kv / 128): dK/dV workgroups per (batch, head) */
  int32_t causal;
  float scale_log2; /* log2(e) / sqrt(D) */
  float scale;      /* 1 / sqrt(D) */
  uint32_t q_bytes, kv_bytes;
  float *Lt; /* [B][H][S_q] workspace: lse * log2(e) (base-2 log-sum-exp) */
  int32_t D; /* head dimension: a multiple of 8 up to the kernel's padded head dimension */
} mtk_attn_bwd_kargs;

/* Convolution weight re-layout OIDHW -> DHWIO (16-bit elements). */
typedef struct {
  const void *src; /* [O][C][KD][KH][KW] */
  void *dst;       /* [KD][KH][KW][C][O] */
  int32_t O, C, T; /* T = KD * KH * KW */
} mtk_permute_args;

#endif
