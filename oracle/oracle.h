/*
 * CPU oracle for the tensor-op path: TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference's CPU validation loops. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker; the product (libmtk.so + its code object)
 * never links or calls it.
 *
 * Sources restated (all paths under the reference repo):
 *   GEMM      Sources/matmul/matmul.swift:498-510        (fp32, bias first, i inner)
 *   attention Sources/attention/Network.swift:134-179, 286-311
 *   attention backward  Sources/attention/Network.swift:205-281 (dP, D-term, dS rows),
 *             313-402 (dV = P^T dO, dK = dS^T Q, dQ = dS K)
 *   conv2d    Sources/ConvolutionShared/ConvolutionShared.swift:4994-5026
 *   conv3d    Sources/ConvolutionShared/ConvolutionShared.swift:5028-5068
 *   conv+bias Sources/ConvolutionShared/ConvolutionShared.swift:5070-5096
 *   weight re-layout  Sources/ConvolutionShared/ConvolutionShared.swift:4606-4627 (OIDHW -> DHWIO)
 *   padded    Sources/convolution2d_padding/convolution2d_padding.swift:79-107,
 *             Sources/convolution3d_padding/convolution3d_padding.swift:202-242
 *
 * Extensions beyond the reference (closed-form generalisations, pinned in
 * tests/test_oracle.py): bf16 inputs, transB=false GEMM, attention batch and
 * causal mask, conv2d bias, conv3d depth padding.
 *
 * Storage: f16/bf16 tensors are uint16_t bit patterns; accumulation and
 * outputs are fp32 ("float"), exactly as the Swift loops accumulate in Float.
 */
#ifndef MTK_ORACLE_H
#define MTK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F16 = 0, ORACLE_BF16 = 1 };

/* ---- scalar conversions (round-to-nearest-even, written from the IEEE formats) */
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float x);
float oracle_bf16_to_f32(uint16_t h);
void oracle_to_f32(int dtype, const uint16_t *src, float *dst, size_t n);
void oracle_from_f32(int dtype, const float *src, uint16_t *dst, size_t n);

/* ---- seeded inputs: SplitMix64 stream -> fp64 -> RNE to dtype */
void oracle_fill_uniform(uint64_t seed, double lo, double hi, int dtype, uint16_t *out, size_t n);
void oracle_fill_normal(uint64_t seed, double mean, double stddev, int dtype, uint16_t *out, size_t n);

/* ---- GEMM: C[m][n] = bias[n] + sum_i A[m][i] * B(i, n)
 * A is [M][K] row-major. trans_b != 0: B is [N][K] (the reference default,
 * matmul.swift:366, CPU check :503); trans_b == 0: B is [K][N].
 * Rows [row_begin, row_end) of C ([M][N], fp32) are written. */
void oracle_gemm(int dtype, int M, int N, int K, int trans_b, const uint16_t *A, const uint16_t *B,
                 const uint16_t *bias, float *C, int row_begin, int row_end, int nthreads);

/* ---- attention forward, layout [B][S][H][D] for Q/O, [B][S][Hkv][D] for K/V (query head h reads
 * K/V head h / (H / Hkv); Hkv divides H).
 * Query rows [q_begin, q_end) of every (b, h) are written (O is full size).
 * causal != 0 keeps keys j <= i + (S_kv - S_q). */
void oracle_attention(int dtype, int B, int H, int Hkv, int S_q, int S_kv, int D, int causal, const uint16_t *Q,
                      const uint16_t *K, const uint16_t *V, float *O, int q_begin, int q_end, int nthreads);

/* ---- attention backward (gradients of the reference's loss Phi = sum dO * O), layout
 * [B][S][H][D] for Q/dO/dQ and [B][S][Hkv][D] for K/V/dK/dV (fp32 outputs); heads grouped as in
 * oracle_attention, dK/dV summing over the group's query heads. The (b, hk) pairs with flat index
 * b*Hkv + hk in [bh_begin, bh_end) are computed (bh_end < 0: all), each with all its query heads;
 * their slices of dQ/dK/dV are overwritten, other slices are left alone. Dterm ([B][H][S_q] fp32,
 * the row sums dO . O with O = P.V in fp32) may be NULL. causal != 0 as in oracle_attention. */
void oracle_attention_bwd(int dtype, int B, int H, int Hkv, int S_q, int S_kv, int D, int causal, const uint16_t *Q,
                          const uint16_t *K, const uint16_t *V, const uint16_t *dO, float *dQ, float *dK, float *dV,
                          float *Dterm, int bh_begin, int bh_end, int nthreads);

/* ---- convolution (cross-correlation), NDHWC activation, DHWIO weights,
 * NDHWC output. A 2-D convolution is D = KD = 1 with no depth padding. */
typedef struct {
  int N, D, H, W, C, O;
  int KD, KH, KW;
  int SZ, SY, SX;
  int DZ, DY, DX;
  int PF, PBk, PT, PB, PL, PR; /* front/back (depth), top/bottom, left/right */
} oracle_conv_dims;

int oracle_conv_out_d(const oracle_conv_dims *d);
int oracle_conv_out_h(const oracle_conv_dims *d);
int oracle_conv_out_w(const oracle_conv_dims *d);
/* Output rows (n, oz, oh) with flat index in [row_begin, row_end) are written;
 * row_end < 0 means all rows. bias may be NULL. */
void oracle_conv(const oracle_conv_dims *d, const uint16_t *x, const uint16_t *w, const uint16_t *bias, float *y,
                 long row_begin, long row_end, int nthreads);

/* ---- weight re-layout: dst[((kd*KH + kh)*KW + kw)*C + c)*O + o] = src[(((o*C + c)*KD + kd)*KH + kh)*KW + kw],
 * 16-bit elements, destination visited in order as the reference's kernel does. */
void oracle_permute_oidhw_to_dhwio(const uint16_t *src, uint16_t *dst, int O, int C, int KD, int KH, int KW);

#ifdef __cplusplus
}
#endif
#endif
