/*
 * mtk.h -- C ABI of the MI355X (gfx950) tensor-op library.
 *
 * Drop-in for the Metal plumbing of liuliu/example_matmul_metal4's tensor-op
 * path. The reference's host code (Swift) does four things around each kernel:
 * kernel-select (build a source / pipeline for a shape), shape/descriptor setup
 * (function constants, buffers, grid), validate, and profile. This header keeps
 * that shape with plain C types so any FFI (Swift modulemap, ctypes, cgo, JNI)
 * can bind it; no HIP or torch types appear in any signature.
 *
 * Each entry point cites the reference interface it replaces (paths relative
 * to the reference repository root).
 *
 * Conventions
 *   - Every call returns an int status: MTK_OK (0) or a negative MTK_ERR_*.
 *     The message for the last failure on the calling thread is returned by
 *     mtk_last_error(). Nothing aborts the process.
 *   - Device pointers are plain void* obtained from mtk_alloc (or any HIP
 *     allocation on the context's device). The caller owns them.
 *   - f16 / bf16 tensors are 16-bit storage; accumulation is fp32.
 *   - One mtk_ctx per host thread. Plans are immutable after creation and may
 *     be shared read-only between threads that use the same context.
 *   - Work is enqueued on the context's stream; mtk_sync waits for it.
 */
#ifndef MTK_H
#define MTK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTK_ABI_VERSION 1

typedef enum {
  MTK_OK = 0,
  MTK_ERR_INVALID = -1,      /* bad argument / descriptor (reference: precondition, NSError code) */
  MTK_ERR_NO_DEVICE = -2,    /* no HIP device (reference: MTLCreateSystemDefaultDevice() == nil) */
  MTK_ERR_UNSUPPORTED = -3,  /* device is not gfx950, or a shape this build does not support */
  MTK_ERR_MODULE = -4,       /* code object missing / corrupt / kernel not found (reference: makeLibrary failure) */
  MTK_ERR_OOM = -5,          /* device allocation failed */
  MTK_ERR_LAUNCH = -6,       /* kernel launch failed */
  MTK_ERR_HIP = -7           /* any other HIP runtime error (reference: commandBuffer.status != .completed) */
} mtk_status;

typedef enum { MTK_F16 = 0, MTK_BF16 = 1, MTK_F32 = 2 } mtk_dtype;

typedef struct mtk_ctx mtk_ctx;
typedef struct mtk_plan mtk_plan;

/* ------------------------------------------------------------------ device / runtime */

typedef struct {
  char name[64];
  char arch[32];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int compute_units;
  int clock_khz;           /* peak engine clock */
  int lds_bytes_per_cu;
  int wavefront_size;
  size_t global_mem_bytes;
  double peak_f16_tflops;  /* dense MFMA f16/bf16 peak = CUs * clock * 4096 FLOP/clk/CU */
} mtk_device_info;

/* Replaces MTLCreateSystemDefaultDevice + supportsFamily(.metal4) + makeCommandQueue +
 * makeLibrary/metallib (Sources/matmul/matmul.swift:349-370; Sources/attention/attention.swift:400-420;
 * Sources/ConvolutionShared/ConvolutionShared.swift:3831-3836, 869-885).
 * code_object_dir: directory holding the mtk_*.hsaco code objects (built by hipcc --genco for
 * gfx950); NULL means $MTK_CODE_OBJECT_DIR, else the directory libmtk.so was loaded from.
 * Returns MTK_ERR_NO_DEVICE without a GPU, MTK_ERR_UNSUPPORTED on a non-gfx950 device. */
int mtk_init(int device, const char *code_object_dir, mtk_ctx **out);
int mtk_destroy(mtk_ctx *ctx);
const char *mtk_last_error(void);
const char *mtk_status_string(int status);
int mtk_device_count(int *count);
int mtk_get_device_info(const mtk_ctx *ctx, mtk_device_info *info);

/* Replaces device.makeBuffer(length:options:.storageModeShared) + contents() copies
 * (Sources/matmul/matmul.swift:392-419; Sources/ConvolutionShared/ConvolutionShared.swift:5102-5136). */
int mtk_alloc(mtk_ctx *ctx, size_t bytes, void **dptr);
int mtk_free(mtk_ctx *ctx, void *dptr);
int mtk_upload(mtk_ctx *ctx, void *dst_device, const void *src_host, size_t bytes);
int mtk_download(mtk_ctx *ctx, void *dst_host, const void *src_device, size_t bytes);
/* Device fill with a 16-bit pattern (a kernel, not hipMemset, so it is graph-capture safe). */
int mtk_fill_u16(mtk_ctx *ctx, void *dst_device, uint16_t value, size_t count);

/* Replaces commandBuffer.commit() + waitUntilCompleted() (matmul.swift:477-478). */
int mtk_sync(mtk_ctx *ctx);

/* Use an external hipStream_t (passed as void*) for all later work, or NULL for the
 * context's own stream. */
int mtk_set_stream(mtk_ctx *ctx, void *hip_stream);

/* ------------------------------------------------------------------ GEMM */

/* Replaces GEMMDimensions / BuildOptions{splitK, swapMN, ...} and the M,N,K function
 * constants (Sources/matmul/matmul.swift:5-16, 232-234, 372-378).
 * C[m][n] = bias[n] + sum_k op(A)[m][k] * op(B)[k][n]
 *   A: trans_a == 0 -> [M][lda] row-major (lda >= K), the reference default;
 *      trans_a != 0 -> [K][lda] (lda >= M, even), the reference's transpose.left
 *      (createSource(transpose: (true, _)), matmul.swift:72-90)
 *   B: trans_b != 0 -> [N][ldb] (the reference default, createSource(transpose: (false, true)),
 *      matmul.swift:366); trans_b == 0 -> [K][ldb]
 *   C: [M][ldc] row-major; bias: [N] (same dtype) or NULL.
 * split_k: 1 = none; >1 = that many K partitions with fp32 partials, summed in partition order
 * with the bias added last (the reference's reduce_sum_2, matmul.swift:298-311, 451-474, without
 * its in-place race); 0 = let the plan choose.
 * tile: 0 = let the plan choose; else 128 or 256 (square MFMA workgroup tile).
 * split_mode (split_k > 1): how the partitions are scheduled; for one partition layout the
 * arithmetic, and so the result, is the same bit for bit:
 *   MTK_SPLIT_AUTO     in-workgroup when the tile grid fills the device and split_k <= 4,
 *                      else two-pass;
 *   MTK_SPLIT_TWO_PASS every partition its own workgroup writing fp32 partials [split_k][M][N],
 *                      then a second kernel sums them and adds the bias (the reference's
 *                      dispatch, matmul.swift:439-474);
 *   MTK_SPLIT_SERIAL   one workgroup per output tile runs the partitions in sequence, keeps the
 *                      running sum of the finished partitions (part of it in the workspace: half
 *                      an fp32 tile per 256x256 output tile, a quarter per 128x128 one; the rest
 *                      on chip) and adds it and the bias in its epilogue: no second kernel
 *                      (split_k <= 4).
 * k_stagger (split_k > 1): partition layout. Partition boundaries of output tile t sit at
 * s * ceil(k_tiles / split_k) + (t % S) - S / 2 K-tiles of 64 (0 < s < split_k), S the span:
 *   0 = the plan's choice (in-workgroup: up to 16, which spreads the tiles' partition ends over
 *       several K-tiles; two-pass: uniform); -1 = uniform (S = 0); > 0 = that span (rounded down
 *       to even and to the largest span that keeps every partition non-empty). */
#define MTK_SPLIT_AUTO 0
#define MTK_SPLIT_TWO_PASS 1
#define MTK_SPLIT_SERIAL 2
typedef struct {
  int M, N, K;
  int lda, ldb, ldc; /* 0 = packed (K or M, K or N, N) */
  int trans_b;
  int dtype;          /* MTK_F16 or MTK_BF16 */
  int has_bias;
  int split_k;
  int tile;
  int trans_a;    /* appended: earlier fields keep their offsets */
  int split_mode; /* MTK_SPLIT_*; appended */
  int k_stagger;  /* appended */
} mtk_gemm_desc;

/* Kernel-select. Replaces createSource(...) + makeLibrary + makeFunction(name:constantValues:) +
 * makeComputePipelineState (matmul.swift:18-329, 364-390). Validates the descriptor. */
int mtk_gemm_plan(mtk_ctx *ctx, const mtk_gemm_desc *desc, mtk_plan **out);

typedef struct {
  const void *A, *B, *bias;
  void *C;
  void *workspace; /* >= mtk_plan_workspace_bytes(plan) bytes, 16-byte aligned, or NULL if 0 */
} mtk_gemm_args;

/* Replaces setBuffer(0..3) + dispatchThreadgroups (+ the reduce_sum_2 encoder)
 * (matmul.swift:427-474). Enqueues; does not wait. */
int mtk_gemm_run(const mtk_plan *plan, const mtk_gemm_args *args);

/* mtk_gemm_run without a caller workspace and without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The plan's workspace (split-K partials or
 * running sums) is a static device array of MTK_NOALLOC_MAX_WORKSPACE bytes inside the library,
 * one per GPU the library is initialised on, held until the process ends; args->workspace must be
 * NULL. Plans whose mtk_plan_workspace_bytes exceeds the maximum return MTK_ERR_UNSUPPORTED (use
 * mtk_gemm_run with a caller workspace). Same kernels and same results, bit for bit, as
 * mtk_gemm_run. Every call on one GPU shares that GPU's array and no kernel needs it cleared
 * (each writes before it reads): calls that overlap on one GPU (several streams or host threads
 * at once) race on it and must be serialised by the caller. */
#define MTK_NOALLOC_MAX_WORKSPACE (64u << 20)
int mtk_gemm_run_noalloc(const mtk_plan *plan, const mtk_gemm_args *args);

/* ------------------------------------------------------------------ attention */

/* Replaces BlockDimenions / AttentionDimensions{R, C, K, Hq, Hk} and the R,C,Hq,Hk function
 * constants (Sources/attention/attention.swift:9-21, 117-120, 423-431).
 * Q, O: [B][S_q][H][D]; K, V: [B][S_kv][H_kv][D] (the reference's [S][H][D] packing,
 * attention.swift:466-468, with a batch dimension). scale = 1/sqrt(D).
 * D (the reference's K, the head dimension: attention.swift:17, 398) is any value from 1 to 256
 * and any multiple of 8 up to MTK_ATTN_MAX_HEAD_DIM (512). The reference covers any K with
 * 128-wide blocks and a masked remainder block (attention.swift:25, 84-91, 192-199); here the
 * forward kernels are compiled for a padded head dimension of 64, 128, 256 or 512 and zero the
 * dims past D. D % 8 == 0 needs 16-byte aligned Q, K, V, O; other D (up to 256) only 2-byte
 * alignment (element-staged kernels, slower). D above 256 runs 64 query rows per workgroup
 * (q_rows must be 0). The backward plan supports every multiple of 8 up to 256
 * (MTK_ERR_UNSUPPORTED otherwise).
 * H_kv (appended; 0 = H) is the reference's Hk: H must be a multiple of it and query head h reads
 * K/V head h / (H / H_kv) (grouped-query attention). The reference declares Hk (attention.swift:20,
 * 131) but slices K and V at the query head (attention.swift:156), so it defines only Hq == Hk,
 * where both mappings agree.
 * causal != 0 keeps keys j <= i + (S_kv - S_q) for query i (bottom-right aligned).
 * q_rows: query rows per workgroup, 0 = let the plan choose; 128 (4 wavefronts of 32 queries, two
 * workgroups per CU) or 256 (8 wavefronts of 32 queries in two groups that alternate MFMA and
 * softmax blocks, one workgroup per CU; D = 128 or 64 only). Same results bit for bit. */
#define MTK_ATTN_MAX_HEAD_DIM 512

typedef struct {
  int B, H, S_q, S_kv, D;
  int causal;
  int dtype;  /* MTK_F16 (MTK_BF16 accepted) */
  int q_rows; /* appended: earlier fields keep their offsets */
  int H_kv;   /* appended: K/V heads, 0 = H */
} mtk_attn_desc;

/* Replaces createSource(blockDimensions:attentionDimensions:buildOptions:) + pipeline setup
 * (attention.swift:23-382, 414-450). */
int mtk_attn_plan(mtk_ctx *ctx, const mtk_attn_desc *desc, mtk_plan **out);

typedef struct {
  const void *Q, *K, *V;
  void *O;
  /* appended: [B][H][S_q] fp32 natural-log log-sum-exp of each query's scaled scores
   * (lse_i = log sum_j exp(q_i . k_j / sqrt(D)), -inf for a query that sees no key), written when
   * not NULL: the backward's input. The reference keeps it in threadgroup memory only
   * (attention.swift:166, 350-352). */
  float *lse;
} mtk_attn_args;

/* Replaces setBuffer(0..3) + setThreadgroupMemoryLength + dispatchThreadgroups
 * (attention.swift:478-501). */
int mtk_attn_run(const mtk_plan *plan, const mtk_attn_args *args);

/* Attention backward: gradients of the loss sum(dO * O) with respect to Q, K and V, the quantities
 * the reference computes on the CPU in Sources/attention/Network.swift:205-281, 313-402
 * (derivativeQ / derivativeK / derivativeV) and has no GPU kernel for:
 *   P = exp(Q K^T / sqrt(D) - lse), D_i = sum_d dO_id O_id, dS = P (dO V^T - D) / sqrt(D),
 *   dV = P^T dO, dK = dS^T Q, dQ = dS K.
 * Same descriptor as the forward (q_rows must be 0); same layouts; causal as in the forward. With
 * H_kv < H, dK and dV of a K/V head sum the contributions of its H / H_kv query heads. The plan
 * needs a workspace of mtk_plan_workspace_bytes (two per-query row terms, D * scale and lse * log2(e), computed by its first kernel). Deterministic: no atomics. */
int mtk_attn_bwd_plan(mtk_ctx *ctx, const mtk_attn_desc *desc, mtk_plan **out);

typedef struct {
  const void *Q, *K, *V, *O, *dO; /* O: the forward's output for these Q, K, V */
  const float *lse;               /* the forward's lse output */
  void *dQ, *dK, *dV;             /* same shapes and dtype as Q, K, V */
  void *workspace;                /* >= mtk_plan_workspace_bytes(plan), 16-byte aligned */
} mtk_attn_bwd_args;

/* Enqueues the three kernels (D-term, dK/dV, dQ). */
int mtk_attn_bwd_run(const mtk_plan *plan, const mtk_attn_bwd_args *args);

/* ------------------------------------------------------------------ convolution */

/* Replaces Conv2DDimensions / Conv3DDimensions (+ the padding fields) and BuildOptions
 * (Sources/ConvolutionShared/ConvolutionShared.swift:5-185).
 * rank 2: x [N][H][W][C], w [KH][KW][C][O] (HWIO), y [N][OH][OW][O]
 * rank 3: x [N][D][H][W][C], w [KD][KH][KW][C][O] (DHWIO), y [N][OD][OH][OW][O]
 * Cross-correlation with stride, dilation and zero padding; output size
 *   OH = (H + pad_top + pad_bottom - ((KH - 1) * dil_h + 1)) / stride_h + 1 (same for W, D).
 * Depth padding (pad_front/pad_back) extends the reference, which has none. bias [O] or NULL.
 * f16 only (the reference's conv path is f16).
 * weight_layout MTK_WEIGHTS_OIDHW: w is [O][C][KD][KH][KW] (rank 2: [O][C][KH][KW]), the layout of
 * the reference's PermuteThenTensorOpSession3D (ConvolutionShared.swift:1676-1857): each run first
 * re-lays the weights out to DHWIO in the caller's workspace (mtk_plan_workspace_bytes, the weight
 * size rounded up to 256 bytes; it must not overlap w), then convolves from there, as the
 * reference's session encodes the permutation and the convolution into one command buffer.
 * There is no in-place OIDHW variant: the implicit GEMM's reduction order must be the same for
 * the activation (channels contiguous per tap) and the weights (taps contiguous per channel in
 * OIDHW), so one of them has to be transposed, and the one-off re-layout (one read and one write
 * of the weights per run) is cheaper than a transpose repeated by every output tile. */
#define MTK_WEIGHTS_DHWIO 0
#define MTK_WEIGHTS_OIDHW 1
typedef struct {
  int rank; /* 2 or 3 */
  int N, D, H, W, C, O;
  int KD, KH, KW;
  int stride_d, stride_h, stride_w;
  int dil_d, dil_h, dil_w;
  int pad_front, pad_back, pad_top, pad_bottom, pad_left, pad_right;
  int has_bias;
  int dtype;         /* MTK_F16 */
  int weight_layout; /* appended: MTK_WEIGHTS_DHWIO (0, the default) or MTK_WEIGHTS_OIDHW */
} mtk_conv_desc;

/* Replaces TensorOpSession / TensorOpSession3D / TensorOpBiasSession3D /
 * TensorOpHorizontalPaddingSession3D init: source generation + pipelines
 * (ConvolutionShared.swift:856-920, 1002-1060, 1282-1336, 1428-1490). One launch for the whole
 * convolution (the reference issues N*OD*KD launches for 3-D). */
int mtk_conv_plan(mtk_ctx *ctx, const mtk_conv_desc *desc, mtk_plan **out);
int mtk_conv_out_shape(const mtk_conv_desc *desc, int *OD, int *OH, int *OW);

typedef struct {
  const void *x, *w, *bias;
  void *y;
  void *workspace;
} mtk_conv_args;

/* Replaces TensorOpSession*.run / runWithoutOutputReadback -> execute (ConvolutionShared.swift:922-965). */
int mtk_conv_run(const mtk_plan *plan, const mtk_conv_args *args);

/* Convolution weight re-layout OIDHW -> DHWIO: replaces permute_oidhw_to_dhwio and
 * WeightPermutationSession3D (Sources/ConvolutionShared/ConvolutionShared.swift:4593-4629,
 * 1577-1674): dst[kd][kh][kw][c][o] = src[o][c][kd][kh][kw], 16-bit elements (f16 or bf16 bits),
 * so PyTorch-style OIDHW (or OIHW with KD = 1) weights can feed mtk_conv_run. Exact copy. */
typedef struct {
  int O, C, KD, KH, KW;
} mtk_permute_desc;

int mtk_permute_plan(mtk_ctx *ctx, const mtk_permute_desc *desc, mtk_plan **out);

typedef struct {
  const void *src; /* [O][C][KD][KH][KW] */
  void *dst;       /* [KD][KH][KW][C][O], must not overlap src */
} mtk_permute_run_args;

int mtk_permute_run(const mtk_plan *plan, const mtk_permute_run_args *args);

/* ------------------------------------------------------------------ plans, validate, profile */

size_t mtk_plan_workspace_bytes(const mtk_plan *plan);
/* Human-readable kernel-select result (kernel names, grid, tile, split-K). */
int mtk_plan_describe(const mtk_plan *plan, char *buf, size_t len);
/* Algorithmic work of one run: FLOPs (2*M*N*K; conv 2*N*OD*OH*OW*O*KD*KH*KW*C with padded taps
 * counted; attention 4*B*H*S_q*S_kv*D, halved-by-mask count for causal) and minimum HBM bytes. */
int mtk_plan_work(const mtk_plan *plan, double *flops, double *bytes);
int mtk_plan_destroy(mtk_plan *plan);

/* Replaces ProfileOptions{warmupIterations, timedIterations, duplicatedCount} and the
 * gpuStartTime/gpuEndTime measurement (ConvolutionShared.swift:237-247, 2522-2539; matmul.swift:480-489).
 * Runs `warmup` untimed iterations, then `iters` timed ones, cycling through `nsets` argument sets
 * (so a large operand can be rotated to defeat the 256 MB Infinity Cache). Each set is the op's
 * args struct (mtk_gemm_args / mtk_attn_args / mtk_attn_bwd_args / mtk_conv_args /
 * mtk_permute_run_args). HIP events on the plan's stream
 * bracket each kernel; results are averages per iteration, in milliseconds. */
typedef struct {
  double total_ms;      /* per iteration, first launch start to last launch end */
  double kernel_ms[4];  /* per iteration, per kernel of the plan, in launch order */
  int n_kernels;
  char kernel_names[4][64];
} mtk_timing;

int mtk_profile(const mtk_plan *plan, const void *arg_sets, int nsets, int warmup, int iters, mtk_timing *out);

/* Repeated runs as one submission: replaces encoding `duplicatedCount` dispatches into one
 * MTLCommandBuffer and committing it once (matmul.swift:447-449, 470-472; attention.swift:498;
 * ConvolutionShared.swift:943-945). mtk_graph_create records `steps` runs of the plan (run i uses
 * argument set i % nsets, each an mtk_*_args struct as for mtk_profile) into a HIP graph on the
 * context's current stream and instantiates it; mtk_graph_launch enqueues all of them at once on
 * that stream (does not wait). Arguments are bound at creation: the buffers must stay valid while
 * the graph exists. The plan's kernels only (no memset nodes). */
typedef struct mtk_graph mtk_graph;
int mtk_graph_create(const mtk_plan *plan, const void *arg_sets, int nsets, int steps, mtk_graph **out);
int mtk_graph_launch(mtk_graph *graph);
int mtk_graph_destroy(mtk_graph *graph);

/* ------------------------------------------------------------------ validate helpers */

/* Compare a device result (16-bit dtype, n elements, on the host) against an fp32 expected
 * vector: relative Frobenius error and max-abs error (the reference's validateOutput /
 * compareOutputs metrics, ConvolutionShared.swift:5174-5322), and the count of elements
 * with |diff| > abs_tol (the reference's mismatch count; its tolerances are 5e-3 GEMM and
 * attention, 2e-2 conv, 0 permutation). */
typedef struct {
  double rel_frobenius;
  double max_abs_error;
  long long mismatches;
} mtk_validation;

int mtk_validate_f16(const uint16_t *actual, int dtype, const float *expected, size_t n, double abs_tol,
                     mtk_validation *out);

#ifdef __cplusplus
}
#endif
#endif
