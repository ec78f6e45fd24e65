// Skinny (decode-shaped) GEMM for gfx950: C[M <= 16][N] = A[M][K] . B[N][K]^T + bias, fp32 accumulate.
//
// The reference's generated GEMM handles M < BM only through its edge-tile path, which ignores
// split-K (Sources/matmul/matmul.swift:280-295). This kernel is the HBM-bound counterpart: B is
// streamed from HBM exactly once, straight into MFMA operands.
//
// Work decomposition
//   * Workgroup = split_k wavefronts; wavefront w owns K partition w for every column group the
//     workgroup processes. The grid is persistent (at most one workgroup per CU): workgroup b
//     walks the 16-column groups b, b + grid, b + 2 grid, ...
//   * 16x16x32 MFMA, lane (r = lane % 16, q = lane / 16). K step s of a partition covers 32
//     columns of K; lane (r, q) supplies elements 8q .. 8q+7 of that step, of A row r and of
//     B row (group column r). One load instruction therefore reads 64 contiguous bytes of each of
//     16 rows.
//   * A partition of up to kSkinnyResident K steps keeps its A fragments in registers for the
//     whole kernel, so only B is streamed; longer partitions reload A per group (from L2).
//   * The next group's B loads are issued before the current group's MFMAs (two register
//     buffers), so every wavefront keeps a full group of loads in flight while it computes.
//   * Per group, the partitions' fp32 16x16 results meet in LDS (double buffered: one barrier
//     per group); the workgroup sums partitions 0, 1, ... in order, adds the bias and stores.
//   * Raw buffer loads: rows m >= M, columns n >= N and K past the partition read zero.
#include "device.hpp"

namespace mtk {

constexpr int kSkinnyResident = 16;  // K steps (x 32) a partition may keep resident: 512 K

template <int DT, int KS>
struct SkinnyWave {
  // KS = K steps per pass over the partition (<= kSkinnyResident)
  u32x4 a[KS];
  uint32_t arow, k0, k_end;

  __device__ void load_a(rsrc_t ra, int kbase, int lane) {
    const int q = lane >> 4;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = kbase + 32 * s + 8 * q;
      a[s] = buf_load16(ra, k < (int)k_end ? arow + (uint32_t)k * 2u : kOOB);
    }
  }
  __device__ void load_b(rsrc_t rb, u32x4 (&b)[KS], int group, int N, int ldb, int kbase, int lane) const {
    const int n = group * 16 + (lane & 15), q = lane >> 4;
    const uint32_t brow = n < N ? (uint32_t)n * (uint32_t)ldb * 2u : kOOB;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = kbase + 32 * s + 8 * q;
      b[s] = buf_load16(rb, (k < (int)k_end && brow != kOOB) ? brow + (uint32_t)k * 2u : kOOB);
    }
  }
  __device__ f32x4 mma(const u32x4 (&b)[KS], f32x4 acc) const {
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma16x16x32<DT>(a[s], b[s], acc);
    return acc;
  }
};

// Partition results of one group are in LDS; after the barrier the workgroup (64 * split_k
// threads) sums them for the 256 outputs of the group.
template <int DT>
__device__ __forceinline__ void skinny_reduce_store(const mtk_skinny_args &p, float (*red)[256], int group, int tid) {
  for (int e = tid; e < 256; e += (int)blockDim.x) {
    const int m = e >> 4, c = e & 15;
    const int n = group * 16 + c;
    float s = red[0][e];
    for (int w = 1; w < p.split_k; ++w) s += red[w][e];
    if (m < p.M && n < p.N) {
      if (p.has_bias) s += from_bits<DT>(((const uint16_t *)p.bias)[n]);
      ((uint16_t *)p.C)[(size_t)m * p.ldc + n] = to_bits<DT>(s);
    }
  }
}

template <int DT, bool RESIDENT>
__device__ __forceinline__ void skinny_gemm(const mtk_skinny_args &p) {
  // two LDS buffers of [partition][16 x 16] fp32
  __shared__ __attribute__((aligned(16))) float red[2][8][256];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int groups = (p.N + 15) / 16;
  const rsrc_t ra = make_rsrc(p.A, p.a_bytes);
  const rsrc_t rb = make_rsrc(p.B, p.b_bytes);

  constexpr int KS = kSkinnyResident;
  SkinnyWave<DT, KS> sw;
  sw.arow = (lane & 15) < p.M ? (uint32_t)(lane & 15) * (uint32_t)p.lda * 2u : kOOB;
  sw.k0 = (uint32_t)(w * p.k_per_split);
  sw.k_end = (uint32_t)min(p.K, (int)sw.k0 + p.k_per_split);

  // 16x16 accumulator layout: lane (c = lane % 16, g = lane / 16), register r -> row 4g + r, col c.
  auto park = [&](int buf, f32x4 acc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[buf][w][(4 * (lane >> 4) + r) * 16 + (lane & 15)] = acc[r];
  };

  if constexpr (RESIDENT) {
    // the partition fits in KS steps: A stays in registers, B double-buffered across groups
    sw.load_a(ra, (int)sw.k0, lane);
    u32x4 b0[KS], b1[KS];
    int g = blockIdx.x;
    if (g < groups) sw.load_b(rb, b0, g, p.N, p.ldb, (int)sw.k0, lane);
    int buf = 0;
    for (; g < groups; g += 2 * gridDim.x) {
      const int g1 = g + gridDim.x;
      if (g1 < groups) sw.load_b(rb, b1, g1, p.N, p.ldb, (int)sw.k0, lane);
      park(buf, sw.mma(b0, f32x4{}));
      __syncthreads();
      skinny_reduce_store<DT>(p, red[buf], g, tid);
      buf ^= 1;
      if (g1 >= groups) break;
      const int g2 = g1 + gridDim.x;
      if (g2 < groups) sw.load_b(rb, b0, g2, p.N, p.ldb, (int)sw.k0, lane);
      park(buf, sw.mma(b1, f32x4{}));
      __syncthreads();
      skinny_reduce_store<DT>(p, red[buf], g1, tid);
      buf ^= 1;
    }
  } else {
    // long partitions: passes of KS steps, A reloaded per pass (L2-resident: A is M x K)
    int buf = 0;
    for (int g = blockIdx.x; g < groups; g += gridDim.x) {
      f32x4 acc = f32x4{};
      u32x4 b[KS];
      for (int kb = (int)sw.k0; kb < (int)sw.k_end; kb += 32 * KS) {
        sw.load_a(ra, kb, lane);
        sw.load_b(rb, b, g, p.N, p.ldb, kb, lane);
        acc = sw.mma(b, acc);
      }
      park(buf, acc);
      __syncthreads();
      skinny_reduce_store<DT>(p, red[buf], g, tid);
      buf ^= 1;
    }
  }
}

}  // namespace mtk

using namespace mtk;

#define SKINNY(NAME, DT, RES) \
  extern "C" __global__ void __launch_bounds__(512) NAME(const mtk_skinny_args a) { skinny_gemm<DT, RES>(a); }

SKINNY(mtk_skinny_f16, DT_F16, true)
SKINNY(mtk_skinny_bf16, DT_BF16, true)
SKINNY(mtk_skinny_f16_long, DT_F16, false)
SKINNY(mtk_skinny_bf16_long, DT_BF16, false)
