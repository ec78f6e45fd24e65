// Skinny (decode-shaped) GEMM for gfx950: C[M <= 16][N] = A[M][K] . B[N][K]^T + bias, fp32 accumulate.
//
// The reference's generated GEMM handles M < BM only through its edge-tile path, which ignores
// split-K (Sources/matmul/matmul.swift:280-295). This kernel is the HBM-bound counterpart: B is
// read exactly once, straight from HBM into MFMA operands.
//
// Work decomposition
//   * Workgroup = split_k wavefronts, all on the same 16 output columns; wavefront w owns K
//     partition w. The partition's fp32 16x16 result goes to LDS and wavefront 0 sums the
//     partitions in order, adds the bias and stores (split-K with the reduction on chip: no
//     workspace, no second pass).
//   * 16x16x32 MFMA: lane (n = lane % 16, g = lane / 16). Over a 128-wide K block, lane (n, g)
//     loads 64 contiguous bytes of B row n (4 x 16 B, K offsets 32g .. 32g+31) and the same K
//     range of A row (lane % 16); the four MFMAs of the block use one 16-byte chunk each. Four
//     lanes cover 256 contiguous bytes of a row, so every load instruction is row-coalesced.
//   * Several K blocks are loaded before any MFMA to keep enough bytes in flight for HBM.
//   * Raw buffer loads: rows m >= M and K past the end read zero.
#include "device.hpp"

namespace mtk {

constexpr int kSkinnyKB = 128;   // K per block (4 MFMAs of K = 32)
constexpr int kSkinnyUnroll = 4; // K blocks in flight per wave

template <int DT>
__device__ __forceinline__ void skinny_gemm(const mtk_skinny_args &a) {
  __shared__ __attribute__((aligned(16))) float red[16][16 * 16 + 4];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int n_lane = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = n0 + n_lane;
  const rsrc_t ra = make_rsrc(a.A, a.a_bytes);
  const rsrc_t rb = make_rsrc(a.B, a.b_bytes);
  const uint32_t arow = n_lane < a.M ? (uint32_t)n_lane * (uint32_t)a.lda * 2u : kOOB;
  const uint32_t brow = n < a.N ? (uint32_t)n * (uint32_t)a.ldb * 2u : kOOB;

  const int k_begin = w * a.k_per_split;
  const int k_end = min(a.K, k_begin + a.k_per_split);

  f32x4 acc = f32x4{};
  for (int kb = k_begin; kb < k_end; kb += kSkinnyKB * kSkinnyUnroll) {
    u32x4 av[kSkinnyUnroll][4], bv[kSkinnyUnroll][4];
#pragma unroll
    for (int u = 0; u < kSkinnyUnroll; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int k = kb + u * kSkinnyKB + 32 * g + 8 * t;
        const bool live = k < k_end;
        bv[u][t] = buf_load16(rb, live ? brow + (uint32_t)k * 2u : kOOB);
        av[u][t] = buf_load16(ra, live ? arow + (uint32_t)k * 2u : kOOB);
      }
#pragma unroll
    for (int u = 0; u < kSkinnyUnroll; ++u)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = mfma16x16x32<DT>(av[u][t], bv[u][t], acc);
  }

  // 16x16 accumulator layout: lane (n_lane, g), register r -> row 4g + r, column n_lane.
#pragma unroll
  for (int r = 0; r < 4; ++r) red[w][(4 * g + r) * 16 + n_lane] = acc[r];
  __syncthreads();
  if (w == 0) {
    float s[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = red[0][(4 * g + r) * 16 + n_lane];
    for (int p = 1; p < a.split_k; ++p)
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] += red[p][(4 * g + r) * 16 + n_lane];
    if (n < a.N) {
      const float bv = a.has_bias ? from_bits<DT>(((const uint16_t *)a.bias)[n]) : 0.0f;
      uint16_t *C = (uint16_t *)a.C;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r;
        if (m < a.M) C[(size_t)m * a.ldc + n] = to_bits<DT>(s[r] + bv);
      }
    }
  }
}

}  // namespace mtk

using namespace mtk;

extern "C" __global__ void __launch_bounds__(512) mtk_skinny_f16(const mtk_skinny_args a) { skinny_gemm<DT_F16>(a); }
extern "C" __global__ void __launch_bounds__(512) mtk_skinny_bf16(const mtk_skinny_args a) { skinny_gemm<DT_BF16>(a); }
