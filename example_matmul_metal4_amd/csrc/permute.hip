// Convolution weight re-layout OIDHW -> DHWIO for gfx950 (16-bit elements; HBM-bound copy).
//
// Replaces the reference's permute_oidhw_to_dhwio kernel (Sources/ConvolutionShared/
// ConvolutionShared.swift:4593-4629, driven by WeightPermutationSession3D, 1577-1674):
//   dst[((kd * KH + kh) * KW + kw) * C + c) * O + o] = src[(((o * C + c) * KD + kd) * KH + kh) * KW + kw]
// With T = KD*KH*KW taps, the source is a matrix [O][C*T] whose column ct = c*T + t goes to
// destination row t*C + c: a tiled transpose. A workgroup moves a 64 (o) x 64 (ct) tile through LDS:
// each source row segment is read contiguously (128 B), each destination row segment of 64
// output channels is written contiguously (128 B). The reference maps one thread to one destination
// element, reading with a stride of C*T elements.
#include "device.hpp"

namespace mtk {

constexpr int kPT = 64;  // tile edge (elements)

// VEC: 16-byte accesses (C*T and O multiples of 8, buffers 16-byte aligned); else 2-byte accesses.
template <bool VEC>
__device__ __forceinline__ void permute_oidhw_dhwio(const mtk_permute_args &a) {
  // [ct][o] in LDS, rows padded by 8 elements (16 bytes) to keep the transposed accesses spread
  // over the banks
  __shared__ __attribute__((aligned(16))) uint16_t tile[kPT][kPT + 8];
  const int CT = a.C * a.T;
  const int tiles_ct = (CT + kPT - 1) / kPT;
  const int o0 = (int)(blockIdx.x / tiles_ct) * kPT;
  const int ct0 = (int)(blockIdx.x % tiles_ct) * kPT;
  const int tid = threadIdx.x;  // 256 threads
  const uint16_t *src = (const uint16_t *)a.src;
  uint16_t *dst = (uint16_t *)a.dst;

  if constexpr (VEC) {
    // read: thread -> source row o0 + tid / 8 (and + 32), 8 elements at ct0 + 8 (tid % 8)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = tid / 8 + 32 * h, cc = 8 * (tid % 8);
      const int o = o0 + r, ct = ct0 + cc;
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (o < a.O && ct < CT) v = *(const u32x4 *)(src + (size_t)o * CT + ct);
#pragma unroll
      for (int e = 0; e < 8; ++e) tile[cc + e][r] = (uint16_t)((e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xffffu));
    }
    __syncthreads();
    // write: thread -> destination row of column ct0 + tid / 8 (and + 32), 8 output channels
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = tid / 8 + 32 * h, oo = 8 * (tid % 8);
      const int ct = ct0 + r, o = o0 + oo;
      if (ct < CT && o < a.O) {
        const int c = ct / a.T, t = ct - c * a.T;
        const u32x4 v = *(const u32x4 *)&tile[r][oo];
        *(u32x4 *)(dst + ((size_t)t * a.C + c) * a.O + o) = v;
      }
    }
  } else {
    // read: thread -> column ct0 + tid % 64 of rows o0 + tid / 64 + 4 i
    for (int i = 0; i < kPT / 4; ++i) {
      const int r = tid / kPT + 4 * i, cc = tid % kPT;
      const int o = o0 + r, ct = ct0 + cc;
      tile[cc][r] = (o < a.O && ct < CT) ? src[(size_t)o * CT + ct] : (uint16_t)0;
    }
    __syncthreads();
    for (int i = 0; i < kPT / 4; ++i) {
      const int r = tid / kPT + 4 * i, oo = tid % kPT;
      const int ct = ct0 + r, o = o0 + oo;
      if (ct < CT && o < a.O) {
        const int c = ct / a.T, t = ct - c * a.T;
        dst[((size_t)t * a.C + c) * a.O + o] = tile[r][oo];
      }
    }
  }
}

}  // namespace mtk

using namespace mtk;

extern "C" __global__ void __launch_bounds__(256) mtk_permute_oidhw_dhwio_v8(const mtk_permute_args a) {
  permute_oidhw_dhwio<true>(a);
}
extern "C" __global__ void __launch_bounds__(256) mtk_permute_oidhw_dhwio_v1(const mtk_permute_args a) {
  permute_oidhw_dhwio<false>(a);
}
