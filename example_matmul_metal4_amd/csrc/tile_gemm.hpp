// Tile GEMM for gfx950: C = A . op(B) (+ bias), fp32 accumulate on MFMA 32x32x16.
//
// One template serves the reference's generated GEMM (Sources/matmul/matmul.swift:239-296,
// B stored [N][K] by default, or [K][N]) and the implicit-GEMM convolution that replaces
// the conv2d / conv3d tensor-op kernels (Sources/ConvolutionShared/ConvolutionShared.swift:
// 4431-4591, 4631-4836): for a convolution, A is the im2col view of the NDHWC activation
// (gathered on the fly, padding read as zero) and B is the DHWIO weight tensor seen as [K][O].
//
// Work decomposition
//   * 256 threads = 4 wavefronts (64 lanes) in a WAVES_M x WAVES_N grid; a workgroup owns a
//     BM x BN output tile and K-tiles of 64. Each wave owns (BM/WAVES_M) x (BN/WAVES_N) as
//     32x32 MFMA blocks whose fp32 accumulators stay in registers for the whole K loop.
//   * Global -> registers -> LDS with two LDS buffers: the next K-tile's global loads are in
//     flight while the MFMAs consume the current buffer; one barrier per K-tile.
//   * LDS rows are 64 halves (8 chunks of 16 B); chunk positions are XOR-swizzled with
//     (row & 7) ^ ((row >> 3) & 7) so the 16-byte fragment reads (32 rows x 1 chunk) and the
//     row-wise / transposed stores are bank-conflict free.
//   * All global reads are raw buffer loads: an offset at or past the buffer's range reads 0.
//     Masked elements (K tail, M/N edges, conv padding) are given an out-of-range offset, so
//     the K tail is handled once, in whichever split owns the last K-tile, with no fault risk.
//   * Split-K: workgroup (split, tile) covers K-tiles [split*kps, (split+1)*kps) and writes
//     fp32 partials; a second pass (splitk_reduce) sums the splits in order and adds the bias.
//     Without split-K the bias is fused into the store.
//   * Workgroup ids are remapped so that neighbouring tiles run on the same XCD (shared L2),
//     then rasterised in groups of GROUP_M tile-rows.
#pragma once

#include <type_traits>

#include "device.hpp"

namespace mtk {

enum { A_MK = 0, A_CONV = 1, A_CONV_GENERIC = 2 };
enum { B_NK = 0, B_KN = 1 };

constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kGroupM = 4;

__device__ __forceinline__ uint32_t lds_off(int row, int chunk) {
  return (uint32_t)(row * 128 + ((chunk ^ (row & 7) ^ ((row >> 3) & 7)) << 4));
}

// lds_off(rowblk + lane % 32, 2 * ks + lane / 32) for a row block rowblk that is a multiple of 32
// (the 32x32x16 fragment a lane reads at k-step ks), written as a uniform part plus a per-lane part
// that takes one of four values (k = 2 * ks ^ 4 * (rowblk / 32 % 2)) shared by every row block and
// operand: the compiler keeps four lane offsets, not one per fragment.
__device__ __forceinline__ uint32_t frag_off(int rowblk, int ks, int lane) {
  const int k = (2 * ks) ^ (4 * ((rowblk >> 5) & 1));
  const int t = (lane >> 5) ^ (lane & 7) ^ ((lane >> 3) & 3);
  return (uint32_t)(rowblk * 128) + (uint32_t)((lane & 31) * 128 + ((k ^ t) << 4));
}

// Assemble a 16-byte chunk (8 halves) from 8/V loads of V halves each; off(g) gives the
// byte offset of group g (out of range when masked).
template <int V, typename OffFn>
__device__ __forceinline__ u32x4 load_chunk(rsrc_t r, OffFn off) {
  if constexpr (V == 8) {
    return buf_load16(r, off(0));
  } else if constexpr (V == 4) {
    u32x2 a = buf_load8(r, off(0)), b = buf_load8(r, off(1));
    return u32x4{a.x, a.y, b.x, b.y};
  } else if constexpr (V == 2) {
    return u32x4{buf_load4(r, off(0)), buf_load4(r, off(1)), buf_load4(r, off(2)), buf_load4(r, off(3))};
  } else {
    uint32_t h[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) h[g] = buf_load2(r, off(g));
    return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
  }
}

// ---------------------------------------------------------------- A / B loaders

// Row-major operand, rows x K (A [M][lda], or B [N][ldb] in the NK layout).
template <int ROWS, int V>
struct LoadRows {
  static constexpr int kPer = ROWS / 32;  // 8 chunks per row, 256 threads -> 32 rows per pass
  uint32_t row_off[kPer];
  int chunk;

  __device__ void init(int tid, int row0, int nrows, int ld) {
    chunk = tid & 7;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int row = row0 + (tid >> 3) + 32 * i;
      row_off[i] = row < nrows ? (uint32_t)row * (uint32_t)ld * 2u : kOOB;
    }
  }
  __device__ void load(rsrc_t r, int kt, int K, u32x4 *out) const {
    const int k = kt * kBK + chunk * 8;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      out[i] = load_chunk<V>(r, [&](int g) {
        const int kk = k + g * V;
        return kk < K ? row_off[i] + (uint32_t)kk * 2u : kOOB;
      });
    }
  }
  __device__ void store(char *lds, int tid, const u32x4 *in) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) *(u32x4 *)(lds + lds_off((tid >> 3) + 32 * i, chunk)) = in[i];
  }
};

// [K][ld] operand (B in the KN layout, conv weights): 8x8 blocks are transposed in registers
// so LDS holds the tile K-contiguous, [COLS][64], like the row-major operands.
template <int COLS, int V>
struct LoadColsT {
  static constexpr int kNB = COLS / 8;
  static constexpr int kBlocks = 8 * kNB;
  static constexpr int kPer = (kBlocks + kThreads - 1) / kThreads;
  int kb[kPer], nb[kPer];
  int n0;

  __device__ void init(int tid, int col0) {
    n0 = col0;
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int b = tid + kThreads * p;
      kb[p] = b / kNB;
      nb[p] = b % kNB;
    }
  }
  __device__ void load(rsrc_t r, int kt, int K, int N, int ld, u32x4 *out, int tid) const {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      if (kBlocks % kThreads != 0 && tid + kThreads * p >= kBlocks) continue;
      u32x4 raw[8];
      const int n = n0 + nb[p] * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = kt * kBK + kb[p] * 8 + i;
        raw[i] = load_chunk<V>(r, [&](int g) {
          const int nn = n + g * V;
          return (k < K && nn < N) ? ((uint32_t)k * (uint32_t)ld + (uint32_t)nn) * 2u : kOOB;
        });
      }
      // out chunk j = column n+j, k = kb*8 .. kb*8+7
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = j >> 1;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          w[q] = (j & 1) ? pack_hi(raw[2 * q][d], raw[2 * q + 1][d]) : pack_lo(raw[2 * q][d], raw[2 * q + 1][d]);
        out[p * 8 + j] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
  }
  __device__ void store(char *lds, int tid, const u32x4 *in) const {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      if (kBlocks % kThreads != 0 && tid + kThreads * p >= kBlocks) continue;
#pragma unroll
      for (int j = 0; j < 8; ++j) *(u32x4 *)(lds + lds_off(nb[p] * 8 + j, kb[p])) = in[p * 8 + j];
    }
  }
};

// Implicit-GEMM activation gather. Row m = (n, oz, oh, ow) of the output, column
// k = ((kd*KH + kh)*KW + kw)*C + c. Per row the valid taps are kept as three bit masks
// (depth, height, width) built once; out-of-range taps read zero (padding).
template <int ROWS, int V, bool FAST>
struct LoadConv {
  static constexpr int kPer = ROWS / 32;
  int pbase[kPer];  // element offset of (n, oz*SZ-PF, oh*SY-PT, ow*SX-PL, 0); may be negative
  uint32_t mz[kPer], mh[kPer], mw[kPer];
  int chunk;

  __device__ void init(const mtk_tile_args &a, int tid, int row0) {
    chunk = tid & 7;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int m = row0 + (tid >> 3) + 32 * i;
      uint32_t z = 0, h = 0, w = 0;
      int base = 0;
      if (m < a.M) {
        const int ow = m % a.cOW;
        const int t1 = m / a.cOW;
        const int oh = t1 % a.cOH;
        const int t2 = t1 / a.cOH;
        const int oz = t2 % a.cOD;
        const int n = t2 / a.cOD;
        const int iz0 = oz * a.cSZ - a.cPF, ih0 = oh * a.cSY - a.cPT, iw0 = ow * a.cSX - a.cPL;
        for (int t = 0; t < a.cKD; ++t) z |= (unsigned)(iz0 + t * a.cDZ >= 0 && iz0 + t * a.cDZ < a.cD) << t;
        for (int t = 0; t < a.cKH; ++t) h |= (unsigned)(ih0 + t * a.cDY >= 0 && ih0 + t * a.cDY < a.cH) << t;
        for (int t = 0; t < a.cKW; ++t) w |= (unsigned)(iw0 + t * a.cDX >= 0 && iw0 + t * a.cDX < a.cW) << t;
        base = (((n * a.cD + iz0) * a.cH + ih0) * a.cW + iw0) * a.cC;
      }
      pbase[i] = base;
      mz[i] = z;
      mh[i] = h;
      mw[i] = w;
    }
  }

  __device__ __forceinline__ uint32_t group_off(const mtk_tile_args &a, int i, int kd, int kh, int kw,
                                                int tap_elems) const {
    const bool ok = (mz[i] >> kd) & (mh[i] >> kh) & (mw[i] >> kw) & 1u;
    return ok ? (uint32_t)(pbase[i] + tap_elems) * 2u : kOOB;
  }

  __device__ void load(rsrc_t r, const mtk_tile_args &a, int kt, u32x4 *out) const {
    if constexpr (FAST) {
      // C % 64 == 0: the whole K-tile lies in one tap; the tap decode is uniform.
      const int k0 = kt * kBK;
      const int tap = k0 / a.cC;
      const int c = k0 - tap * a.cC + chunk * 8;
      const int kw = tap % a.cKW;
      const int kh = (tap / a.cKW) % a.cKH;
      const int kd = tap / (a.cKW * a.cKH);
      const bool live = k0 < a.K;
      const int tap_elems = ((kd * a.cDZ * a.cH + kh * a.cDY) * a.cW + kw * a.cDX) * a.cC + c;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const uint32_t o = live ? group_off(a, i, kd, kh, kw, tap_elems) : kOOB;
        out[i] = buf_load16(r, o);
      }
    } else {
      int kd[8 / V], kh[8 / V], kw[8 / V], te[8 / V];
      bool live[8 / V];
#pragma unroll
      for (int g = 0; g < 8 / V; ++g) {
        const int k = kt * kBK + chunk * 8 + g * V;
        const int tap = k / a.cC;
        const int c = k - tap * a.cC;
        kw[g] = tap % a.cKW;
        kh[g] = (tap / a.cKW) % a.cKH;
        kd[g] = tap / (a.cKW * a.cKH);
        live[g] = k < a.K;
        te[g] = ((kd[g] * a.cDZ * a.cH + kh[g] * a.cDY) * a.cW + kw[g] * a.cDX) * a.cC + c;
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        out[i] = load_chunk<V>(r, [&](int g) { return live[g] ? group_off(a, i, kd[g], kh[g], kw[g], te[g]) : kOOB; });
      }
    }
  }
  __device__ void store(char *lds, int tid, const u32x4 *in) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) *(u32x4 *)(lds + lds_off((tid >> 3) + 32 * i, chunk)) = in[i];
  }
};

template <int AKIND, int ROWS, int V>
struct ASel;
template <int ROWS, int V>
struct ASel<A_MK, ROWS, V> {
  using T = LoadRows<ROWS, V>;
};
template <int ROWS, int V>
struct ASel<A_CONV, ROWS, V> {
  using T = LoadConv<ROWS, V, true>;
};
template <int ROWS, int V>
struct ASel<A_CONV_GENERIC, ROWS, V> {
  using T = LoadConv<ROWS, V, false>;
};

// ---------------------------------------------------------------- the kernel body

// First K-tile of split-K partition s of a tile (s = split_k: one past the last). Every
// partition is non-empty: the plan picks split_k = ceil(k_tiles / k_tiles_per_split).
// First K-tile of split-K partition s of output tile t (partition split_k ends at k_tiles).
// Interior boundaries move by a per-tile offset in [-k_stagger/2, k_stagger/2) (the host keeps
// every partition non-empty).
__device__ __forceinline__ int split_first_tile(const mtk_tile_args &a, int s, int t) {
  if (s <= 0) return 0;
  if (s >= a.split_k) return a.k_tiles;
  const int off = a.k_stagger > 1 ? t % a.k_stagger - a.k_stagger / 2 : 0;
  return s * a.k_tiles_per_split + off;
}

template <int DT, int BM, int BN, int WAVES_M, int WAVES_N, int AKIND, int BKIND, int VA, int VB>
__device__ __forceinline__ void tile_gemm(const mtk_tile_args &a) {
  static_assert(WAVES_M * WAVES_N == 4, "4 wavefronts per workgroup");
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32-aligned");
  constexpr int kStage = (BM + BN) * 128;  // bytes per LDS stage

  __shared__ __attribute__((aligned(16))) char smem[2 * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_m = wave / WAVES_N, wave_n = wave % WAVES_N;

  // ---- which tile / split
  const int tiles = a.tiles_m * a.tiles_n;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int split = id / tiles;
  const int t = id - split * tiles;
  const int group = kGroupM * a.tiles_n;
  const int first_m = (t / group) * kGroupM;
  const int gm = min(a.tiles_m - first_m, kGroupM);
  const int tm = first_m + (t % group) % gm;
  const int tn = (t % group) / gm;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kt0 = split_first_tile(a, split, t);
  const int kt1 = split_first_tile(a, split + 1, t);

  const rsrc_t ra = make_rsrc(a.A, a.a_bytes);
  const rsrc_t rb = make_rsrc(a.B, a.b_bytes);

  typename ASel<AKIND, BM, VA>::T la;
  if constexpr (AKIND == A_MK) {
    la.init(tid, m0, a.M, a.lda);
  } else {
    la.init(a, tid, m0);
  }
  constexpr int NA = BM / 32;
  u32x4 rga[NA];

  using LB = typename std::conditional<BKIND == B_NK, LoadRows<BN, VB>, LoadColsT<BN, VB>>::type;
  LB lb;
  if constexpr (BKIND == B_NK) {
    lb.init(tid, n0, a.N, a.ldb);
  } else {
    lb.init(tid, n0);
  }
  constexpr int NB = (BKIND == B_NK) ? BN / 32 : LoadColsT<BN, 1>::kPer * 8;
  u32x4 rgb[NB];

  auto gload = [&](int kt) {
    if constexpr (AKIND == A_MK) {
      la.load(ra, kt, a.K, rga);
    } else {
      la.load(ra, a, kt, rga);
    }
    if constexpr (BKIND == B_NK) {
      lb.load(rb, kt, a.K, rgb);
    } else {
      lb.load(rb, kt, a.K, a.N, a.ldb, rgb, tid);
    }
  };
  auto lstore = [&](int s) {
    la.store(smem + s * kStage, tid, rga);
    lb.store(smem + s * kStage + BM * 128, tid, rgb);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

  // Fragment rows and the lane's chunk half within each 16-wide k step.
  const int frow = lane & 31;
  const int fhalf = lane >> 5;

  gload(kt0);
  lstore(0);
  __syncthreads();

  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) gload(kt + 1);
    const char *sa = smem + cur * kStage;
    const char *sb = sa + BM * 128;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      u32x4 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *(const u32x4 *)(sa + lds_off(wave_m * WTM + i * 32 + frow, 2 * ks + fhalf));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *(const u32x4 *)(sb + lds_off(wave_n * WTN + j * 32 + frow, 2 * ks + fhalf));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16<DT>(fa[i], fb[j], acc[i][j]);
    }
    if (more) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue. 32x32 accumulator layout: lane l, register r holds
  //      row 8*(r/4) + 4*(l/32) + r%4, column l%32 of its block.
  const int col_l = lane & 31;
  const int row_l = 4 * (lane >> 5);
  if (a.partial != nullptr) {
    float *P = a.partial + (size_t)split * a.M * a.N;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wave_n * WTN + j * 32 + col_l;
      if (col >= a.N) continue;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wave_m * WTM + i * 32 + 8 * (r >> 2) + row_l + (r & 3);
          if (row < a.M) P[(size_t)row * a.N + col] = acc[i][j][r];
        }
    }
  } else {
    uint16_t *C = (uint16_t *)a.C;
    const uint16_t *bias = (const uint16_t *)a.bias;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + wave_n * WTN + j * 32 + col_l;
      if (col >= a.N) continue;
      const float bv = a.has_bias ? from_bits<DT>(bias[col]) : 0.0f;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wave_m * WTM + i * 32 + 8 * (r >> 2) + row_l + (r & 3);
          if (row < a.M) C[(size_t)row * a.ldc + col] = to_bits<DT>(acc[i][j][r] + bv);
        }
    }
  }
}

// Second pass of split-K: C[m][n] = (sum over splits, in order) + bias[n], rounded once.
// HBM-bound: reads the split_k fp32 partials once (non-temporally: they are streamed once each
// way) and writes C once. Vector path (N, ldc % 4 == 0; C and bias 8-byte aligned): a thread owns 4
// consecutive outputs and issues its S 16-byte loads at once (split count unrolled for 2..8).
// Measured on MI355X at config 2 (4 x 64 MiB of partials): 4 outputs per thread 55.9 us, 8 per
// thread 59 us, 16 per thread 88 us.
template <int DT, int S>
__device__ __forceinline__ void splitk_reduce4(const mtk_reduce_args &a) {
  const uint16_t *bias = (const uint16_t *)a.bias;
  uint16_t *C = (uint16_t *)a.C;
  const size_t plane = (size_t)a.M * a.N;
  const size_t groups = plane / 4;
  for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += (size_t)gridDim.x * blockDim.x) {
    const size_t e = g * 4;
    const int m = (int)(e / a.N), n = (int)(e % a.N);
    f32x4 v[S];
#pragma unroll
    for (int s = 0; s < S; ++s) v[s] = __builtin_nontemporal_load((const f32x4 *)(a.partial + s * plane + e));
    f32x4 acc = v[0];
#pragma unroll
    for (int s = 1; s < S; ++s) acc += v[s];
    if (a.has_bias) {
      const u32x2 b = *(const u32x2 *)(bias + n);
      acc += f32x4{from_bits<DT>(b.x & 0xffff), from_bits<DT>(b.x >> 16), from_bits<DT>(b.y & 0xffff),
                   from_bits<DT>(b.y >> 16)};
    }
    *(u32x2 *)(C + (size_t)m * a.ldc + n) = u32x2{pack2<DT>(acc.x, acc.y), pack2<DT>(acc.z, acc.w)};
  }
}

// More than 8 splits (the reference's own default run uses 30): the partial loads go out in batches
// of 8 so that 8 are in flight per thread instead of one; the sum keeps the split order.
template <int DT, int V>
__device__ __forceinline__ void splitk_reduce_batched(const mtk_reduce_args &a) {
  using vec = typename std::conditional<V == 4, f32x4, float>::type;
  const uint16_t *bias = (const uint16_t *)a.bias;
  uint16_t *C = (uint16_t *)a.C;
  const size_t plane = (size_t)a.M * a.N;
  const size_t groups = plane / V;
  for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += (size_t)gridDim.x * blockDim.x) {
    const size_t e = g * V;
    const int m = (int)(e / a.N), n = (int)(e % a.N);
    vec acc{};
    for (int s0 = 0; s0 < a.split_k; s0 += 8) {
      vec v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < a.split_k) v[u] = __builtin_nontemporal_load((const vec *)(a.partial + (s0 + u) * plane + e));
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < a.split_k) acc = (s0 + u == 0) ? v[u] : acc + v[u];
    }
    if constexpr (V == 4) {
      if (a.has_bias) {
        const u32x2 b = *(const u32x2 *)(bias + n);
        acc += f32x4{from_bits<DT>(b.x & 0xffff), from_bits<DT>(b.x >> 16), from_bits<DT>(b.y & 0xffff),
                     from_bits<DT>(b.y >> 16)};
      }
      *(u32x2 *)(C + (size_t)m * a.ldc + n) = u32x2{pack2<DT>(acc.x, acc.y), pack2<DT>(acc.z, acc.w)};
    } else {
      if (a.has_bias) acc += from_bits<DT>(bias[n]);
      C[(size_t)m * a.ldc + n] = to_bits<DT>(acc);
    }
  }
}

template <int DT>
__device__ __forceinline__ void splitk_reduce(const mtk_reduce_args &a) {
  if (a.vec4) {
    switch (a.split_k) {
      case 2: return splitk_reduce4<DT, 2>(a);
      case 3: return splitk_reduce4<DT, 3>(a);
      case 4: return splitk_reduce4<DT, 4>(a);
      case 5: return splitk_reduce4<DT, 5>(a);
      case 6: return splitk_reduce4<DT, 6>(a);
      case 7: return splitk_reduce4<DT, 7>(a);
      case 8: return splitk_reduce4<DT, 8>(a);
      default: return splitk_reduce_batched<DT, 4>(a);
    }
  }
  splitk_reduce_batched<DT, 1>(a);
}

}  // namespace mtk
