// Flash-attention forward for head dimensions above 256 (multiples of 8 up to 512), gfx950,
// fp16/bf16 in and out, fp32 softmax and accumulation. The reference runs any head dimension K by
// tiling it in 128-wide blocks with a masked remainder (Sources/attention/attention.swift:25,
// 84-91, 192-199); the kernels of attention.hpp keep a wavefront's 32 queries x D output and its Q
// rows in registers, which stops at D = 256. Here a wavefront owns 16 queries and uses
// v_mfma_f32_16x16x32 (lane l: A[m = l % 16][k = 8 (l / 16) .. + 7],
// B[k = 8 (l / 16) .. + 7][n = l % 16], D[m = 4 (l / 16) .. + 3][n = l % 16]):
//   S = Q.K^T per tile of 32 keys (Q rows in registers as A operands, K rows read from LDS as B
//   operands), online softmax in base 2 (row maxima and sums across the 16 lanes that hold a
//   query's keys), P rounded to the input type through a per-wavefront LDS scratch into A-operand
//   layout, O += P.V with V read transposed from LDS (ds_read_b64_tr_b16), O / l at the end.
// One workgroup per 64 queries of one (batch, head), 4 wavefronts; K / V tiles of 32 rows of
// 1 KB, double buffered by direct-to-LDS loads (128 KB: one workgroup per CU). 16-byte chunk c of
// row r of a staged tile sits at chunk c ^ f(r), f(r) = 2 (r % 8) + (r / 8) % 2: conflict-free row
// reads of 16 rows and transposed reads of 4 rows x 2 chunks. Chunks past D are loaded as zeros
// and never stored; keys past S_kv and (causal) past the diagonal are masked.
#include "device.hpp"

namespace mtk {
namespace wide {

constexpr int kDP = 512;               // padded head dimension
constexpr int kRowB = kDP * 2;         // staged row: 1 KB
constexpr int kTileB = 32 * kRowB;     // 32 KB per staged tile of 32 rows
constexpr int kQueriesWG = 64;         // 4 wavefronts x 16 queries
constexpr int kSteps = kDP / 32;       // 32-dim MFMA steps of S
constexpr int kDBlocks = kDP / 16;     // 16-dim output blocks
constexpr int kScrRow = 80;            // scratch row stride in bytes: 32 elements + 16 (no conflicts)
constexpr int kScrB = 16 * kScrRow;

__device__ __forceinline__ int swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }
__device__ __forceinline__ uint32_t chunk_off(int r, int c) { return (uint32_t)(r * kRowB + ((c ^ swz(r)) << 4)); }

// Stage a 32-row tile: 32 direct-to-LDS instructions of 1 KB (one row each), eight per wavefront;
// lane l of instruction i writes row i, physical chunk l, which holds global chunk l ^ f(i). Rows at
// or past rows_valid and chunks at or past nchunk read zero.
__device__ __forceinline__ void stage_tile(rsrc_t r, char *tile, uint32_t base, uint32_t rs, int rows_valid,
                                           int nchunk, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 8 * wave + j;
    const int gc = lane ^ swz(row);
    lds_direct16(r, tile + row * kRowB, row < rows_valid && gc < nchunk ? base + (uint32_t)row * rs + 16u * gc : kOOB);
  }
}

__device__ __forceinline__ u32x4 rd128(uint32_t addr) {
  u32x4 w;
  asm volatile("ds_read_b128 %0, %1" : "=v"(w) : "v"(addr));
  return w;
}
__device__ __forceinline__ u32x4 rd_tr(uint32_t a0, uint32_t a1) {
  u32x2 w0, w1;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(w0) : "v"(a0));
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(w1) : "v"(a1));
  return u32x4{w0.x, w0.y, w1.x, w1.y};
}
__device__ __forceinline__ void wr16(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b16 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void wait_lds(u32x4 &f) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f)); }
// lgkmcnt(N): all but the N youngest LDS reads done (they complete in issue order), tied to the
// fragment about to be used
template <int N>
__device__ __forceinline__ void wait_lds_n(u32x4 &f) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(f) : "i"(N));
}
// reads issued after step k's in a pipeline of ns steps read r steps ahead, rps reads per step
constexpr int ring_younger(int k, int ns, int r, int rps) { return rps * (k + r < ns ? r : ns - 1 - k); }

// max / sum over the 16 lanes that share l / 16 (the keys of one query row)
__device__ __forceinline__ float row16_max(float x) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}
__device__ __forceinline__ float row16_sum(float x) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

template <int DT, bool CAUSAL>
__device__ __forceinline__ void fwd(const mtk_attn_kargs &a) {
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileB + 4 * kScrB];  // 2 slots x (K, V), scratch
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  int bh = id / a.q_blocks;
  int qblk = id - bh * a.q_blocks;
  if (CAUSAL) {
    int rank;
    causal_order(id, a.q_blocks, a.B * a.H, bh, rank);
    qblk = a.q_blocks - 1 - rank;  // heaviest (last) query blocks first
  }
  const int b = bh / a.H, h = bh - b * a.H;
  const int hk = h / (a.H / a.H_kv);
  const int q0 = qblk * kQueriesWG + 16 * wave;  // this wavefront's first query
  const int nchunk = a.D >> 3;
  const uint32_t rs = (uint32_t)a.H * a.D * 2, rkv = (uint32_t)a.H_kv * a.D * 2;
  const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * a.D * 2);
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H_kv + hk) * a.D * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const int diag = a.S_kv - a.S_q;
  const float c = a.scale_log2;

  // Q rows of query q0 + l % 16 as A operands: step s holds dims 32 s + 8 (l / 16) .. + 7
  const int qa = q0 + l16;
  u32x4 qf[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const uint32_t off = qa < a.S_q && 4 * s + g < nchunk ? qbase + (uint32_t)qa * rs + (uint32_t)(32 * s + 8 * g) * 2u : kOOB;
    qf[s] = buf_load16(rq, off);
  }
  // accumulator rows of this lane: queries q0 + 4 (l / 16) + e; running max (base 2) and this
  // lane's part of the row sums (its keys l % 16 and 16 + l % 16 of every tile). (The 128-query
  // kernel's lazy rescale, O rescaled only when the max moves by more than 8, spilled here: the
  // branch around the 128 accumulator registers' rescale took 200 bytes per lane of scratch.)
  f32x4 o[kDBlocks];
#pragma unroll
  for (int i = 0; i < kDBlocks; ++i) o[i] = f32x4{};
  float mrow[4], lsum[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    mrow[e] = -INFINITY;
    lsum[e] = 0.0f;
  }

  const int qwg = qblk * kQueriesWG;
  const int kv_end = CAUSAL ? min(a.S_kv, qwg + kQueriesWG + diag) : a.S_kv;
  const int n_tiles = kv_end > 0 ? (kv_end + 31) / 32 : 0;
  auto stage = [&](int slot, int t) {
    const uint32_t tb = kvbase + (uint32_t)(t * 32) * rkv;
    char *st = smem + slot * 2 * kTileB;
    stage_tile(rk, st, tb, rkv, a.S_kv - 32 * t, nchunk, wave, lane);
    stage_tile(rv, st + kTileB, tb, rkv, a.S_kv - 32 * t, nchunk, wave, lane);
  };
  const uint32_t scr = lds_addr(smem + 4 * kTileB + wave * kScrB);

  if (n_tiles > 0) stage(0, 0);
  for (int t = 0; t < n_tiles; ++t) {
    wait_vmem();
    __syncthreads();  // tile t is in LDS; every wavefront is done with the other slot
    if (t + 1 < n_tiles) stage((t + 1) & 1, t + 1);
    const char *kt = smem + (t & 1) * 2 * kTileB, *vt = kt + kTileB;

    // S = Q.K^T for the tile's two blocks of 16 keys: 2 kSteps steps (d-step outer, key block inner,
    // so the two accumulator chains alternate), K fragments read kR1 steps ahead through a ring
    f32x4 s[2] = {f32x4{}, f32x4{}};
    {
      constexpr int kNS = 2 * kSteps, kR1 = 8;
      u32x4 fr[kR1 + 1];
      auto rd = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if constexpr (k < kNS) fr[k % (kR1 + 1)] = rd128(lds_addr(kt) + chunk_off(16 * (k % 2) + l16, 4 * (k / 2) + g));
      };
      static_for<0, kR1>(rd);
      static_for<0, kNS>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        rd(std::integral_constant<int, k + kR1>{});
        wait_lds_n<ring_younger(k, kNS, kR1, 1)>(fr[k % (kR1 + 1)]);
        s[k % 2] = mfma16x16x32<DT>(qf[k / 2], fr[k % (kR1 + 1)], s[k % 2]);
      });
    }
    // V^T fragments of the P.V product (keys 8 (l / 16) .. + 7 of dim 16 db + l % 16), read kR2
    // steps ahead; the first kR2 go out before the softmax work
    constexpr int kR2 = 6;
    u32x4 fv[kR2 + 1];
    auto rdv = [&](auto kc) {
      constexpr int db = decltype(kc)::value;
      if constexpr (db < kDBlocks) {
        const int sl = lane & 15;
        uint32_t ad[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int row = 8 * g + 4 * hf + (sl >> 2);
          const int d = 16 * db + 4 * (sl & 3);
          ad[hf] = lds_addr(vt) + (uint32_t)(row * kRowB + (((d >> 3) ^ swz(row)) << 4) + 2 * (d & 7));
        }
        fv[db % (kR2 + 1)] = rd_tr(ad[0], ad[1]);
      }
    };
    static_for<0, kR2>(rdv);
    // online softmax in base 2: x = S scale log2(e), masked to -inf past S_kv or the diagonal
    float x[2][4], mt[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int qi = q0 + 4 * g + e;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int key = 32 * t + 16 * nb + l16;
        const bool ok = key < a.S_kv && (!CAUSAL || key <= qi + diag);
        x[nb][e] = ok ? s[nb][e] * c : -INFINITY;
      }
      mt[e] = row16_max(fmaxf(x[0][e], x[1][e]));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float mn = fmaxf(mrow[e], mt[e]);
      const float off = mn == -INFINITY ? 0.0f : mn;  // a row with no visible key yet keeps P = 0
      const float corr = __builtin_amdgcn_exp2f(mrow[e] - off);
      mrow[e] = mn;
      lsum[e] *= corr;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) o[db][e] *= corr;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const float p = __builtin_amdgcn_exp2f(x[nb][e] - off);
        lsum[e] += p;
        wr16(scr + (uint32_t)((4 * g + e) * kScrRow + (16 * nb + l16) * 2), to_bits<DT>(p));
      }
    }
    // P as the A operand: query l % 16, keys 8 (l / 16) .. + 7 (this wavefront's writes come first;
    // the wait also covers the V^T reads issued before them)
    u32x4 pa = rd128(scr + (uint32_t)(l16 * kScrRow + 16 * g));
    wait_lds(pa);
    // O += P.V, one MFMA per 16-dim block (two transposed reads per step)
    static_for<0, kDBlocks>([&](auto kc) {
      constexpr int db = decltype(kc)::value;
      rdv(std::integral_constant<int, db + kR2>{});
      wait_lds_n<ring_younger(db, kDBlocks, kR2, 2)>(fv[db % (kR2 + 1)]);
      o[db] = mfma16x16x32<DT>(pa, fv[db % (kR2 + 1)], o[db]);
    });
  }

  // O / l; lse = (m + log2 l) ln 2 (natural log), -inf for a row that sees no key (O = 0)
  float inv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float l = row16_sum(lsum[e]);
    inv[e] = l > 0.0f ? 1.0f / l : 0.0f;
    const int qi = q0 + 4 * g + e;
    if (a.lse != nullptr && l16 == 0 && qi < a.S_q)
      a.lse[((size_t)b * a.H + h) * a.S_q + qi] = l > 0.0f ? (mrow[e] + __builtin_amdgcn_logf(l)) * 0.6931471805599453f : -INFINITY;
  }
  wait_vmem();
  __syncthreads();  // the slots are free: park the output rows there, then store whole chunks
  char *park = smem + wave * (16 * kRowB);
#pragma unroll
  for (int db = 0; db < kDBlocks; ++db)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * g + e, d = 16 * db + l16;
      *(uint16_t *)(park + r * kRowB + (((d >> 3) ^ swz(r)) << 4) + 2 * (d & 7)) = to_bits<DT>(o[db][e] * inv[e]);
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's parking writes are done
  uint16_t *O = (uint16_t *)a.O;
  const size_t ld = (size_t)a.H * a.D;
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int r = it, cc = lane;  // row it, chunk lane (64 chunks of 16 bytes)
    const u32x4 v = *(const u32x4 *)(park + chunk_off(r, cc));
    const int qi = q0 + r;
    if (qi < a.S_q && cc < nchunk) *(u32x4 *)(O + ((size_t)b * a.S_q + qi) * ld + (size_t)h * a.D + 8 * cc) = v;
  }
}

}  // namespace wide
}  // namespace mtk

using namespace mtk;

#define FWD_WIDE(NAME, DT, CAUSAL)                                                  \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_attn_kargs a) { \
    wide::fwd<DT, CAUSAL>(a);                                                      \
  }

FWD_WIDE(mtk_attn_fwd_d512_f16, DT_F16, false)
FWD_WIDE(mtk_attn_fwd_d512_f16_causal, DT_F16, true)
FWD_WIDE(mtk_attn_fwd_d512_bf16, DT_BF16, false)
FWD_WIDE(mtk_attn_fwd_d512_bf16_causal, DT_BF16, true)
