// Flash-attention backward for head dimensions above 128 (multiples of 8 up to 256), gfx950,
// fp16/bf16 in and out, fp32 accumulate. The same gradients as attention_bwd.hip (the reference's
// CPU restatement: Sources/attention/Network.swift:205-281 dP row / D-term / dS row, 313-402
// dV = P^T dO, dK = dS^T Q, dQ = dS K), from the same row terms (its attn_bwd_pre kernel writes
// D * scale and the base-2 lse), with the causal mask and grouped K/V heads of the forward.
//
// At D = 256 the 32-key wavefronts of the D <= 128 kernels do not fit the register file (their K
// and V rows alone would take 128 registers, the dK / dV accumulators 256), so these kernels give a
// wavefront 16 keys (dK/dV) or 16 queries (dQ) and use v_mfma_f32_16x16x32:
//   lane l holds A[m = l % 16][k = 8 (l / 16) .. + 7], B[k = 8 (l / 16) .. + 7][n = l % 16] and
//   D[m = 4 (l / 16) .. + 3][n = l % 16].
// attn_bwd256_dkdv  one workgroup per 64 keys of one (batch, K/V head), 4 wavefronts x 16 keys;
//                   query tiles of 32 rows (every query head of the K/V head's group) stream
//                   through LDS, double buffered by direct-to-LDS loads. S^T = K.Q^T and
//                   dP^T = V.dO^T with the wavefront's K / V rows in registers (A operands) and
//                   Q / dO rows read from LDS (B operands); P^T and dS^T go through a small
//                   per-wavefront LDS scratch into A-operand layout; dV += P^T.dO and dK += dS^T.Q
//                   read dO / Q transposed (ds_read_b64_tr_b16).
// attn_bwd256_dq    one workgroup per 64 queries of one (batch, head), 4 wavefronts x 16 queries;
//                   key tiles of 32 rows of K and V stream through LDS; S = Q.K^T, dP = dO.V^T
//                   (Q, dO rows in registers), dS through the scratch, dQ += dS.K with K read
//                   transposed.
// Staged tiles are 32 rows of 512 bytes; 16-byte chunk c of row r sits at chunk c ^ f(r) with
// f(r) = 2 (r % 8) + (r / 8) % 2: the 16 rows of a row read hit 16 distinct 16-byte bank groups,
// and the 4 rows x 2 chunks of a transposed read 8 distinct ones. Chunks past D and rows past
// the sequence are loaded as zeros (exact zeros in every product); they are never stored.
#include "device.hpp"

namespace mtk {
namespace bwd256 {

constexpr int kRowB = 512;                // staged row: 256 elements
constexpr int kTileB = 32 * kRowB;        // 16 KB per staged tile of 32 rows
constexpr int kRowsWG = 64;               // keys (dK/dV) or queries (dQ) per workgroup
constexpr int kScrRow = 80;               // scratch row stride in bytes: 32 elements + 16 (no conflicts)
constexpr int kScrB = 16 * kScrRow;       // one 16 x 32 scratch matrix

__device__ __forceinline__ int swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

// Byte offset of 16-byte chunk c of row r in a staged tile.
__device__ __forceinline__ uint32_t chunk_off(int r, int c) { return (uint32_t)(r * kRowB + ((c ^ swz(r)) << 4)); }

// Stage a 32-row tile: 16 direct-to-LDS instructions of 1 KB (two rows each), four per wavefront.
// Lane l of instruction i writes row 2 i + l / 32, physical chunk l % 32, which holds global chunk
// (l % 32) ^ f(row). Rows at or past rows_valid and chunks at or past nchunk read zero.
__device__ __forceinline__ void stage_tile(rsrc_t r, char *tile, uint32_t base, uint32_t rs, int rows_valid,
                                           int nchunk, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = 4 * wave + j;
    const int row = 2 * i + (lane >> 5);
    const int gc = (lane & 31) ^ swz(row);
    lds_direct16(r, tile + i * 1024, row < rows_valid && gc < nchunk ? base + (uint32_t)row * rs + 16u * gc : kOOB);
  }
}

// B operand of a row-major product: rows (queries or keys) n0 .. n0 + 15 of the tile as columns,
// 32 dims of d-step s: lane l reads row n0 + l % 16, chunk 4 s + l / 16.
__device__ __forceinline__ uint32_t row_frag_addr(const char *tile, int n0, int s, int lane) {
  return lds_addr(tile) + chunk_off(n0 + (lane & 15), 4 * s + (lane >> 4));
}

// B operand of a transposed product: rows 8 (l / 16) .. + 7 of the tile (the K dimension: queries
// or keys) at column 16 db + l % 16. Two ds_read_b64_tr_b16: in each 16-lane group lane s
// addresses row k0 + s / 4 (k0 = 8 (l / 16), then + 4), columns 16 db + 4 (s % 4) .. + 3, and
// receives column 16 db + s at rows k0 .. k0 + 3.
__device__ __forceinline__ uint32_t tr_addr(const char *tile, int db, int half, int lane) {
  const int s = lane & 15;
  const int row = 8 * (lane >> 4) + 4 * half + (s >> 2);
  const int d = 16 * db + 4 * (s & 3);
  return lds_addr(tile) + (uint32_t)(row * kRowB + (((d >> 3) ^ swz(row)) << 4) + 2 * (d & 7));
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
// 16-bit scratch write (inline asm, like the reads: the compiler would otherwise order it behind
// the direct-to-LDS loads in flight)
__device__ __forceinline__ void wr16(uint32_t addr, uint32_t v) {
  asm volatile("ds_write_b16 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void wait_lds(u32x4 &f) { asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f)); }
__device__ __forceinline__ void wait_lds2(u32x4 &f0, u32x4 &f1) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f0), "+v"(f1));
}
// lgkmcnt(N): all but the N youngest LDS reads done (they complete in issue order), tied to the
// pair of fragments about to be used
template <int N>
__device__ __forceinline__ void wait_lds2_n(u32x4 &f0, u32x4 &f1) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(f0), "+v"(f1) : "i"(N));
}
template <int N>
__device__ __forceinline__ void wait_lds_n(u32x4 &f) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(f) : "i"(N));
}
// Fragment reads ahead of their MFMAs: a step pipeline of NS steps whose fragments are read R
// steps ahead into a ring of R + 1 register sets (each step's reads are RPS LDS instructions).
constexpr int ring_younger(int k, int ns, int r, int rps) { return rps * (k + r < ns ? r : ns - 1 - k); }

// Park a wavefront's 16 x 256 accumulator tile (lane: rows 4 (l / 16) + e, column 16 db + l % 16)
// in LDS as 512-byte rows and store chunks below nchunk of rows below rows_valid, 16 bytes per
// lane: dst + row * ld elements.
template <int DT>
__device__ __forceinline__ void store_tile(char *park, const f32x4 (&acc)[16], uint16_t *dst, size_t ld, int rows_valid,
                                           int nchunk, int lane) {
  const int l16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int db = 0; db < 16; ++db)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * g + e, d = 16 * db + l16;
      *(uint16_t *)(park + r * kRowB + (((d >> 3) ^ swz(r)) << 4) + 2 * (d & 7)) = to_bits<DT>(acc[db][e]);
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's parking writes are done
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = 2 * it + (lane >> 5), c = lane & 31;
    const u32x4 v = *(const u32x4 *)(park + chunk_off(r, c));
    if (r < rows_valid && c < nchunk) *(u32x4 *)(dst + (size_t)r * ld + 8 * c) = v;
  }
}

template <int DT, bool CAUSAL>
__device__ __forceinline__ void dkdv(const mtk_attn_bwd_kargs &a) {
  // two slots of (Q tile, dO tile), then the wavefronts' P^T / dS^T scratch
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileB + 4 * 2 * kScrB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  int bh = id / a.k_blocks;
  int kb = id - bh * a.k_blocks;
  if (CAUSAL) causal_order(id, a.k_blocks, a.B * a.H_kv, bh, kb);  // heaviest (first) key blocks first
  const int b = bh / a.H_kv, hk = bh - b * a.H_kv;
  const int group = a.H / a.H_kv;
  const int k0 = kb * kRowsWG + 16 * wave;  // this wavefront's first key
  const int nchunk = a.D >> 3;
  const uint32_t rs = (uint32_t)a.H * a.D * 2, rkv = (uint32_t)a.H_kv * a.D * 2;
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H_kv + hk) * a.D * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rg = make_rsrc(a.dO, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const uint32_t row_bytes = (uint32_t)a.B * a.H * a.S_q * 4u;
  const rsrc_t rl = make_rsrc(a.Lt, row_bytes);
  const rsrc_t rd = make_rsrc(a.Dt, row_bytes);
  const int diag = a.S_kv - a.S_q;
  const float c = a.scale_log2;

  // K and V rows of key k0 + l % 16 as A operands: d-step s holds dims 32 s + 8 (l / 16) .. + 7
  const int key_a = k0 + l16;
  u32x4 kf[8], vf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint32_t off = key_a < a.S_kv && 4 * s + g < nchunk ? kvbase + (uint32_t)key_a * rkv + (uint32_t)(32 * s + 8 * g) * 2u : kOOB;
    kf[s] = buf_load16(rk, off);
    vf[s] = buf_load16(rv, off);
  }
  f32x4 dk[16], dv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    dk[i] = f32x4{};
    dv[i] = f32x4{};
  }

  // query tiles of 32 that see one of this workgroup's keys, for every query head of the group
  const int kwg = kb * kRowsWG;
  const int t0 = CAUSAL ? max(0, kwg - diag) / 32 : 0;
  const int n_tiles = (a.S_q + 31) / 32;
  const int per_head = max(0, n_tiles - t0);
  const int n_steps = group * per_head;
  auto stage = [&](int slot, int i) {
    const int h = hk * group + i / per_head, t = t0 + i % per_head;
    const uint32_t tb = (uint32_t)(((size_t)b * a.S_q * a.H + h) * a.D * 2) + (uint32_t)(t * 32) * rs;
    char *st = smem + slot * 2 * kTileB;
    stage_tile(rq, st, tb, rs, a.S_q - 32 * t, nchunk, wave, lane);
    stage_tile(rg, st + kTileB, tb, rs, a.S_q - 32 * t, nchunk, wave, lane);
  };
  const uint32_t scr_p = lds_addr(smem + 4 * kTileB + wave * 2 * kScrB), scr_s = scr_p + kScrB;

  if (n_steps > 0) stage(0, 0);
  for (int i = 0; i < n_steps; ++i) {
    const int h = hk * group + i / per_head, t = t0 + i % per_head;
    const int qt0 = 32 * t;
    // this lane's row terms: queries qt0 + 16 nb + l % 16 (loaded before the next tile's staging)
    const uint32_t rb = (uint32_t)(((size_t)b * a.H + h) * a.S_q) * 4u;
    float lse2[2], dd[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int qi = qt0 + 16 * nb + l16;
      const uint32_t off = qi < a.S_q ? rb + (uint32_t)qi * 4u : kOOB;
      lse2[nb] = __builtin_bit_cast(float, buf_load4(rl, off));
      dd[nb] = __builtin_bit_cast(float, buf_load4(rd, off));
    }
    wait_vmem();
    __syncthreads();  // tile i is in LDS; every wavefront is done with the other slot
    if (i + 1 < n_steps) stage((i + 1) & 1, i + 1);
    const char *qt = smem + (i & 1) * 2 * kTileB, *gt = qt + kTileB;

    // S^T = K.Q^T and dP^T = V.dO^T for the tile's two blocks of 16 queries: 16 steps (d-step st,
    // query block nb inner, so four accumulator chains alternate), fragments read kR1 steps ahead
    f32x4 s[2] = {f32x4{}, f32x4{}}, p[2] = {f32x4{}, f32x4{}};
    {
      constexpr int kNS = 16, kR1 = 4;
      u32x4 fr[kR1 + 1][2];
      auto rd = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if constexpr (k < kNS) {
          fr[k % (kR1 + 1)][0] = rd128(row_frag_addr(qt, 16 * (k % 2), k / 2, lane));
          fr[k % (kR1 + 1)][1] = rd128(row_frag_addr(gt, 16 * (k % 2), k / 2, lane));
        }
      };
      static_for<0, kR1>(rd);
      static_for<0, kNS>([&](auto kc) {
        constexpr int k = decltype(kc)::value, st = k / 2, nb = k % 2;
        rd(std::integral_constant<int, k + kR1>{});
        wait_lds2_n<ring_younger(k, kNS, kR1, 2)>(fr[k % (kR1 + 1)][0], fr[k % (kR1 + 1)][1]);
        s[nb] = mfma16x16x32<DT>(kf[st], fr[k % (kR1 + 1)][0], s[nb]);
        p[nb] = mfma16x16x32<DT>(vf[st], fr[k % (kR1 + 1)][1], p[nb]);
      });
    }
    // dV / dK fragments: the first kR2 steps' transposed reads go out before the softmax work
    constexpr int kNS2 = 16, kR2 = 3;
    u32x4 fr2[kR2 + 1][2];
    auto rd2 = [&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if constexpr (k < kNS2) {
        fr2[k % (kR2 + 1)][0] = rd_tr(tr_addr(gt, k, 0, lane), tr_addr(gt, k, 1, lane));
        fr2[k % (kR2 + 1)][1] = rd_tr(tr_addr(qt, k, 0, lane), tr_addr(qt, k, 1, lane));
      }
    };
    static_for<0, kR2>(rd2);
    // P^T = exp2(S^T scale log2e - lse2) and dS^T = P^T (dP^T scale - D scale), masked, rounded to
    // the input type into the scratch ([16 keys][32 queries])
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int qi = qt0 + 16 * nb + l16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = k0 + 4 * g + e;
        const bool ok = key < a.S_kv && qi < a.S_q && (!CAUSAL || key <= qi + diag);
        const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[nb][e], c, -lse2[nb]));
        const float pv = ok ? pe : 0.0f;
        const float sv = ok ? pe * __builtin_fmaf(p[nb][e], a.scale, -dd[nb]) : 0.0f;
        const uint32_t o = (uint32_t)((4 * g + e) * kScrRow + (16 * nb + l16) * 2);
        wr16(scr_p + o, to_bits<DT>(pv));
        wr16(scr_s + o, to_bits<DT>(sv));
      }
    }
    // A operands: key l % 16, queries 8 (l / 16) .. + 7 (the same wavefront's writes above come first;
    // the wait also covers the transposed reads issued before them)
    u32x4 pa = rd128(scr_p + (uint32_t)(l16 * kScrRow + 16 * g));
    u32x4 sa = rd128(scr_s + (uint32_t)(l16 * kScrRow + 16 * g));
    wait_lds2(pa, sa);
    // dV += P^T.dO and dK += dS^T.Q, 16 blocks of 16 dims each, fragments kR2 steps ahead (four
    // transposed reads per step)
    static_for<0, kNS2>([&](auto kc) {
      constexpr int db = decltype(kc)::value;
      rd2(std::integral_constant<int, db + kR2>{});
      wait_lds2_n<ring_younger(db, kNS2, kR2, 4)>(fr2[db % (kR2 + 1)][0], fr2[db % (kR2 + 1)][1]);
      dv[db] = mfma16x16x32<DT>(pa, fr2[db % (kR2 + 1)][0], dv[db]);
      dk[db] = mfma16x16x32<DT>(sa, fr2[db % (kR2 + 1)][1], dk[db]);
    });
  }

  wait_vmem();
  __syncthreads();  // every wavefront is done with the tiles; the slots hold the output rows now
  char *park = smem + wave * 2 * (16 * kRowB);
  const size_t ld = (size_t)a.H_kv * a.D;
  const size_t e0 = ((size_t)b * a.S_kv + k0) * ld + (size_t)hk * a.D;
  store_tile<DT>(park, dk, (uint16_t *)a.dK + e0, ld, a.S_kv - k0, nchunk, lane);
  store_tile<DT>(park + 16 * kRowB, dv, (uint16_t *)a.dV + e0, ld, a.S_kv - k0, nchunk, lane);
}

// Read-ahead depths of dQ's two step pipelines: the deepest that keep two wavefronts per SIMD
// (deeper rings measured slower at one: 2,663 against 2,085 us at the config 5 shape, D = 256;
// the causal kernel's masks take the registers of one more step)
template <int DT, bool CAUSAL, int kDqAhead1 = CAUSAL ? 1 : 2, int kDqAhead2 = 2>
__device__ __forceinline__ void dq(const mtk_attn_bwd_kargs &a) {
  // two slots of (K tile, V tile), then the wavefronts' dS scratch
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileB + 4 * kScrB];
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
  const int q0 = qblk * kRowsWG + 16 * wave;  // this wavefront's first query
  const int nchunk = a.D >> 3;
  const uint32_t rs = (uint32_t)a.H * a.D * 2, rkv = (uint32_t)a.H_kv * a.D * 2;
  const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * a.D * 2);
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H_kv + hk) * a.D * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rg = make_rsrc(a.dO, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const uint32_t row_bytes = (uint32_t)a.B * a.H * a.S_q * 4u;
  const rsrc_t rl = make_rsrc(a.Lt, row_bytes);
  const rsrc_t rd = make_rsrc(a.Dt, row_bytes);
  const int diag = a.S_kv - a.S_q;
  const float c = a.scale_log2;

  // Q and dO rows of query q0 + l % 16 as A operands
  const int qa = q0 + l16;
  u32x4 qf[8], gf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint32_t off = qa < a.S_q && 4 * s + g < nchunk ? qbase + (uint32_t)qa * rs + (uint32_t)(32 * s + 8 * g) * 2u : kOOB;
    qf[s] = buf_load16(rq, off);
    gf[s] = buf_load16(rg, off);
  }
  // row terms of the accumulator rows this lane holds: queries q0 + 4 (l / 16) + e
  float lse2[4], dd[4];
  const uint32_t rb = (uint32_t)(((size_t)b * a.H + h) * a.S_q) * 4u;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int qi = q0 + 4 * g + e;
    const uint32_t off = qi < a.S_q ? rb + (uint32_t)qi * 4u : kOOB;
    lse2[e] = __builtin_bit_cast(float, buf_load4(rl, off));
    dd[e] = __builtin_bit_cast(float, buf_load4(rd, off));
  }
  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4{};

  const int qwg = qblk * kRowsWG;
  const int kv_end = CAUSAL ? min(a.S_kv, qwg + kRowsWG + diag) : a.S_kv;
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

    // S = Q.K^T and dP = dO.V^T for the tile's two blocks of 16 keys (the same step pipeline as the
    // dK/dV kernel's)
    f32x4 s[2] = {f32x4{}, f32x4{}}, p[2] = {f32x4{}, f32x4{}};
    {
      constexpr int kNS = 16, kR1 = kDqAhead1;
      u32x4 fr[kR1 + 1][2];
      auto rd = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if constexpr (k < kNS) {
          fr[k % (kR1 + 1)][0] = rd128(row_frag_addr(kt, 16 * (k % 2), k / 2, lane));
          fr[k % (kR1 + 1)][1] = rd128(row_frag_addr(vt, 16 * (k % 2), k / 2, lane));
        }
      };
      static_for<0, kR1>(rd);
      static_for<0, kNS>([&](auto kc) {
        constexpr int k = decltype(kc)::value, st = k / 2, nb = k % 2;
        rd(std::integral_constant<int, k + kR1>{});
        wait_lds2_n<ring_younger(k, kNS, kR1, 2)>(fr[k % (kR1 + 1)][0], fr[k % (kR1 + 1)][1]);
        s[nb] = mfma16x16x32<DT>(qf[st], fr[k % (kR1 + 1)][0], s[nb]);
        p[nb] = mfma16x16x32<DT>(gf[st], fr[k % (kR1 + 1)][1], p[nb]);
      });
    }
    // dQ fragments: the first kR2 steps' transposed reads go out before the softmax work
    constexpr int kNS2 = 16, kR2 = kDqAhead2;
    u32x4 fr2[kR2 + 1];
    auto rd2 = [&](auto kc) {
      constexpr int k = decltype(kc)::value;
      if constexpr (k < kNS2) fr2[k % (kR2 + 1)] = rd_tr(tr_addr(kt, k, 0, lane), tr_addr(kt, k, 1, lane));
    };
    static_for<0, kR2>(rd2);
    // dS = P (dP scale - D scale), P = exp2(S scale log2e - lse2), masked, into the scratch
    // ([16 queries][32 keys])
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int key = 32 * t + 16 * nb + l16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int qi = q0 + 4 * g + e;
        const bool ok = key < a.S_kv && qi < a.S_q && (!CAUSAL || key <= qi + diag);
        const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[nb][e], c, -lse2[e]));
        const float sv = ok ? pe * __builtin_fmaf(p[nb][e], a.scale, -dd[e]) : 0.0f;
        wr16(scr + (uint32_t)((4 * g + e) * kScrRow + (16 * nb + l16) * 2), to_bits<DT>(sv));
      }
    }
    u32x4 sa = rd128(scr + (uint32_t)(l16 * kScrRow + 16 * g));
    wait_lds(sa);
    // dQ += dS.K, 16 blocks of 16 dims, fragments kR2 steps ahead (two transposed reads per step)
    static_for<0, kNS2>([&](auto kc) {
      constexpr int db = decltype(kc)::value;
      rd2(std::integral_constant<int, db + kR2>{});
      wait_lds_n<ring_younger(db, kNS2, kR2, 2)>(fr2[db % (kR2 + 1)]);
      acc[db] = mfma16x16x32<DT>(sa, fr2[db % (kR2 + 1)], acc[db]);
    });
  }

  wait_vmem();
  __syncthreads();
  char *park = smem + wave * (16 * kRowB);
  const size_t ld = (size_t)a.H * a.D;
  store_tile<DT>(park, acc, (uint16_t *)a.dQ + ((size_t)b * a.S_q + q0) * ld + (size_t)h * a.D, ld, a.S_q - q0,
                 nchunk, lane);
}

}  // namespace bwd256
}  // namespace mtk

using namespace mtk;

#define BWD256_DKDV(NAME, DT, CAUSAL)                                                 \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_attn_bwd_kargs a) { \
    bwd256::dkdv<DT, CAUSAL>(a);                                                       \
  }
#define BWD256_DQ(NAME, DT, CAUSAL)                                                   \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_attn_bwd_kargs a) { \
    bwd256::dq<DT, CAUSAL>(a);                                                         \
  }

BWD256_DKDV(mtk_attn_bwd256_dkdv_f16, DT_F16, false)
BWD256_DKDV(mtk_attn_bwd256_dkdv_f16_causal, DT_F16, true)
BWD256_DKDV(mtk_attn_bwd256_dkdv_bf16, DT_BF16, false)
BWD256_DKDV(mtk_attn_bwd256_dkdv_bf16_causal, DT_BF16, true)
BWD256_DQ(mtk_attn_bwd256_dq_f16, DT_F16, false)
BWD256_DQ(mtk_attn_bwd256_dq_f16_causal, DT_F16, true)
BWD256_DQ(mtk_attn_bwd256_dq_bf16, DT_BF16, false)
BWD256_DQ(mtk_attn_bwd256_dq_bf16_causal, DT_BF16, true)
