// Flash-attention backward for gfx950 (head dimensions that are multiples of 8 up to 128: the
// kernels are templated on a padded head dimension DP of 64 or 128, chunks of 8 elements past D are
// loaded as zeros, contribute exact zeros to every product, and are not stored), fp16/bf16 in and
// out, fp32 accumulate.
//
// The reference has no GPU backward; its CPU restatement of the gradients of the loss
// Phi = sum dO * O is Sources/attention/Network.swift:205-281 (dP row, D-term, dS row) and
// 313-402 (dV = P^T dO, dK = dS^T Q, dQ = dS K). These kernels compute the same quantities for
// tensors laid out [B][S][H][D] (the forward's layout), with the causal mask of the forward:
//   P  = exp(Q K^T * scale - lse)          (lse: the forward's row log-sum-exp, natural log)
//   D  = rowsum(dO * O)                     (O: the forward's output)
//   dS = P * (dO V^T - D) * scale
//   dV = P^T dO,  dK = dS^T Q,  dQ = dS K
// Three kernels, no atomics (every output element is written once, sums in a fixed order):
//   attn_bwd_pre   D for every query row.
//   attn_bwd_dkdv  one workgroup per 128 keys of one (batch, K/V head), 4 wavefronts x 32 keys; the
//                  query rows of every query head sharing that K/V head stream through LDS in tiles
//                  of 64 (grouped-query attention: H query heads over H_kv K/V heads, query head h
//                  reads K/V head h / (H / H_kv); dK and dV sum over the group). S = Q.K^T is
//                  computed with the key as the accumulator column, Q rows fed in the order
//                  swap_bits_2_3(m) so that accumulator registers 0-7 / 8-15 hold 8 consecutive
//                  queries: P and dS leave the
//                  accumulators as the B operands of dV^T += dO^T.P and dK^T += Q^T.dS, whose
//                  A operands are transposed LDS reads (ds_read_b64_tr_b16) of the dO / Q tiles.
//                  Software-pipelined: the S / dP MFMAs of tile i + 1 run interleaved with the
//                  softmax work of tile i (one or two elements per MFMA), then the dV / dK MFMAs
//                  of tile i.
//   attn_bwd_dq    one workgroup per 256 queries, 8 wavefronts x 32 queries (the forward's shape):
//                  S^T = K.Q^T and dP^T = V.dO^T with the query as the accumulator column, then
//                  dQ^T += K^T.dS^T with K^T read transposed from LDS.
// Each LDS operand tile is 64 rows of 2 DP bytes with the forward's swizzles for that width
// (AttnLayout): at DP = 128 tiles read as rows use the chunk swizzle chunk ^ (row & 15), tiles read
// transposed chunk ^ 4 * (row & 3); at DP = 64 (two rows per 256-byte bank line) chunk ^ ((row >> 1)
// & 7) and chunk ^ 4 * ((row >> 1) & 1) (all conflict-free); an operand read both ways is staged
// twice.
#include "attention.hpp"  // AttnLayout: the LDS row layouts and swizzles shared with the forward

namespace mtk {

constexpr int kBwdKeys = 128;            // keys per dK/dV workgroup
constexpr int kBwdQTile = 64;            // queries per LDS tile of the dK/dV kernel
constexpr int kBwdQRows = 256;           // queries per dQ workgroup
constexpr int kBwdKTile = 64;            // keys per LDS tile of the dQ kernel

__device__ __forceinline__ int bwd_swap_bits_2_3(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// Row-read tile (rows of DP elements): byte offset of 16-byte chunk `chunk` of row `row`.
template <int DP>
__device__ __forceinline__ uint32_t row_off(int row, int chunk) {
  using L = AttnLayout<DP>;
  return (uint32_t)(row * L::kRowB + ((chunk ^ L::kswz(row)) << 4));
}

// Transposed-read fragment base for d block db: lane (h = lane / 16, s = lane % 16) reads rows
// 8 (h / 2) + s / 4 (+ 4 e, + 16 js) at d = 32 db + 16 (h & 1) + 4 (s & 3); the result is the A
// operand [32 d][16 rows] of a 32x32x16 MFMA: lane gets d = 32 db + lane % 32 at rows
// 16 js + 8 (lane / 32) + 0..7.
// (The swizzle of the base row holds for the rows 4 and 16 js further on.)
template <int DP>
__device__ __forceinline__ uint32_t tr_base(const char *tile, int db, int lane) {
  using L = AttnLayout<DP>;
  const int s = lane & 15, h = lane >> 4;
  const int d = 32 * db + 16 * (h & 1) + 4 * (s & 3);
  const int row = 8 * (h >> 1) + (s >> 2);
  return lds_addr(tile) + (uint32_t)(row * L::kRowB + 16 * ((d >> 3) ^ L::vswz(row)) + 2 * (d & 7));
}

// Transposed fragment for row step js (16 rows) from a base made by tr_base (+ a tile offset).
template <int DP, int JS>
__device__ __forceinline__ u32x4 tr_frag(uint32_t base) {
  constexpr int R = AttnLayout<DP>::kRowB;
  const u32x2 w0 = ds_read_tr16_at<16 * R * JS>(base);
  const u32x2 w1 = ds_read_tr16_at<16 * R * JS + 4 * R>(base);
  return u32x4{w0.x, w0.y, w1.x, w1.y};
}

// Operand fragments read ahead of their MFMAs, in MFMA steps: dK/dV S / dP products and dV / dK
// products, dQ S^T / dP^T products and dQ products (the measured best of each).
constexpr int kBwdSdpAhead = 8;
constexpr int kBwdTrAhead = 8;
constexpr int kDqSdpAhead = 4;
constexpr int kDqTrAhead = 4;
// The dQ kernel's MFMA sections run at raised wave issue priority (of the two wavefronts of a SIMD,
// the one in an MFMA section issues first): causal 3 % faster, non-causal unchanged.
// Wait until at most N LDS operations are outstanding; f (filled by an inline-asm read) is handed
// on through the wait, so its consumers cannot be scheduled above it.
template <int N>
__device__ __forceinline__ void lgkm_wait_n(u32x4 &f) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(f) : "n"(N));
}

// Stage rows [row0, row0 + R n) of a 64-row operand tile (R = 1024 / row bytes: 4 rows of 256
// bytes, or 8 of 128): instruction i fills R rows (1 KB), lane l writes row row0 + R i + l / C,
// LDS chunk l % C (C chunks per row), which holds global chunk (l % C) ^ swizzle(row). Rows at or
// past `rows_valid` and chunks at or past `nchunk` (head dimensions below DP: 8 elements per
// chunk) read zero.
template <int DP, int N, bool TR>
__device__ __forceinline__ void stage_rows(rsrc_t r, char *tile, int row0, uint32_t base, uint32_t rs, int rows_valid,
                                           int nchunk, int lane) {
  using L = AttnLayout<DP>;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int row = row0 + L::kRpi * i + (int)((unsigned)lane / L::kCpr);
    const int pc = (int)((unsigned)lane % L::kCpr);
    const int gc = TR ? (pc ^ L::vswz(row)) : (pc ^ L::kswz(row));
    lds_direct16(r, tile + (row0 + L::kRpi * i) * L::kRowB,
                 row < rows_valid && gc < nchunk ? base + (uint32_t)row * rs + 16u * gc : kOOB);
  }
}

// ------------------------------------------------------------------------------------- D-term

template <int DT>
__device__ __forceinline__ void attn_bwd_pre(const mtk_attn_bwd_kargs &a) {
  // 16 lanes per (b, q, h) row of D <= 256 elements: lane j takes elements 8 j .. 8 j + 7 of O and
  // dO, then (D > 128) 8 (j + 16) .. + 7 (zero past D)
  const long long row = (long long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const long long rows = (long long)a.B * a.S_q * a.H;
  if (row >= rows) return;
  const int j = threadIdx.x & 15;
  const rsrc_t ro = make_rsrc(a.O, a.q_bytes);
  const rsrc_t rg = make_rsrc(a.dO, a.q_bytes);
  float s = 0.0f;
  for (int cj = j; cj < 32 && 8 * (cj - j) < a.D; cj += 16) {
    const uint32_t off = 8 * cj < a.D ? (uint32_t)(row * a.D + 8 * cj) * 2u : kOOB;
    const u32x4 o = buf_load16(ro, off), g = buf_load16(rg, off);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s = __builtin_fmaf(from_bits<DT>(o[e] & 0xffffu), from_bits<DT>(g[e] & 0xffffu), s);
      s = __builtin_fmaf(from_bits<DT>(o[e] >> 16), from_bits<DT>(g[e] >> 16), s);
    }
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) s += __shfl_xor(s, m, 16);
  if (j == 0) {
    const int h = (int)(row % a.H);
    const long long bq = row / a.H;
    const int q = (int)(bq % a.S_q), b = (int)(bq / a.S_q);
    const size_t i = ((size_t)b * a.H + h) * a.S_q + q;
    // the row terms of the other two kernels, scaled once per row: D * scale (dS = P (dP - D) scale
    // = P (dP scale - D scale)) and the base-2 log-sum-exp (P = exp2(S scale log2e - lse log2e))
    a.Dt[i] = s * a.scale;
    a.Lt[i] = a.lse[i] * 1.4426950408889634f;
  }
}

// ------------------------------------------------------------------------------------- dK, dV

template <int DT, bool CAUSAL, int DP>
__device__ __forceinline__ void attn_bwd_dkdv(const mtk_attn_bwd_kargs &a) {
  using L = AttnLayout<DP>;
  constexpr int kRowTile = L::kTile, kRowB = L::kRowB, kKs = L::kKs, kDb = L::kDb;
  // LDS: two slots of (Q rows, dO rows) read by S = Q.K^T and dP = dO.V^T, two slots of (Q, dO
  // transposed-read copies) read by dV and dK, two slots of a tile's 64 lse and 64 D values. Step
  // i's row tiles are read one step before its transposed tiles: the S / dP MFMAs of step i + 1 run
  // beside the softmax work of step i, then the dV / dK MFMAs of step i.
  constexpr int kPair = 2 * kRowTile;
  constexpr int kRowsOff = 0, kTrOff = 2 * kPair, kRtOff = 4 * kPair;
  __shared__ __attribute__((aligned(1024))) char smem[4 * kPair + 2 * 2048];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..3
  const int g = lane >> 5, col = lane & 31;

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  int bh = id / a.k_blocks;  // (batch, K/V head)
  int kb = id - bh * a.k_blocks;
  if (CAUSAL) causal_order(id, a.k_blocks, a.B * a.H_kv, bh, kb);  // heaviest (first) key blocks first
  const int b = bh / a.H_kv, hk = bh - b * a.H_kv;
  const int group = a.H / a.H_kv;  // query heads hk * group .. hk * group + group - 1
  const int k0 = kb * kBwdKeys;
  // rows of D elements (a multiple of 8, at most DP): chunks at or past nchunk are zeros
  const int nchunk = a.D >> 3;
  const uint32_t rs = (uint32_t)a.H * a.D * 2, rkv = (uint32_t)a.H_kv * a.D * 2;
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H_kv + hk) * a.D * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rg = make_rsrc(a.dO, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const uint32_t row_bytes = (uint32_t)a.B * a.H * a.S_q * 4u;  // row terms: [B][H][S_q] fp32
  const rsrc_t rl = make_rsrc(a.Lt, row_bytes);
  const rsrc_t rd = make_rsrc(a.Dt, row_bytes);
  const int diag = a.S_kv - a.S_q;  // key j is visible to query i iff j <= i + diag (causal)
  const float c = a.scale_log2;

  // this lane's key (accumulator column) and its K / V rows as B operands (steps of 16 dims)
  const int key = k0 + wave * 32 + col;
  const bool key_ok = key < a.S_kv;
  u32x4 kf[kKs], vf[kKs];
#pragma unroll
  for (int ds = 0; ds < kKs; ++ds) {
    const uint32_t off = key_ok && 2 * ds + g < nchunk ? kvbase + (uint32_t)key * rkv + (uint32_t)(16 * ds + 8 * g) * 2u : kOOB;
    kf[ds] = buf_load16(rk, off);
    vf[ds] = buf_load16(rv, off);
  }

  // query tiles that see at least one of this workgroup's keys: t0 .. n_tiles - 1 of each query
  // head of the group, visited head by head (step i: head hk * group + i / per_head, tile
  // t0 + i % per_head)
  int t0 = 0;
  if (CAUSAL) t0 = max(0, k0 - diag) / kBwdQTile;
  const int n_tiles = (a.S_q + kBwdQTile - 1) / kBwdQTile;
  const int per_head = max(0, n_tiles - t0);
  const int n_steps = group * per_head;

  // Staging of step i (clamped to the last step: past the end a slot is refilled, never read
  // for a result) into the slots given.
  auto tile_of = [&](int i, int &valid, uint32_t &tb, uint32_t &row_base, int &t) {
    const int h = hk * group + i / per_head;
    t = t0 + i % per_head;
    valid = a.S_q - t * kBwdQTile;
    const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * a.D * 2);
    row_base = (uint32_t)(((size_t)b * a.H + h) * a.S_q) * 4u;
    tb = qbase + (uint32_t)(t * kBwdQTile) * rs;
  };
  auto stage_rows_to = [&](int slot, int i) {
    char *st = smem + kRowsOff + slot * kPair;
    int valid, t;
    uint32_t tb, row_base;
    tile_of(i, valid, tb, row_base, t);
    stage_rows<DP, 16 / L::kRpi, false>(rq, st, 16 * wave, tb, rs, valid, nchunk, lane);
    stage_rows<DP, 16 / L::kRpi, false>(rg, st + kRowTile, 16 * wave, tb, rs, valid, nchunk, lane);
  };
  auto stage_tr_to = [&](int slot, int i) {
    char *st = smem + kTrOff + slot * kPair;
    int valid, t;
    uint32_t tb, row_base;
    tile_of(i, valid, tb, row_base, t);
    stage_rows<DP, 16 / L::kRpi, true>(rq, st, 16 * wave, tb, rs, valid, nchunk, lane);
    stage_rows<DP, 16 / L::kRpi, true>(rg, st + kRowTile, 16 * wave, tb, rs, valid, nchunk, lane);
    // lse (wave 0) and D (wave 1) of the tile's queries: lanes 0-15 load 4 values each (entries past
    // S_q are never used unmasked); lanes 16-63 write zeros
    if (wave < 2) {
      const uint32_t off = lane < 16 ? row_base + (uint32_t)(t * kBwdQTile + 4 * lane) * 4u : kOOB;
      lds_direct16(wave == 0 ? rl : rd, smem + kRtOff + slot * 2048 + wave * 1024, off);
    }
  };

  // A-operand rows of S = Q.K^T / dP = dO.V^T: MFMA row m reads query swap_bits_2_3(m) of the block
  const int arow = bwd_swap_bits_2_3(col);
  f32x16 dk[kDb], dv[kDb];
#pragma unroll
  for (int i = 0; i < kDb; ++i) {
    dk[i] = f32x16{};
    dv[i] = f32x16{};
  }

  // S and dP of the step whose rows are in rows slot `slot`, for the two 32-query blocks of the
  // tile: 4 kKs MFMAs in four interleaved accumulation chains (step k: d step k / 4; S of block 0,
  // dP of block 0, S of block 1, dP of block 1), each operand fragment read kBwdSdpAhead steps
  // ahead of its MFMA; after MFMA k, vstep runs 32 / (4 kKs) of the 32 elements of the previous
  // step's softmax. The fence per step keeps that order; every chain still accumulates its d steps
  // in order.
  constexpr int kSdpSteps = 4 * kKs, kElPerStep = 32 / kSdpSteps;
  auto sdp = [&](int slot, f32x16 (&s_)[2], f32x16 (&p_)[2], auto &&vstep) {
    const char *qrow = smem + kRowsOff + slot * kPair, *grow = qrow + kRowTile;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      s_[qb] = f32x16{};
      p_[qb] = f32x16{};
    }
    constexpr int D = kBwdSdpAhead;
    auto rdf = [&](int k) {
      const int ds = k >> 2, qb = (k >> 1) & 1;
      return *(const u32x4 *)(((k & 1) ? grow : qrow) + row_off<DP>(32 * qb + arow, 2 * ds + g));
    };
    u32x4 fr[D];
#pragma unroll
    for (int k = 0; k < D; ++k) fr[k] = rdf(k);
    static_for<0, kSdpSteps>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      __builtin_amdgcn_sched_barrier(0);
      constexpr int ds = k >> 2, qb = (k >> 1) & 1;
      if constexpr (k & 1)
        p_[qb] = mfma32x32x16<DT>(fr[k % D], vf[ds], p_[qb]);
      else
        s_[qb] = mfma32x32x16<DT>(fr[k % D], kf[ds], s_[qb]);
      static_for<0, kElPerStep>([&](auto ec) { vstep(std::integral_constant<int, k * kElPerStep + decltype(ec)::value>{}); });
      if constexpr (k + D < kSdpSteps) fr[k % D] = rdf(k + D);
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x16 s[2], p[2];
  if (n_steps > 0) {
    stage_rows_to(0, 0);
    stage_tr_to(0, 0);
    stage_rows_to(1, min(1, n_steps - 1));
    wait_vmem();
    __syncthreads();
    sdp(0, s, p, [](auto) {});
  }
  for (int i = 0; i < n_steps; ++i) {
    wait_vmem();
    // rows of step i + 1, transposed tiles and row terms of step i have landed; every wave is done
    // with the rows of step i, the transposed tiles and row terms of step i - 1
    __syncthreads();
    stage_rows_to(i & 1, min(i + 2, n_steps - 1));
    stage_tr_to((i + 1) & 1, min(i + 1, n_steps - 1));
    const char *tst = smem + kTrOff + (i & 1) * kPair;
    const char *qtr = tst, *gtr = tst + kRowTile;
    const float *lse_t = (const float *)(smem + kRtOff + (i & 1) * 2048), *d_t = lse_t + 256;
    const int qt0 = (t0 + i % per_head) * kBwdQTile;

    // P and dS of step i; register r of block qb is query qt0 + 32 qb + (r < 8 ? 8 g + r : 16 + 8 g
    // + r - 8). Masks only where the tile needs them (this wave's keys past S_kv, queries past S_q,
    // or keys past the causal diagonal of the tile's first query): elsewhere every element is kept,
    // with the same bits. Element k (qb = k / 16, half = k / 8 % 2, e = k % 8) runs beside MFMA k of
    // the next step's S / dP.
    const int wave_k_max = k0 + wave * 32 + 31;
    const bool need_mask = wave_k_max >= a.S_kv || qt0 + kBwdQTile > a.S_q || (CAUSAL && wave_k_max > qt0 + diag);
    u32x4 pb[4], sb[4];
    float pv0 = 0.0f, sv0 = 0.0f;
    float lse8[8], dd8[8];
    // the returned element step takes the mask choice by value (nothing of this call's frame)
    auto soft = [&](auto mask_c) {
      return [&, mask_c](auto kc) {
        constexpr bool MASK = decltype(mask_c)::value;
        constexpr int k = decltype(kc)::value;
        constexpr int qb = k >> 4, half = (k >> 3) & 1, e = k & 7;
        constexpr int qr = 32 * qb + 16 * half;  // + 8 g: first of this lane's 8 queries
        if constexpr (e == 0) {
          const f32x4 l0 = *(const f32x4 *)(lse_t + qr + 8 * g), l1 = *(const f32x4 *)(lse_t + qr + 8 * g + 4);
          const f32x4 d0 = *(const f32x4 *)(d_t + qr + 8 * g), d1 = *(const f32x4 *)(d_t + qr + 8 * g + 4);
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            lse8[x] = l0[x];
            lse8[4 + x] = l1[x];
            dd8[x] = d0[x];
            dd8[4 + x] = d1[x];
          }
        }
        const float lse_e = lse8[e], dd_e = dd8[e];
        constexpr int r = 8 * half + e;
        const int qi = qt0 + qr + 8 * g + e;
        const bool ok = !MASK || (key_ok && qi < a.S_q && (!CAUSAL || key <= qi + diag));
        const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][r], c, -lse_e));
        const float pv = ok ? pe : 0.0f;
        const float sv = ok ? pe * __builtin_fmaf(p[qb][r], a.scale, -dd_e) : 0.0f;
        if constexpr (e & 1) {
          constexpr int js = 2 * qb + half;
          pb[js][e >> 1] = pack2<DT>(pv0, pv);
          sb[js][e >> 1] = pack2<DT>(sv0, sv);
        } else {
          pv0 = pv;
          sv0 = sv;
        }
      };
    };
    f32x16 s2[2], p2[2];
    const int nslot = (i + 1) & 1;  // past the last step: rows of no step (never used)
    if (need_mask)
      sdp(nslot, s2, p2, soft(std::true_type{}));
    else
      sdp(nslot, s2, p2, soft(std::false_type{}));

    // dV^T += dO^T . P and dK^T += Q^T . dS: 8 kDb MFMAs in 2 kDb interleaved accumulation
    // chains (step k: 16-query step js = k / (2 kDb), d block (k / 2) % kDb, dV for even k, dK for
    // odd k), each transposed operand fragment read kBwdTrAhead steps ahead; every dV[db] / dK[db]
    // still accumulates js = 0..3 in order.
    {
      constexpr int D = kBwdTrAhead, kTrSteps = 8 * kDb;
      uint32_t tb[2 * kDb];
#pragma unroll
      for (int db = 0; db < kDb; ++db) {
        tb[2 * db] = tr_base<DP>(gtr, db, lane);
        tb[2 * db + 1] = tr_base<DP>(qtr, db, lane);
      }
      u32x4 tf[D];
      auto rdt = [&](auto kc) {
        constexpr int K = decltype(kc)::value;
        tf[K % D] = tr_frag<DP, K / (2 * kDb)>(tb[K % (2 * kDb)]);
      };
      static_for<0, D>([&](auto kc) { rdt(kc); });
      static_for<0, kTrSteps>([&](auto kc) {
        constexpr int K = decltype(kc)::value;
        constexpr int kAfter = (kTrSteps - 1 - K) < (D - 1) ? (kTrSteps - 1 - K) : (D - 1);  // fragments read after K
        __builtin_amdgcn_sched_barrier(0);
        lgkm_wait_n<2 * kAfter>(tf[K % D]);
        constexpr int js = K / (2 * kDb), db = (K >> 1) % kDb;
        if constexpr (K & 1)
          dk[db] = mfma32x32x16<DT>(tf[K % D], sb[js], dk[db]);
        else
          dv[db] = mfma32x32x16<DT>(tf[K % D], pb[js], dv[db]);
        if constexpr (K + D < kTrSteps) rdt(std::integral_constant<int, K + D>{});
      });
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      s[qb] = s2[qb];
      p[qb] = p2[qb];
    }
  }

  // dK[key][d], dV[key][d]: lane = key, register 4 rq + e of block db = d 32 db + 8 rq + 4 g + e.
  // The tiles go through LDS (free after the loop): each wave parks its 32 keys as rows of DP
  // elements (16-byte chunk c of row r at chunk c ^ kswz(r)), then stores whole rows, 16 bytes per
  // lane, so every store instruction writes complete rows instead of 8-byte pieces of 32 rows.
  // The last iterations issue clamped loads past the end into the stages; they must have landed
  // before the stages are reused for the output tiles (explicit, not left to the fence's own wait).
  wait_vmem();
  __syncthreads();  // every wave is done reading the last stage
  char *pk = smem + wave * (2 * 32 * kRowB), *pv = pk + 32 * kRowB;
#pragma unroll
  for (int db = 0; db < kDb; ++db)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const uint32_t o = (uint32_t)(col * kRowB + (((4 * db + rq) ^ L::kswz(col)) << 4) + 8 * g);
      *(u32x2 *)(pk + o) = u32x2{pack2<DT>(dk[db][4 * rq], dk[db][4 * rq + 1]),
                                 pack2<DT>(dk[db][4 * rq + 2], dk[db][4 * rq + 3])};
      *(u32x2 *)(pv + o) = u32x2{pack2<DT>(dv[db][4 * rq], dv[db][4 * rq + 1]),
                                 pack2<DT>(dv[db][4 * rq + 2], dv[db][4 * rq + 3])};
    }
  __syncthreads();
  uint16_t *dK = (uint16_t *)a.dK;
  uint16_t *dV = (uint16_t *)a.dV;
  const size_t base0 = ((size_t)b * a.S_kv * a.H_kv + hk) * a.D;
#pragma unroll
  for (int it = 0; it < 32 / L::kRpi; ++it) {
    const int r = L::kRpi * it + (int)((unsigned)lane / L::kCpr), pc = (int)((unsigned)lane % L::kCpr);
    const int kr = k0 + wave * 32 + r;
    const uint32_t o = (uint32_t)(r * kRowB + ((pc ^ L::kswz(r)) << 4));
    const u32x4 vk = *(const u32x4 *)(pk + o), vv = *(const u32x4 *)(pv + o);
    if (kr < a.S_kv && pc < nchunk) {
      const size_t e = base0 + (size_t)kr * a.H_kv * a.D + 8 * pc;
      *(u32x4 *)(dK + e) = vk;
      *(u32x4 *)(dV + e) = vv;
    }
  }
}

// ------------------------------------------------------------------------------------- dQ

template <int DT, bool CAUSAL, int DP>
__device__ __forceinline__ void attn_bwd_dq(const mtk_attn_bwd_kargs &a) {
  using L = AttnLayout<DP>;
  constexpr int kRowTile = L::kTile, kRowB = L::kRowB, kKs = L::kKs, kDb = L::kDb;
  // per stage: K rows, K transposed-read copy, V rows
  __shared__ __attribute__((aligned(1024))) char smem[2 * 3 * kRowTile];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..7
  const int g = lane >> 5, col = lane & 31;

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  int bh = id / a.q_blocks;
  int qblk = id - bh * a.q_blocks;
  if (CAUSAL) {  // heaviest (last) query blocks first
    causal_order(id, a.q_blocks, a.B * a.H, bh, qblk);
    qblk = a.q_blocks - 1 - qblk;
  }
  const int b = bh / a.H, h = bh - b * a.H;
  const int hk = h / (a.H / a.H_kv);  // K/V head of query head h
  const int q0 = qblk * kBwdQRows;
  const int nchunk = a.D >> 3;  // rows of D elements: chunks at or past nchunk are zeros
  const uint32_t rs = (uint32_t)a.H * a.D * 2, rkv = (uint32_t)a.H_kv * a.D * 2;
  const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * a.D * 2);
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H_kv + hk) * a.D * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rg = make_rsrc(a.dO, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const int diag = a.S_kv - a.S_q;
  const float c = a.scale_log2;

  // this lane's query (accumulator column): Q and dO rows as B operands, its lse and D
  const int qi = q0 + wave * 32 + col;
  const bool q_ok = qi < a.S_q;
  u32x4 qf[kKs], gf[kKs];
#pragma unroll
  for (int ds = 0; ds < kKs; ++ds) {
    const uint32_t off = q_ok && 2 * ds + g < nchunk ? qbase + (uint32_t)qi * rs + (uint32_t)(16 * ds + 8 * g) * 2u : kOOB;
    qf[ds] = buf_load16(rq, off);
    gf[ds] = buf_load16(rg, off);
  }
  const size_t ridx = ((size_t)b * a.H + h) * a.S_q + (size_t)(q_ok ? qi : 0);
  const float lse2 = q_ok ? a.Lt[ridx] : 0.0f;   // base-2 lse
  const float dterm = q_ok ? a.Dt[ridx] : 0.0f;  // D * scale

  int kv_end = a.S_kv;
  if (CAUSAL) kv_end = min(a.S_kv, q0 + kBwdQRows + diag);
  const int n_tiles = kv_end > 0 ? (kv_end + kBwdKTile - 1) / kBwdKTile : 0;

  auto stage = [&](int slot, int t) {
    char *st = smem + slot * 3 * kRowTile;
    const int valid = a.S_kv - t * kBwdKTile;
    const uint32_t tb = kvbase + (uint32_t)(t * kBwdKTile) * rkv;
    stage_rows<DP, 8 / L::kRpi, false>(rk, st, 8 * wave, tb, rkv, valid, nchunk, lane);
    stage_rows<DP, 8 / L::kRpi, true>(rk, st + kRowTile, 8 * wave, tb, rkv, valid, nchunk, lane);
    stage_rows<DP, 8 / L::kRpi, false>(rv, st + 2 * kRowTile, 8 * wave, tb, rkv, valid, nchunk, lane);
  };

  const int arow = bwd_swap_bits_2_3(col);  // MFMA row m reads key swap_bits_2_3(m) of the block
  f32x16 dq[kDb];
#pragma unroll
  for (int i = 0; i < kDb; ++i) dq[i] = f32x16{};

  if (n_tiles > 0) stage(0, 0);
  for (int t = 0; t < n_tiles; ++t) {
    wait_vmem();
    __syncthreads();  // tile t is in LDS; everyone is done with tile t-1's slot
    if (t + 1 < n_tiles) stage((t + 1) & 1, t + 1);
    const char *st = smem + (t & 1) * 3 * kRowTile;
    const char *krow = st, *ktr = st + kRowTile, *vrow = st + 2 * kRowTile;
    const int j0 = t * kBwdKTile;

    // The tile in two halves of 32 keys (kb = 0, 1): S^T and dP^T of the half, its dS^T, then the
    // dQ MFMAs of its two 16-key steps. Per d block dQ still accumulates the tile's key steps in
    // order (the same bits as a whole tile at once); half a tile of scores leaves the registers for
    // operand fragments read ahead (read just before its MFMA, every fragment waited for its read).
    const int wave_q0 = q0 + wave * 32;
    const bool need_mask = wave_q0 + 31 >= a.S_q || j0 + kBwdKTile > a.S_kv || (CAUSAL && j0 + kBwdKTile - 1 > wave_q0 + diag);
    static_for<0, 2>([&](auto kc) {
      constexpr int kb = decltype(kc)::value;
      // S^T and dP^T: 2 kKs MFMAs in two chains (step k: d step k / 2, S for even k, dP for odd
      // k), each fragment read kDqSdpAhead steps ahead; the fence per step keeps that order
      f32x16 s = f32x16{}, p = f32x16{};
      {
        constexpr int D = kDqSdpAhead;
        auto rdf = [&](int k) {
          return *(const u32x4 *)(((k & 1) ? vrow : krow) + row_off<DP>(32 * kb + arow, 2 * (k >> 1) + g));
        };
        u32x4 fr[D];
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int k = 0; k < D; ++k) fr[k] = rdf(k);
#pragma unroll
        for (int k = 0; k < 2 * kKs; ++k) {
          __builtin_amdgcn_sched_barrier(0);
          if (k & 1)
            p = mfma32x32x16<DT>(fr[k % D], gf[k >> 1], p);
          else
            s = mfma32x32x16<DT>(fr[k % D], qf[k >> 1], s);
          if (k + D < 2 * kKs) fr[k % D] = rdf(k + D);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
      }

      // dS^T; register r is key j0 + 32 kb + (r < 8 ? 8 g + r : 16 + 8 g + r - 8). Masks only where
      // the tile needs them (as in the dK/dV kernel).
      u32x4 sb[2];
      auto softmax_half = [&](auto mask_c) {
        constexpr bool MASK = decltype(mask_c)::value;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float sv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int r = 8 * half + e;
            const int kj = j0 + 32 * kb + 16 * half + 8 * g + e;
            const bool ok = !MASK || (q_ok && kj < a.S_kv && (!CAUSAL || kj <= qi + diag));
            const float pe = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -lse2));
            sv[e] = ok ? pe * __builtin_fmaf(p[r], a.scale, -dterm) : 0.0f;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) sb[half][e] = pack2<DT>(sv[2 * e], sv[2 * e + 1]);
        }
      };
      if (need_mask)
        softmax_half(std::true_type{});
      else
        softmax_half(std::false_type{});

      // dQ^T += K^T . dS^T for key steps 2 kb, 2 kb + 1: 2 kDb MFMAs (step K: d block K / 2, key
      // step 2 kb + K % 2), each transposed fragment read kDqTrAhead steps ahead
      {
        constexpr int D = kDqTrAhead < 2 * kDb ? kDqTrAhead : 2 * kDb, kQSteps = 2 * kDb;
        uint32_t tb[kDb];
#pragma unroll
        for (int db = 0; db < kDb; ++db) tb[db] = tr_base<DP>(ktr, db, lane);
        u32x4 tf[D];
        auto rdt = [&](auto kc2) {
          constexpr int K = decltype(kc2)::value;
          tf[K % D] = tr_frag<DP, 2 * kb + (K & 1)>(tb[K >> 1]);
        };
        static_for<0, D>([&](auto kc2) { rdt(kc2); });
        __builtin_amdgcn_s_setprio(1);
        static_for<0, kQSteps>([&](auto kc2) {
          constexpr int K = decltype(kc2)::value;
          constexpr int kAfter = (kQSteps - 1 - K) < (D - 1) ? (kQSteps - 1 - K) : (D - 1);  // fragments read after K
          __builtin_amdgcn_sched_barrier(0);
          lgkm_wait_n<2 * kAfter>(tf[K % D]);
          dq[K >> 1] = mfma32x32x16<DT>(tf[K % D], sb[K & 1], dq[K >> 1]);
          if constexpr (K + D < kQSteps) rdt(std::integral_constant<int, K + D>{});
        });
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
      }
    });
  }

  // dQ[qi][d]: lane = query, register 4 rq + e of block db = d 32 db + 8 rq + 4 g + e; parked in
  // LDS as rows of DP elements and stored as whole rows, as in the dK/dV kernel (no loads are in flight
  // here: the loop stages no tile past the last and waits for each tile it staged)
  __syncthreads();  // every wave is done reading the last stage
  char *pq = smem + wave * (32 * kRowB);
#pragma unroll
  for (int db = 0; db < kDb; ++db)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq)
      *(u32x2 *)(pq + col * kRowB + (((4 * db + rq) ^ L::kswz(col)) << 4) + 8 * g) =
          u32x2{pack2<DT>(dq[db][4 * rq], dq[db][4 * rq + 1]), pack2<DT>(dq[db][4 * rq + 2], dq[db][4 * rq + 3])};
  __syncthreads();
  uint16_t *dQ = (uint16_t *)a.dQ;
#pragma unroll
  for (int it = 0; it < 32 / L::kRpi; ++it) {
    const int r = L::kRpi * it + (int)((unsigned)lane / L::kCpr), pc = (int)((unsigned)lane % L::kCpr);
    const int qr = q0 + wave * 32 + r;
    const u32x4 v = *(const u32x4 *)(pq + r * kRowB + ((pc ^ L::kswz(r)) << 4));
    if (qr < a.S_q && pc < nchunk) *(u32x4 *)(dQ + (((size_t)b * a.S_q + qr) * a.H + h) * a.D + 8 * pc) = v;
  }
}

}  // namespace mtk

using namespace mtk;

#define BWD_PRE(NAME, DT) \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_attn_bwd_kargs a) { attn_bwd_pre<DT>(a); }
#define BWD_DKDV(NAME, DT, CAUSAL, DP)                                               \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_attn_bwd_kargs a) { \
    attn_bwd_dkdv<DT, CAUSAL, DP>(a);                                                \
  }
#define BWD_DQ(NAME, DT, CAUSAL, DP)                                                 \
  extern "C" __global__ void __launch_bounds__(512) NAME(const mtk_attn_bwd_kargs a) { \
    attn_bwd_dq<DT, CAUSAL, DP>(a);                                                  \
  }

BWD_PRE(mtk_attn_bwd_pre_f16, DT_F16)
BWD_PRE(mtk_attn_bwd_pre_bf16, DT_BF16)
BWD_DKDV(mtk_attn_bwd_dkdv_f16, DT_F16, false, 128)
BWD_DKDV(mtk_attn_bwd_dkdv_bf16, DT_BF16, false, 128)
BWD_DKDV(mtk_attn_bwd_dkdv_f16_causal, DT_F16, true, 128)
BWD_DKDV(mtk_attn_bwd_dkdv_bf16_causal, DT_BF16, true, 128)
BWD_DQ(mtk_attn_bwd_dq_f16, DT_F16, false, 128)
BWD_DQ(mtk_attn_bwd_dq_bf16, DT_BF16, false, 128)
BWD_DQ(mtk_attn_bwd_dq_f16_causal, DT_F16, true, 128)
BWD_DQ(mtk_attn_bwd_dq_bf16_causal, DT_BF16, true, 128)
// head dimensions up to 64: the same kernels laid out for 64 (rows of 128 bytes)
BWD_DKDV(mtk_attn_bwd_dkdv_d64_f16, DT_F16, false, 64)
BWD_DKDV(mtk_attn_bwd_dkdv_d64_bf16, DT_BF16, false, 64)
BWD_DKDV(mtk_attn_bwd_dkdv_d64_f16_causal, DT_F16, true, 64)
BWD_DKDV(mtk_attn_bwd_dkdv_d64_bf16_causal, DT_BF16, true, 64)
BWD_DQ(mtk_attn_bwd_dq_d64_f16, DT_F16, false, 64)
BWD_DQ(mtk_attn_bwd_dq_d64_bf16, DT_BF16, false, 64)
BWD_DQ(mtk_attn_bwd_dq_d64_f16_causal, DT_F16, true, 64)
BWD_DQ(mtk_attn_bwd_dq_d64_bf16_causal, DT_BF16, true, 64)
