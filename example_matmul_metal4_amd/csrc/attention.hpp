// Flash-attention forward for gfx950, fp16/bf16 in, fp32 softmax and accumulate: the 128-query
// kernel, templated on the head dimension.
//
// Replaces the reference's generated `attention` kernel (Sources/attention/attention.swift:133-380):
// O = softmax(Q K^T / sqrt(D)) V with base-2 online softmax (its dotScale = log2(e)/sqrt(D),
// attention.swift:24), per (batch, head), tensors laid out [B][S][H][D] (attention.swift:466-468
// with a batch dimension). Extensions: batch, causal mask (keys j <= i + S_kv - S_q), bf16, and
// grouped K/V heads: K, V are [B][S_kv][H_kv][D] and query head h reads K/V head h / (H / H_kv)
// (the reference declares Hk but indexes K/V with the query head, attention.swift:155-156).
//
// Head dimension. The reference takes any head dimension K: its generator tiles K in blocks
// (kBlocks, attention.swift:25), keeps one output accumulator per block and masks the last block's
// store (84-91); the Q.K^T product walks K with a remainder block (192-199). Here the kernel is
// compiled for a padded head dimension DP (a multiple of 32: 64, 128 or 256) and runs any D <= DP:
//   * D % 8 == 0: every 16-byte chunk of a row lies entirely inside or outside the row, so chunks
//     past D are loaded as zeros (out-of-range buffer offsets) for Q and K, skipped for V, and the
//     output is stored for d < D only. The padding contributes exact zeros to Q.K^T.
//   * any other D (GEN = true): rows are no longer 16-byte aligned; Q, K and V are loaded element by
//     element (elements past D read as zero), staged into the same LDS layout by ordinary LDS
//     writes, and O is stored element by element. Same arithmetic, slower staging.
//
// Work decomposition
//   * Workgroup = 4 wavefronts = 128 query rows of one (batch, head); each wave owns 32 queries,
//     held in registers as the B operand of S^T = K . Q^T. K and V stream through LDS in tiles of
//     64 keys, two LDS slots each, filled by direct-to-LDS loads (no register staging).
//   * Scores are computed transposed on 32x32x16 MFMA: the accumulator column (lane % 32) is the
//     query, so each lane owns one query and the softmax row max / row sum are in-register
//     reductions plus one exchange with lane ^ 32 (v_permlane32_swap, no LDS round trip).
//   * K rows are fed to the MFMA in a permuted order (MFMA row m reads key swap_bits_2_3(m)); with
//     that order accumulator register r of lane (i, g = lane/32) holds key 8g + r (r < 8) or
//     16 + 8g + (r - 8), which is exactly the B-operand layout of the P.V MFMA (O^T = V^T . P^T).
//     P goes from the S accumulators to the next MFMA with only an fp32 -> 16-bit conversion.
//   * V stays [key][d] in LDS; the V^T operand is read with transposed LDS reads
//     (ds_read_b64_tr_b16, two per fragment). The row swizzles (AttnLayout) keep the K row reads and
//     the V^T transposed reads free of bank conflicts for every DP (64 banks of 4 bytes).
//   * Software pipeline across key tiles, in one wavefront's instruction stream: the MFMAs of
//     S(t+1) are interleaved with the exponentials of softmax(t), and the P(t).V(t) MFMAs with the
//     row maxima of S(t+1), so the matrix cores and the vector ALUs work at the same time.
//   * Lazy rescale: the exponent offset of a query moves only when its running max exceeds it by
//     more than 8 (log2 domain), so P <= 2^8 (exact in fp16/bf16 range) and O is rescaled on few
//     tiles; 1/l at the end makes the result independent of the offsets.
//   * Global reads are raw buffer loads: keys past S_kv and queries past S_q read zero.
//   * Causal: a workgroup stops at its last visible key tile; heavy query blocks are dispatched
//     first; query blocks of one (batch, head) are kept on one XCD for K/V reuse in L2.
#pragma once

#include "device.hpp"

// Wave issue priority over phase A of the 128-query kernel (S(t+1) MFMAs with the exponentials of
// tile t): of the two wavefronts of a SIMD (two workgroups per CU, out of step), the one in phase A
// issues first. 1-2.5 % faster than equal priorities (priority over phase B instead: mixed).

namespace mtk {

constexpr int kBQ = 128;
constexpr int kBKV = 64;
constexpr float kRescaleSlack = 8.0f;  // log2-domain headroom before O is rescaled

__device__ __forceinline__ int swap_bits_2_3(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// LDS layout of one K or V tile (64 keys x DP head elements) for padded head dimension DP.
template <int DP>
struct AttnLayout {
  static_assert(DP == 64 || DP == 128 || DP == 256, "padded head dimension");
  static constexpr int kRowB = DP * 2;             // bytes per key row
  static constexpr int kTile = kBKV * kRowB;       // bytes per tile
  static constexpr int kCpr = DP / 8;              // 16-byte chunks per row
  static constexpr int kRpi = 64 / kCpr;           // rows per 1 KB staging instruction
  static constexpr int kNi = kTile / 4 / 1024;     // staging instructions per wave per tile
  static constexpr int kKs = DP / 16;              // k-steps of S = K.Q^T
  static constexpr int kDb = DP / 32;              // 32-wide output blocks
  // K tile, read as rows by 16 lanes at a time (16 bytes each): rows of 256 B or more start on the
  // same bank, so the chunk is XORed with the row; 128-byte rows pair up in one 256-byte bank line,
  // so the XOR uses row / 2.
  static __device__ __forceinline__ int kswz(int row) { return DP >= 128 ? (row & 15) : ((row >> 1) & 7); }
  // V tile, read transposed by 32 lanes at a time (8 bytes each, 4 rows x 64 bytes): the four rows'
  // 64-byte windows are moved apart by XORing the chunk with a multiple of 4.
  static __device__ __forceinline__ int vswz(int row) { return DP >= 128 ? 4 * (row & 3) : 4 * ((row >> 1) & 1); }
};

// Row log-sum-exp for the backward (natural log of sum_j exp(s_ij * scale)): the exponent offset
// m_off (log2 domain) plus log2 of the row sum, converted to natural log; -inf for a query that
// sees no key. One lane of each lane pair (lane, lane ^ 32) writes.
__device__ __forceinline__ void store_lse(const mtk_attn_kargs &a, int b, int h, int qi, int g, float m_off,
                                          float l_tot) {
  if (a.lse != nullptr && qi < a.S_q && g == 0) {
    const float lse2 = l_tot > 0.0f ? m_off + __builtin_amdgcn_logf(l_tot) : -INFINITY;
    a.lse[((size_t)b * a.H + h) * a.S_q + qi] = lse2 * 0.6931471805599453f;
  }
}

// 8 consecutive 16-bit elements at byte offset `off`, element e read only when e < n (else zero):
// for rows that are not 16-byte aligned (GEN kernels).
__device__ __forceinline__ u32x4 load8_elems(rsrc_t r, uint32_t off, int n) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = (2 * i < n) ? buf_load2(r, off + 4u * i) : 0u;
    const uint32_t hi = (2 * i + 1 < n) ? buf_load2(r, off + 4u * i + 2u) : 0u;
    w[i] = (lo & 0xffffu) | (hi << 16);
  }
  return u32x4{w[0], w[1], w[2], w[3]};
}

template <int DT, bool CAUSAL, int DP, bool GEN>
__device__ __forceinline__ void attn_fwd(const mtk_attn_kargs &a) {
  using L = AttnLayout<DP>;
  constexpr int kTile = L::kTile, kRowB = L::kRowB, kNi = L::kNi, kKs = L::kKs, kDb = L::kDb;
  // K slots 0, 1 then V slots 0, 1
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTile];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, col = lane & 31;
  const int D = a.D;  // head dimension (<= DP)

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  int bh = id / a.q_blocks;
  int qb = id - bh * a.q_blocks;
  if (CAUSAL) {  // heaviest (last) query blocks first
    causal_order(id, a.q_blocks, a.B * a.H, bh, qb);
    qb = a.q_blocks - 1 - qb;
  }
  const int b = bh / a.H, h = bh - b * a.H;
  const int q0 = qb * kBQ;
  const uint32_t rs = (uint32_t)a.H * D * 2;      // bytes between sequence positions of Q / O
  const uint32_t rkv = (uint32_t)a.H_kv * D * 2;  // ... of K / V ([B][S_kv][H_kv][D])
  const int hk = h / (a.H / a.H_kv);              // the key/value head this query head reads
  const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * D * 2);
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H_kv + hk) * D * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const int diag = a.S_kv - a.S_q;  // key j is visible to query i iff j <= i + diag (causal)

  // ---- this lane's query row, as the B operand of S^T = K . Q^T (k-steps of 16 dims); dims past
  // D read as zero
  const int qi = q0 + wave * 32 + col;
  u32x4 qf[kKs];
#pragma unroll
  for (int ds = 0; ds < kKs; ++ds) {
    const int d0 = 16 * ds + 8 * g;
    const uint32_t off = qbase + (uint32_t)qi * rs + (uint32_t)d0 * 2u;
    if constexpr (GEN)
      qf[ds] = load8_elems(rq, off, qi < a.S_q ? D - d0 : 0);
    else
      qf[ds] = buf_load16(rq, (qi < a.S_q && d0 < D) ? off : kOOB);
  }

  int kv_end = a.S_kv;
  if (CAUSAL) kv_end = min(a.S_kv, q0 + kBQ + diag);
  const int n_tiles = kv_end > 0 ? (kv_end + kBKV - 1) / kBKV : 0;

  // ---- staging: each wave fills a quarter of a tile, kNi instructions of 1 KB (kRpi rows each).
  // LDS chunk pc of row r holds global chunk pc ^ kswz(r) (K) or pc ^ vswz(r) (V); chunks past D
  // read as zero (K) or are not loaded (V: they only reach output dims that are never stored).
  int srow[kNi];
  uint32_t kcol[kNi], vcol[kNi], klane[kNi], vlane[kNi];
  bool kin[kNi], vin[kNi];
#pragma unroll
  for (int i = 0; i < kNi; ++i) {
    srow[i] = (wave * kNi + i) * L::kRpi + lane / L::kCpr;
    const int pc = lane % L::kCpr;
    const int kc = pc ^ L::kswz(srow[i]), vc = pc ^ L::vswz(srow[i]);
    kcol[i] = 16u * (uint32_t)kc;
    vcol[i] = 16u * (uint32_t)vc;
    kin[i] = 8 * kc < D;
    vin[i] = 8 * vc < D;
    klane[i] = kin[i] ? (uint32_t)srow[i] * rkv + kcol[i] : kOOB;
    vlane[i] = vin[i] ? (uint32_t)srow[i] * rkv + vcol[i] : kOOB;
  }
  // A tile inside S_kv goes out with its base as the uniform scalar offset (no per-row work); the
  // tile crossing S_kv is loaded row-checked, rows past S_kv reading zero. GEN kernels load the
  // chunk element-wise into registers and write it to the same LDS place (the slot is free when
  // the load is issued; the barrier before its first read waits for the LDS writes).
  auto issue = [&](const rsrc_t &r, char *dst, const uint32_t (&lane_off)[kNi], const uint32_t (&colb)[kNi],
                   const bool (&in)[kNi], int t) {
    const int key0 = t * kBKV;
    if constexpr (GEN) {
#pragma unroll
      for (int i = 0; i < kNi; ++i) {
        const int key = key0 + srow[i];
        const int n = (key < a.S_kv && in[i]) ? D - (int)(colb[i] >> 1) : 0;
        *(u32x4 *)(dst + i * 1024 + lane * 16) = load8_elems(r, kvbase + (uint32_t)key * rkv + colb[i], n);
      }
    } else if (key0 + kBKV <= a.S_kv) {
      const uint32_t tb = kvbase + (uint32_t)key0 * rkv;
#pragma unroll
      for (int i = 0; i < kNi; ++i) lds_direct16_s(r, dst + i * 1024, lane_off[i], tb);
    } else {
#pragma unroll
      for (int i = 0; i < kNi; ++i) {
        const int key = key0 + srow[i];
        lds_direct16(r, dst + i * 1024, (key < a.S_kv && in[i]) ? kvbase + (uint32_t)key * rkv + colb[i] : kOOB);
      }
    }
  };
  auto issue_k = [&](int slot, int t) { issue(rk, smem + slot * kTile + wave * (kTile / 4), klane, kcol, kin, t); };
  auto issue_v = [&](int slot, int t) { issue(rv, smem + (2 + slot) * kTile + wave * (kTile / 4), vlane, vcol, vin, t); };

  // ---- fragment reads
  // Per-lane LDS offsets are computed once; per tile only the slot base is added (K: one offset per
  // k-step, key block 1 at +32 rows; V^T: one per d block, key step js and half e at +16 js + 4 e
  // rows, folded into the instructions' offset fields).
  const int krow = swap_bits_2_3(col);
  uint32_t kq[kKs];
#pragma unroll
  for (int ds = 0; ds < kKs; ++ds) kq[ds] = (uint32_t)(krow * kRowB + (((2 * ds + g) ^ L::kswz(krow)) << 4));
  // V^T fragment for d block db, key step js (16 keys): lane (h = lane / 16, s = lane % 16) gets
  // d = 32 db + lane % 32 at keys 16 js + 8 (lane / 32) + 0..7 (two transposed reads, rows
  // 16 js + 8 (h / 2) + 4 e + s / 4); the row swizzle depends only on s / 4 and h / 2.
  const int vs = lane & 15, vh = lane >> 4;
  uint32_t vq[kDb];
#pragma unroll
  for (int db = 0; db < kDb; ++db) {
    const int d = 32 * db + 16 * (vh & 1) + 4 * (vs & 3);
    const int row = 8 * (vh >> 1) + (vs >> 2);
    vq[db] = lds_addr(smem) + (uint32_t)(row * kRowB + 16 * ((d >> 3) ^ L::vswz(row)) + 2 * (d & 7));
  }
  auto kfrag = [&](const uint32_t (&kb)[kKs], int blk, int ds) -> u32x4 {
    return *(const u32x4 *)(smem + kb[ds] + blk * 32 * kRowB);
  };
  auto kbase = [&](uint32_t (&kb)[kKs], int slot) {
#pragma unroll
    for (int ds = 0; ds < kKs; ++ds) kb[ds] = kq[ds] + (uint32_t)(slot * kTile);
  };
  auto vread = [&](u32x4 (&dst)[4], uint32_t vb) {
    static_for<0, 4>([&](auto jc) {
      constexpr int JS = decltype(jc)::value;
      const u32x2 w0 = ds_read_tr16_at<16 * kRowB * JS>(vb);
      const u32x2 w1 = ds_read_tr16_at<16 * kRowB * JS + 4 * kRowB>(vb);
      dst[JS] = u32x4{w0.x, w0.y, w1.x, w1.y};
    });
  };

  float m_off = -INFINITY;  // exponent offset of this lane's query (log2 domain)
  float l_run = 0.0f;       // this lane's half of the running row sum
  f32x16 o[kDb];
#pragma unroll
  for (int i = 0; i < kDb; ++i) o[i] = f32x16{};
  const float c = a.scale_log2;
  const int wave_q_min = q0 + wave * 32;
  // the 8 register pairs of each score block are exponentiated over the k-steps of S(t+1):
  // kPps pairs every kEvery k-steps
  constexpr int kEvery = kKs > 8 ? kKs / 8 : 1;
  constexpr int kPps = kKs >= 8 ? 1 : 8 / kKs;

  if (n_tiles > 0) {
    f32x16 s0 = f32x16{}, s1 = f32x16{};  // S^T of the tile being softmaxed
    issue_k(0, 0);
    wait_vmem();
    __syncthreads();
    if (n_tiles > 1) issue_k(1, 1);
    issue_v(0, 0);
    {
      uint32_t kb[kKs];
      kbase(kb, 0);
#pragma unroll
      for (int ds = 0; ds < kKs; ++ds) {
        s0 = mfma32x32x16<DT>(kfrag(kb, 0, ds), qf[ds], s0);
        s1 = mfma32x32x16<DT>(kfrag(kb, 1, ds), qf[ds], s1);
      }
    }
    // row max of tile 0
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = vmax3(mx, s0[r], s1[r]);

    for (int t = 0; t < n_tiles; ++t) {
      wait_vmem();
      __syncthreads();  // K(t+1) and V(t) are in LDS; K slot t&1 and V slot (t+1)&1 are free
      // (on the last tile, S(t+1) is computed from whatever the K slot holds and discarded)
      if (t + 2 < n_tiles) issue_k(t & 1, t + 2);
      if (t + 1 < n_tiles) issue_v((t + 1) & 1, t + 1);
      uint32_t kn[kKs];
      kbase(kn, (t + 1) & 1);
      const uint32_t vt = (uint32_t)((2 + (t & 1)) * kTile);

      // mask of tile t (only tiles crossing S_kv or the causal diagonal)
      const int j0 = t * kBKV;
      if ((j0 + kBKV > a.S_kv) || (CAUSAL && j0 + kBKV - 1 > wave_q_min + diag)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kr0 = (r < 8) ? (8 * g + r) : (16 + 8 * g + (r - 8));
          const int key0 = j0 + kr0, key1 = j0 + 32 + kr0;
          s0[r] = (key0 < a.S_kv && (!CAUSAL || key0 <= qi + diag)) ? s0[r] : -INFINITY;
          s1[r] = (key1 < a.S_kv && (!CAUSAL || key1 <= qi + diag)) ? s1[r] : -INFINITY;
        }
        mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = vmax3(mx, s0[r], s1[r]);
      }
      mx = half_max(mx);
      const float m_tile = mx * c;
      float alpha = 1.0f;
      if (m_tile > m_off + kRescaleSlack) {
        alpha = __builtin_amdgcn_exp2f(m_off - m_tile);
        m_off = m_tile;
      }
      const float moff = m_off == -INFINITY ? 0.0f : m_off;  // fully masked so far: P = 0
      // rescale here, not after phase A: a branch between the MFMAs and the exponentials would let
      // the compiler sink the exponentials past it and lose the interleave
      l_run *= alpha;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int i = 0; i < kDb; ++i) o[i] *= alpha;
      }

      // phase A: S(t+1) MFMAs interleaved with exp / sum / pack of tile t. At DP = 256 (one
      // wavefront per SIMD, nothing else to cover a read's latency) the K fragments of both key
      // blocks are read by inline asm kLookA k-steps ahead into a ring; each k-step waits until only
      // the reads issued after its own are outstanding (LDS reads complete in order), its registers
      // tied to the wait (D = 256 config 5 shape: 1532 -> 1446 us, causal 835 -> 795 us). With two
      // wavefronts per SIMD (DP <= 128) the compiler's placement, each pair read right before its
      // MFMAs, measured faster (D = 64: 399 against 424 us; D = 128 causal: 356 against 361 us).
      __builtin_amdgcn_s_setprio(1);
      f32x16 n0 = f32x16{}, n1 = f32x16{};
      u32x4 pf[4];
      float psum = 0.0f;
      constexpr bool kRingA = DP >= 256;
      constexpr int kLookA = 4;
      u32x4 kring[kLookA + 1][2];
      const uint32_t kslot = lds_addr(smem);
      auto kread = [&](auto dc) {
        constexpr int ds = decltype(dc)::value;
        if constexpr (ds < kKs) {
          kring[ds % (kLookA + 1)][0] = ds_read_b128_at<0>(kslot + kn[ds]);
          kring[ds % (kLookA + 1)][1] = ds_read_b128_at<32 * kRowB>(kslot + kn[ds]);
        }
      };
      if constexpr (kRingA) static_for<0, kLookA>(kread);
      static_for<0, kKs>([&](auto dc) {
        constexpr int ds = decltype(dc)::value;
        if constexpr (kRingA) {
          kread(std::integral_constant<int, ds + kLookA>{});
          constexpr int kYounger = 2 * (ds + kLookA < kKs ? kLookA : kKs - 1 - ds);
          asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(kring[ds % (kLookA + 1)][0]), "+v"(kring[ds % (kLookA + 1)][1])
                       : "i"(kYounger));
          n0 = mfma32x32x16<DT>(kring[ds % (kLookA + 1)][0], qf[ds], n0);
          n1 = mfma32x32x16<DT>(kring[ds % (kLookA + 1)][1], qf[ds], n1);
        } else {
          n0 = mfma32x32x16<DT>(kfrag(kn, 0, ds), qf[ds], n0);
          n1 = mfma32x32x16<DT>(kfrag(kn, 1, ds), qf[ds], n1);
        }
        if constexpr ((ds + 1) % kEvery == 0) {
#pragma unroll
          for (int pp = 0; pp < kPps; ++pp) {
            // register pair r, r+1 of both blocks
            const int r = 2 * ((ds / kEvery) * kPps + pp);
            const float p00 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], c, -moff));
            const float p01 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r + 1], c, -moff));
            const float p10 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], c, -moff));
            const float p11 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r + 1], c, -moff));
            psum += (p00 + p01) + (p10 + p11);
            // registers 0..7 -> keys 0..15 of the block (P k-step 2*blk), 8..15 -> keys 16..31
            pf[r >> 3][(r & 7) >> 1] = pack2<DT>(p00, p01);
            pf[2 + (r >> 3)][(r & 7) >> 1] = pack2<DT>(p10, p11);
          }
        }
      });
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
      l_run += psum;

      // phase B: O^T += V^T(t) . P^T(t), interleaved with the row max of S(t+1); the next d
      // block's V^T fragments are read while the current block's MFMAs run. The 16 register
      // maxima are spread over the d blocks.
      constexpr int kMaxPer = kDb >= 4 ? 4 : 16 / kDb;  // registers per d block (first 16 / kMaxPer blocks)
      u32x4 vf[2][4];
      vread(vf[0], vq[0] + vt);
      float mn = -INFINITY;
#pragma unroll
      for (int db = 0; db < kDb; ++db) {
        const int cb = db & 1, nb = cb ^ 1;
        lgkm_wait0(vf[cb]);
        if (db + 1 < kDb) vread(vf[nb], vq[db + 1] + vt);
#pragma unroll
        for (int js = 0; js < 4; ++js) o[db] = mfma32x32x16<DT>(vf[cb][js], pf[js], o[db]);
        if (db * kMaxPer < 16) {
#pragma unroll
          for (int r = db * kMaxPer; r < db * kMaxPer + kMaxPer; ++r) mn = vmax3(mn, n0[r], n1[r]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      s0 = n0;
      s1 = n1;
      mx = mn;
    }
  }

  // ---- epilogue: O[qi][h][d] = O^T[d][qi] / l, dims d < D
  const float l_tot = half_sum(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  store_lse(a, b, h, qi, g, m_off, l_tot);
  if (qi < a.S_q) {
    uint16_t *O = (uint16_t *)a.O;
    const size_t obase = (((size_t)b * a.S_q + qi) * a.H + h) * D;
#pragma unroll
    for (int db = 0; db < kDb; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + 8 * rq + 4 * g;
        const uint32_t w0 = pack2<DT>(o[db][4 * rq + 0] * inv, o[db][4 * rq + 1] * inv);
        const uint32_t w1 = pack2<DT>(o[db][4 * rq + 2] * inv, o[db][4 * rq + 3] * inv);
        if constexpr (GEN) {
          const uint16_t e[4] = {(uint16_t)w0, (uint16_t)(w0 >> 16), (uint16_t)w1, (uint16_t)(w1 >> 16)};
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (d + k < D) O[obase + d + k] = e[k];
        } else if (d < D) {
          *(u32x2 *)(O + obase + d) = u32x2{w0, w1};
        }
      }
  }
}

}  // namespace mtk

#define MTK_ATTN_FWD_KERNEL(NAME, DT, CAUSAL, DP, GEN, WAVES)                                      \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WAVES, WAVES))) \
  NAME(const mtk_attn_kargs a) {                                                                   \
    mtk::attn_fwd<DT, CAUSAL, DP, GEN>(a);                                                         \
  }
