// Flash-attention forward for gfx950 (head dim 128), fp16/bf16 in, fp32 softmax and accumulate.
//
// Replaces the reference's generated `attention` kernel (Sources/attention/attention.swift:133-380):
// O = softmax(Q K^T / sqrt(D)) V with base-2 online softmax (its dotScale = log2(e)/sqrt(D),
// attention.swift:24), per (batch, head), tensors laid out [B][S][H][D] (attention.swift:466-468
// with a batch dimension). Extensions: batch, causal mask (keys j <= i + S_kv - S_q), bf16.
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
//     (ds_read_b64_tr_b16, two per fragment). K rows (256 B) use a chunk ^ (row & 15) swizzle,
//     V rows chunk ^ 4 * (row & 3): both keep the fragment reads free of bank conflicts.
//   * Software pipeline across key tiles, in one wavefront's instruction stream: the MFMAs of
//     S(t+1) are interleaved with the exponentials of softmax(t), and the P(t).V(t) MFMAs with the
//     row maxima of S(t+1), so the matrix cores and the vector ALUs work at the same time.
//   * Lazy rescale: the exponent offset of a query moves only when its running max exceeds it by
//     more than 8 (log2 domain), so P <= 2^8 (exact in fp16/bf16 range) and O is rescaled on few
//     tiles; 1/l at the end makes the result independent of the offsets.
//   * Global reads are raw buffer loads: keys past S_kv and queries past S_q read zero.
//   * Causal: a workgroup stops at its last visible key tile; heavy query blocks are dispatched
//     first; query blocks of one (batch, head) are kept on one XCD for K/V reuse in L2.
#include "device.hpp"

namespace mtk {

constexpr int kD = 128;
constexpr int kBQ = 128;
constexpr int kBKV = 64;
constexpr int kTile = kBKV * kD * 2;   // bytes of one K or V tile in LDS
constexpr float kRescaleSlack = 8.0f;  // log2-domain headroom before O is rescaled

__device__ __forceinline__ int swap_bits_2_3(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

__device__ __forceinline__ uint32_t k_off(int row, int chunk) {  // K tile: 64 rows x 256 B
  return (uint32_t)(row * 256 + ((chunk ^ (row & 15)) << 4));
}

template <int DT, bool CAUSAL>
__device__ __forceinline__ void attn_fwd(const mtk_attn_kargs &a) {
  // K slots 0, 1 then V slots 0, 1
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTile];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, col = lane & 31;

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = id / a.q_blocks;
  int qb = id - bh * a.q_blocks;
  if (CAUSAL) qb = a.q_blocks - 1 - qb;  // heaviest query blocks first
  const int b = bh / a.H, h = bh - b * a.H;
  const int q0 = qb * kBQ;
  const uint32_t rs = (uint32_t)a.H * kD * 2;  // bytes between sequence positions
  const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * kD * 2);
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H + h) * kD * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const int diag = a.S_kv - a.S_q;  // key j is visible to query i iff j <= i + diag (causal)

  // ---- this lane's query row, as the B operand of S^T = K . Q^T (8 k-steps of 16 dims)
  const int qi = q0 + wave * 32 + col;
  u32x4 qf[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds)
    qf[ds] = buf_load16(rq, qi < a.S_q ? qbase + (uint32_t)qi * rs + (uint32_t)(16 * ds + 8 * g) * 2u : kOOB);

  int kv_end = a.S_kv;
  if (CAUSAL) kv_end = min(a.S_kv, q0 + kBQ + diag);
  const int n_tiles = kv_end > 0 ? (kv_end + kBKV - 1) / kBKV : 0;

  // ---- direct-to-LDS staging: each wave fills 4 KB of a tile (4 rows of 256 B per instruction).
  // K: LDS chunk pc of row r holds global chunk pc ^ (r & 15); V: pc ^ 4 * (r & 3).
  int srow[4];
  uint32_t kcol[4], vcol[4], klane[4], vlane[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    srow[i] = (wave * 4 + i) * 4 + (lane >> 4);
    const int pc = lane & 15;
    kcol[i] = 16u * (uint32_t)(pc ^ (srow[i] & 15));
    vcol[i] = 16u * (uint32_t)(pc ^ (4 * (srow[i] & 3)));
    klane[i] = (uint32_t)srow[i] * rs + kcol[i];
    vlane[i] = (uint32_t)srow[i] * rs + vcol[i];
  }
  // A tile inside S_kv goes out with its base as the uniform scalar offset (no per-row work); the
  // tile crossing S_kv is loaded row-checked, rows past S_kv reading zero.
  auto issue = [&](const rsrc_t &r, char *dst, const uint32_t (&lane_off)[4], const uint32_t (&col)[4], int t) {
    const int key0 = t * kBKV;
    if (key0 + kBKV <= a.S_kv) {
      const uint32_t tb = kvbase + (uint32_t)key0 * rs;
#pragma unroll
      for (int i = 0; i < 4; ++i) lds_direct16_s(r, dst + i * 1024, lane_off[i], tb);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = key0 + srow[i];
        lds_direct16(r, dst + i * 1024, key < a.S_kv ? kvbase + (uint32_t)key * rs + col[i] : kOOB);
      }
    }
  };
  auto issue_k = [&](int slot, int t) { issue(rk, smem + slot * kTile + wave * 4096, klane, kcol, t); };
  auto issue_v = [&](int slot, int t) { issue(rv, smem + (2 + slot) * kTile + wave * 4096, vlane, vcol, t); };

  // ---- fragment reads
  // Fragment reads. Per-lane LDS offsets are computed once; per tile only the slot base is added
  // (K: one offset per k-step, key block 1 at +8192; V^T: one per d block, key step js and half e
  // at +4096 js + 1024 e, folded into the instructions' offset fields).
  const int krow = swap_bits_2_3(col);
  uint32_t kq[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) kq[ds] = k_off(krow, 2 * ds + g);
  // V^T fragment for d block db, key step js (16 keys): lane (h = lane / 16, s = lane % 16) gets
  // d = 32 db + lane % 32 at keys 16 js + 8 (lane / 32) + 0..7 (two transposed reads, rows
  // 16 js + 8 (h / 2) + 4 e + s / 4); the row swizzle depends only on s / 4.
  const int vs = lane & 15, vh = lane >> 4;
  uint32_t vq[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const int d = 32 * db + 16 * (vh & 1) + 4 * (vs & 3);
    const int row = 8 * (vh >> 1) + (vs >> 2);
    vq[db] = lds_addr(smem) + (uint32_t)(row * 256 + 16 * ((d >> 3) ^ (4 * (row & 3))) + 2 * (d & 7));
  }
  auto kfrag = [&](const uint32_t (&kb)[8], int blk, int ds) -> u32x4 {
    return *(const u32x4 *)(smem + kb[ds] + blk * 8192);
  };
  auto kbase = [&](uint32_t (&kb)[8], int slot) {
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) kb[ds] = kq[ds] + (uint32_t)(slot * kTile);
  };
  auto vread = [&](u32x4 (&dst)[4], uint32_t vb) {
    static_for<0, 4>([&](auto jc) {
      constexpr int JS = decltype(jc)::value;
      const u32x2 w0 = ds_read_tr16_at<4096 * JS>(vb);
      const u32x2 w1 = ds_read_tr16_at<4096 * JS + 1024>(vb);
      dst[JS] = u32x4{w0.x, w0.y, w1.x, w1.y};
    });
  };

  float m_off = -INFINITY;  // exponent offset of this lane's query (log2 domain)
  float l_run = 0.0f;       // this lane's half of the running row sum
  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  const float c = a.scale_log2;
  const int wave_q_min = q0 + wave * 32;

  if (n_tiles > 0) {
    f32x16 s0 = f32x16{}, s1 = f32x16{};  // S^T of the tile being softmaxed
    issue_k(0, 0);
    wait_vmem();
    __syncthreads();
    if (n_tiles > 1) issue_k(1, 1);
    issue_v(0, 0);
    {
      uint32_t kb[8];
      kbase(kb, 0);
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) {
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
      uint32_t kn[8];
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
        for (int i = 0; i < 4; ++i) o[i] *= alpha;
      }

      // phase A: S(t+1) MFMAs interleaved with exp / sum / pack of tile t
      f32x16 n0 = f32x16{}, n1 = f32x16{};
      u32x4 pf[4];
      float psum = 0.0f;
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) {
        n0 = mfma32x32x16<DT>(kfrag(kn, 0, ds), qf[ds], n0);
        n1 = mfma32x32x16<DT>(kfrag(kn, 1, ds), qf[ds], n1);
        // 4 of the 32 scores per step: registers 2*ds, 2*ds+1 of both blocks
        const int r = 2 * ds;
        const float p00 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], c, -moff));
        const float p01 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r + 1], c, -moff));
        const float p10 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], c, -moff));
        const float p11 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r + 1], c, -moff));
        psum += (p00 + p01) + (p10 + p11);
        // registers 0..7 -> keys 0..15 of the block (P k-step 2*blk), 8..15 -> keys 16..31
        pf[r >> 3][(r & 7) >> 1] = pack2<DT>(p00, p01);
        pf[2 + (r >> 3)][(r & 7) >> 1] = pack2<DT>(p10, p11);
      }
      // machine-scheduler pattern for phase A: each MFMA followed by one K fragment read and a
      // share of the softmax VALU work
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // first two K fragment reads
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (i < 14) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // next K fragment read
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
      }
      __builtin_amdgcn_sched_barrier(0);
      l_run += psum;

      // phase B: O^T += V^T(t) . P^T(t), interleaved with the row max of S(t+1); the next d
      // block's V^T fragments are read while the current block's MFMAs run
      u32x4 vf[2][4];
      vread(vf[0], vq[0] + vt);
      float mn = -INFINITY;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int cb = db & 1, nb = cb ^ 1;
        lgkm_wait0(vf[cb]);
        if (db + 1 < 4) vread(vf[nb], vq[db + 1] + vt);
#pragma unroll
        for (int js = 0; js < 4; ++js) o[db] = mfma32x32x16<DT>(vf[cb][js], pf[js], o[db]);
#pragma unroll
        for (int r = 4 * db; r < 4 * db + 4; ++r) mn = vmax3(mn, n0[r], n1[r]);
        __builtin_amdgcn_sched_barrier(0);
      }
      s0 = n0;
      s1 = n1;
      mx = mn;
    }
  }

  // ---- epilogue: O[qi][h][d] = O^T[d][qi] / l
  const float l_tot = half_sum(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (qi < a.S_q) {
    uint16_t *O = (uint16_t *)a.O;
    const size_t obase = (((size_t)b * a.S_q + qi) * a.H + h) * kD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + 8 * rq + 4 * g;
        const u32x2 v{pack2<DT>(o[db][4 * rq + 0] * inv, o[db][4 * rq + 1] * inv),
                      pack2<DT>(o[db][4 * rq + 2] * inv, o[db][4 * rq + 3] * inv)};
        *(u32x2 *)(O + obase + d) = v;
      }
  }
}

// ---------------------------------------------------------------------------------------------
// Wide-query variant: 64 queries per wavefront (two 32-query blocks), 256 per workgroup, one
// wavefront per SIMD with the whole register file. Every K fragment read from LDS feeds the S MFMAs
// of both query blocks and every V^T fragment the P.V MFMAs of both: half the LDS reads per MFMA of
// the 32-query kernel above, and registers to read fragments further ahead. Same data layout,
// permutations, lazy rescale and pipeline; the softmax state is kept per query block.
constexpr int kBQW = 256;

template <int DT, bool CAUSAL>
__device__ __forceinline__ void attn_fwd_wide(const mtk_attn_kargs &a) {
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTile];  // K slots 0, 1 then V slots 0, 1

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, col = lane & 31;

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = id / a.q_blocks;
  int qb_id = id - bh * a.q_blocks;
  if (CAUSAL) qb_id = a.q_blocks - 1 - qb_id;  // heaviest query blocks first
  const int b = bh / a.H, h = bh - b * a.H;
  const int q0 = qb_id * kBQW;
  const uint32_t rs = (uint32_t)a.H * kD * 2;
  const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * kD * 2);
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H + h) * kD * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const int diag = a.S_kv - a.S_q;

  // this lane's two queries (one per query block) as B operands of S^T = K . Q^T
  int qi[2];
  u32x4 qf[2][8];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    qi[qb] = q0 + wave * 64 + qb * 32 + col;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
      qf[qb][ds] =
          buf_load16(rq, qi[qb] < a.S_q ? qbase + (uint32_t)qi[qb] * rs + (uint32_t)(16 * ds + 8 * g) * 2u : kOOB);
  }

  int kv_end = a.S_kv;
  if (CAUSAL) kv_end = min(a.S_kv, q0 + kBQW + diag);
  const int n_tiles = kv_end > 0 ? (kv_end + kBKV - 1) / kBKV : 0;

  int srow[4];
  uint32_t kcol[4], vcol[4], klane[4], vlane[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    srow[i] = (wave * 4 + i) * 4 + (lane >> 4);
    const int pc = lane & 15;
    kcol[i] = 16u * (uint32_t)(pc ^ (srow[i] & 15));
    vcol[i] = 16u * (uint32_t)(pc ^ (4 * (srow[i] & 3)));
    klane[i] = (uint32_t)srow[i] * rs + kcol[i];
    vlane[i] = (uint32_t)srow[i] * rs + vcol[i];
  }
  // A tile inside S_kv goes out with its base as the uniform scalar offset (no per-row work); the
  // tile crossing S_kv is loaded row-checked, rows past S_kv reading zero.
  auto issue = [&](const rsrc_t &r, char *dst, const uint32_t (&lane_off)[4], const uint32_t (&col)[4], int t) {
    const int key0 = t * kBKV;
    if (key0 + kBKV <= a.S_kv) {
      const uint32_t tb = kvbase + (uint32_t)key0 * rs;
#pragma unroll
      for (int i = 0; i < 4; ++i) lds_direct16_s(r, dst + i * 1024, lane_off[i], tb);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = key0 + srow[i];
        lds_direct16(r, dst + i * 1024, key < a.S_kv ? kvbase + (uint32_t)key * rs + col[i] : kOOB);
      }
    }
  };
  auto issue_k = [&](int slot, int t) { issue(rk, smem + slot * kTile + wave * 4096, klane, kcol, t); };
  auto issue_v = [&](int slot, int t) { issue(rv, smem + (2 + slot) * kTile + wave * 4096, vlane, vcol, t); };

  // Fragment reads. Per-lane LDS offsets are computed once; per tile only the slot base is added
  // (K: one offset per k-step, key block 1 at +8192; V^T: one per d block, key step js and half e
  // at +4096 js + 1024 e, folded into the instructions' offset fields).
  const int krow = swap_bits_2_3(col);
  uint32_t kq[8];
#pragma unroll
  for (int ds = 0; ds < 8; ++ds) kq[ds] = k_off(krow, 2 * ds + g);
  // V^T fragment for d block db, key step js (16 keys): lane (h = lane / 16, s = lane % 16) gets
  // d = 32 db + lane % 32 at keys 16 js + 8 (lane / 32) + 0..7 (two transposed reads, rows
  // 16 js + 8 (h / 2) + 4 e + s / 4); the row swizzle depends only on s / 4.
  const int vs = lane & 15, vh = lane >> 4;
  uint32_t vq[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const int d = 32 * db + 16 * (vh & 1) + 4 * (vs & 3);
    const int row = 8 * (vh >> 1) + (vs >> 2);
    vq[db] = lds_addr(smem) + (uint32_t)(row * 256 + 16 * ((d >> 3) ^ (4 * (row & 3))) + 2 * (d & 7));
  }
  auto kfrag = [&](const uint32_t (&kb)[8], int blk, int ds) -> u32x4 {
    return *(const u32x4 *)(smem + kb[ds] + blk * 8192);
  };
  auto kbase = [&](uint32_t (&kb)[8], int slot) {
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) kb[ds] = kq[ds] + (uint32_t)(slot * kTile);
  };
  auto vread = [&](u32x4 (&dst)[4], uint32_t vb) {
    static_for<0, 4>([&](auto jc) {
      constexpr int JS = decltype(jc)::value;
      const u32x2 w0 = ds_read_tr16_at<4096 * JS>(vb);
      const u32x2 w1 = ds_read_tr16_at<4096 * JS + 1024>(vb);
      dst[JS] = u32x4{w0.x, w0.y, w1.x, w1.y};
    });
  };

  float m_off[2] = {-INFINITY, -INFINITY};  // exponent offset per query block (log2 domain)
  float l_run[2] = {0.0f, 0.0f};            // this lane's half of the running row sums
  f32x16 o[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int i = 0; i < 4; ++i) o[qb][i] = f32x16{};
  const float c = a.scale_log2;
  const int wave_q_min = q0 + wave * 64;

  if (n_tiles > 0) {
    f32x16 s[2][2];  // [key block][query block]: S^T of the tile being softmaxed
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) s[kb][qb] = f32x16{};
    issue_k(0, 0);
    wait_vmem();
    __syncthreads();
    if (n_tiles > 1) issue_k(1, 1);
    issue_v(0, 0);
    uint32_t kb0[8];
    kbase(kb0, 0);
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const u32x4 kf = kfrag(kb0, kb, ds);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) s[kb][qb] = mfma32x32x16<DT>(kf, qf[qb][ds], s[kb][qb]);
      }
    float mx[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      mx[qb] = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx[qb] = vmax3(mx[qb], s[0][qb][r], s[1][qb][r]);
    }

    for (int t = 0; t < n_tiles; ++t) {
      wait_vmem();
      __syncthreads();  // K(t+1) and V(t) are in LDS; K slot t&1 and V slot (t+1)&1 are free
      if (t + 2 < n_tiles) issue_k(t & 1, t + 2);
      if (t + 1 < n_tiles) issue_v((t + 1) & 1, t + 1);
      uint32_t kn[8];
      kbase(kn, (t + 1) & 1);
      const uint32_t vt = (uint32_t)((2 + (t & 1)) * kTile);
      // K(t+1) fragments of the first two k-steps: read now, consumed after the softmax
      // bookkeeping below; later k-steps are read two k-steps ahead inside phase A
      u32x4 kf[8][2];
#pragma unroll
      for (int ds = 0; ds < 2; ++ds)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) kf[ds][kb] = kfrag(kn, kb, ds);

      const int j0 = t * kBKV;
      if ((j0 + kBKV > a.S_kv) || (CAUSAL && j0 + kBKV - 1 > wave_q_min + diag)) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kr0 = (r < 8) ? (8 * g + r) : (16 + 8 * g + (r - 8));
            const int key0 = j0 + kr0, key1 = j0 + 32 + kr0;
            s[0][qb][r] = (key0 < a.S_kv && (!CAUSAL || key0 <= qi[qb] + diag)) ? s[0][qb][r] : -INFINITY;
            s[1][qb][r] = (key1 < a.S_kv && (!CAUSAL || key1 <= qi[qb] + diag)) ? s[1][qb][r] : -INFINITY;
          }
          mx[qb] = -INFINITY;
#pragma unroll
          for (int r = 0; r < 16; ++r) mx[qb] = vmax3(mx[qb], s[0][qb][r], s[1][qb][r]);
        }
      }
      float moff[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float m = half_max(mx[qb]);
        const float m_tile = m * c;
        float alpha = 1.0f;
        if (m_tile > m_off[qb] + kRescaleSlack) {
          alpha = __builtin_amdgcn_exp2f(m_off[qb] - m_tile);
          m_off[qb] = m_tile;
        }
        moff[qb] = m_off[qb] == -INFINITY ? 0.0f : m_off[qb];
        l_run[qb] *= alpha;
        if (__any(alpha != 1.0f)) {
#pragma unroll
          for (int i = 0; i < 4; ++i) o[qb][i] *= alpha;
        }
      }

      // phase A: S(t+1) MFMAs (each K fragment feeds both query blocks) interleaved with the
      // exponentials / sums / packing of tile t
      f32x16 n[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) n[kb][qb] = f32x16{};
      u32x4 pf[2][4];
      float psum[2] = {0.0f, 0.0f};
      u32x4 vf[2][4];
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) {
        if (ds + 2 < 8) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) kf[ds + 2][kb] = kfrag(kn, kb, ds + 2);
        } else if (ds == 7) {
          // the first d block's V^T fragments for phase B (V(t) is in LDS since the barrier)
          vread(vf[0], vq[0] + vt);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) n[kb][qb] = mfma32x32x16<DT>(kf[ds][kb], qf[qb][ds], n[kb][qb]);
        const int r = 2 * ds;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float p00 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[0][qb][r], c, -moff[qb]));
          const float p01 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[0][qb][r + 1], c, -moff[qb]));
          const float p10 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[1][qb][r], c, -moff[qb]));
          const float p11 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[1][qb][r + 1], c, -moff[qb]));
          psum[qb] += (p00 + p01) + (p10 + p11);
          pf[qb][r >> 3][(r & 7) >> 1] = pack2<DT>(p00, p01);
          pf[qb][2 + (r >> 3)][(r & 7) >> 1] = pack2<DT>(p10, p11);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      l_run[0] += psum[0];
      l_run[1] += psum[1];

      // phase B: O^T += V^T(t) . P^T(t) for both query blocks, interleaved with the row maxima of
      // S(t+1); the next d block's V^T fragments are read while the current block's MFMAs run
      float mn[2] = {-INFINITY, -INFINITY};
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int cb = db & 1, nb = cb ^ 1;
        lgkm_wait0(vf[cb]);
        if (db + 1 < 4) vread(vf[nb], vq[db + 1] + vt);
#pragma unroll
        for (int js = 0; js < 4; ++js)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) o[qb][db] = mfma32x32x16<DT>(vf[cb][js], pf[qb][js], o[qb][db]);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int r = 4 * db; r < 4 * db + 4; ++r) mn[qb] = vmax3(mn[qb], n[0][qb][r], n[1][qb][r]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) s[kb][qb] = n[kb][qb];
      mx[0] = mn[0];
      mx[1] = mn[1];
    }
  }

  // ---- epilogue: O[qi][h][d] = O^T[d][qi] / l, per query block
  uint16_t *O = (uint16_t *)a.O;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float l_tot = half_sum(l_run[qb]);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (qi[qb] < a.S_q) {
      const size_t obase = (((size_t)b * a.S_q + qi[qb]) * a.H + h) * kD;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int d = db * 32 + 8 * rq + 4 * g;
          const u32x2 v{pack2<DT>(o[qb][db][4 * rq + 0] * inv, o[qb][db][4 * rq + 1] * inv),
                        pack2<DT>(o[qb][db][4 * rq + 2] * inv, o[qb][db][4 * rq + 3] * inv)};
          *(u32x2 *)(O + obase + d) = v;
        }
    }
  }
}

}  // namespace mtk

using namespace mtk;

#define ATTN_KERNEL(NAME, DT, CAUSAL)                                                                  \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))        \
  NAME(const mtk_attn_kargs a) {                                                                       \
    attn_fwd<DT, CAUSAL>(a);                                                                           \
  }

ATTN_KERNEL(mtk_attn_fwd_f16, DT_F16, false)
ATTN_KERNEL(mtk_attn_fwd_bf16, DT_BF16, false)
ATTN_KERNEL(mtk_attn_fwd_f16_causal, DT_F16, true)
ATTN_KERNEL(mtk_attn_fwd_bf16_causal, DT_BF16, true)

#define ATTN_WIDE_KERNEL(NAME, DT, CAUSAL)                                                             \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))        \
  NAME(const mtk_attn_kargs a) {                                                                       \
    attn_fwd_wide<DT, CAUSAL>(a);                                                                      \
  }

ATTN_WIDE_KERNEL(mtk_attn_fwd_w_f16, DT_F16, false)
ATTN_WIDE_KERNEL(mtk_attn_fwd_w_bf16, DT_BF16, false)
ATTN_WIDE_KERNEL(mtk_attn_fwd_w_f16_causal, DT_F16, true)
ATTN_WIDE_KERNEL(mtk_attn_fwd_w_bf16_causal, DT_BF16, true)
