// Flash-attention forward for gfx950, head dimension 128: the 128-query kernel (attention.hpp,
// padded head dimension 128) and the ping-pong kernel below, compiled for D = 128 and D = 64
// exactly. Other head dimensions are instantiated in attention_hd.hip.
//
// Two kernels share the arithmetic at D = 128 (their outputs are equal bit for bit): attn_fwd, 4
// wavefronts x 32 queries with the MFMA and softmax work of consecutive tiles interleaved in each
// wavefront, two workgroups per CU; and attn_fwd_pp, 8 wavefronts x 32 queries in two groups that
// alternate whole MFMA blocks and softmax blocks one block apart, so the matrix cores of a SIMD
// serve one group while its VALU serves the other.
#include "attention.hpp"

namespace mtk {


// ---------------------------------------------------------------------------------------------
// Ping-pong variant: 8 wavefronts (two per SIMD) per workgroup, 256 queries, 32 per wavefront, one
// workgroup per CU; the K/V tiles in LDS serve all 256 queries. Each wavefront alternates an MFMA
// block (P(t-1).V(t-1) and S(t) = K(t).Q^T: 32 MFMAs and their fragment reads, no VALU) with a VALU
// block (mask, row max, lazy rescale, exponentials, sums, packing of tile t). The two groups of four
// wavefronts (queries 0-127 and 128-255 of the block) run one block apart, separated by workgroup
// barriers, so on every SIMD one wavefront is in its MFMA block while the other is in its VALU
// block. Slot i of the schedule (between barriers i-1 and i) is, for group g and j = i - g: MFMA
// block j/2 for even j, VALU block (j-1)/2 for odd j, nothing for j < 0 or VALU block n_tiles.
// K(k+2) and V(k+1) are loaded during slots 2k+2 and 2k+3 (their LDS slots were last read in slot
// 2k+1) and waited for before barrier 2k+3. Same arithmetic as attn_fwd (attention.hpp) at D = 128.
constexpr int kBQP = 256;

// DP: the head dimension (128, or 64: the same schedule with half the k-steps and d blocks, rows of
// 128 bytes in LDS with the 128-query kernel's swizzles for that width).
template <int DT, bool CAUSAL, int DP = 128>
__device__ __forceinline__ void attn_fwd_pp(const mtk_attn_kargs &a) {
  using L = AttnLayout<DP>;
  static_assert(DP == 128 || DP == 64, "ping-pong head dimension");
  constexpr int kD = DP, kTile = L::kTile, kRowB = L::kRowB, kKs = L::kKs, kDb = L::kDb;
  constexpr int kNiW = kTile / 1024 / 8;  // staging instructions per wavefront and tile
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTile];  // K slots 0, 1 then V slots 0, 1

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..7
  const int grp = wave >> 2;                                  // 0: queries 0-127, 1: 128-255
  const int g = lane >> 5, col = lane & 31;

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  int bh = id / a.q_blocks;
  int qb = id - bh * a.q_blocks;
  if (CAUSAL) {  // heaviest (last) query blocks first
    causal_order(id, a.q_blocks, a.B * a.H, bh, qb);
    qb = a.q_blocks - 1 - qb;
  }
  const int b = bh / a.H, h = bh - b * a.H;
  const int q0 = qb * kBQP;
  const uint32_t rs = (uint32_t)a.H * kD * 2;
  const uint32_t rkv = (uint32_t)a.H_kv * kD * 2;
  const int hk = h / (a.H / a.H_kv);
  const uint32_t qbase = (uint32_t)(((size_t)b * a.S_q * a.H + h) * kD * 2);
  const uint32_t kvbase = (uint32_t)(((size_t)b * a.S_kv * a.H_kv + hk) * kD * 2);
  const rsrc_t rq = make_rsrc(a.Q, a.q_bytes);
  const rsrc_t rk = make_rsrc(a.K, a.kv_bytes);
  const rsrc_t rv = make_rsrc(a.V, a.kv_bytes);
  const int diag = a.S_kv - a.S_q;

  const int wave_q_min = q0 + wave * 32;
  const int qi = wave_q_min + col;
  u32x4 qf[kKs];
#pragma unroll
  for (int ds = 0; ds < kKs; ++ds)
    qf[ds] = buf_load16(rq, qi < a.S_q ? qbase + (uint32_t)qi * rs + (uint32_t)(16 * ds + 8 * g) * 2u : kOOB);

  int kv_end = a.S_kv;
  if (CAUSAL) kv_end = min(a.S_kv, q0 + kBQP + diag);
  const int n_tiles = kv_end > 0 ? (kv_end + kBKV - 1) / kBKV : 0;

  // direct-to-LDS staging: each wavefront fills an eighth of a tile (D = 128: two instructions of
  // 4 rows; D = 64: one of 8 rows). LDS chunk pc of row r holds global chunk pc ^ kswz(r) (K) or
  // pc ^ vswz(r) (V) (D = 128: r & 15 and 4 (r & 3)). Only the in-range offsets are kept in
  // registers; the row-checked path of the tile crossing S_kv recomputes them.
  auto stage_row = [&](int i) { return (wave * kNiW + i) * L::kRpi + lane / L::kCpr; };
  auto stage_col = [&](int i, bool is_k) {
    const int r = stage_row(i), pc = lane % L::kCpr;
    return 16u * (uint32_t)(is_k ? (pc ^ L::kswz(r)) : (pc ^ L::vswz(r)));
  };
  uint32_t klane[kNiW], vlane[kNiW];
#pragma unroll
  for (int i = 0; i < kNiW; ++i) {
    klane[i] = (uint32_t)stage_row(i) * rkv + stage_col(i, true);
    vlane[i] = (uint32_t)stage_row(i) * rkv + stage_col(i, false);
  }
  auto issue = [&](const rsrc_t &r, char *dst, const uint32_t (&lane_off)[kNiW], bool is_k, int t) {
    const int key0 = t * kBKV;
    if (key0 + kBKV <= a.S_kv) {
      const uint32_t tb = kvbase + (uint32_t)key0 * rkv;
#pragma unroll
      for (int i = 0; i < kNiW; ++i) lds_direct16_s(r, dst + i * 1024, lane_off[i], tb);
    } else {
#pragma unroll
      for (int i = 0; i < kNiW; ++i) {
        const int key = key0 + stage_row(i);
        lds_direct16(r, dst + i * 1024, key < a.S_kv ? kvbase + (uint32_t)key * rkv + stage_col(i, is_k) : kOOB);
      }
    }
  };
  auto issue_k = [&](int t) { issue(rk, smem + (t & 1) * kTile + wave * (kTile / 8), klane, true, t); };
  auto issue_v = [&](int t) { issue(rv, smem + (2 + (t & 1)) * kTile + wave * (kTile / 8), vlane, false, t); };

  // Fragment addresses from one base per lane: K k-step ds is at chunk (2 ds + g) ^ (krow & 15) =
  // 2 (ds ^ zh) + ((g ^ krow) & 1) with zh = (krow & 15) >> 1; V^T d block db at chunk
  // (4 db + x) ^ 4 y = 4 (db ^ y) + x (x, y: the V^T read's chunk and row parts). Fewer live registers
  // than a table.
  // (D = 64: the same chunks from the 128-byte rows' swizzles, k-step ds and d block db folded into
  // the per-lane offset.)
  const int krow = swap_bits_2_3(col);
  const uint32_t kbase0 = (uint32_t)(krow * 256 + 16 * ((g ^ krow) & 1));
  const int kzh = (krow & 15) >> 1;
  auto kq = [&](int ds) {
    if constexpr (DP == 128)
      return kbase0 + 32u * (uint32_t)(ds ^ kzh);
    else
      return (uint32_t)(krow * kRowB + (((2 * ds + g) ^ L::kswz(krow)) << 4));
  };
  const int vs = lane & 15, vh = lane >> 4;
  const int vrow = 8 * (vh >> 1) + (vs >> 2), vy = vrow & 3;
  const uint32_t vbase0 = lds_addr(smem) + (uint32_t)(vrow * 256 + 16 * (2 * (vh & 1) + ((vs & 3) >> 1)) + 2 * (4 * (vs & 3) & 7));
  auto vq = [&](int db) {
    if constexpr (DP == 128) {
      return vbase0 + 64u * (uint32_t)(db ^ vy);
    } else {
      const int d = 32 * db + 16 * (vh & 1) + 4 * (vs & 3);
      return lds_addr(smem) + (uint32_t)(vrow * kRowB + 16 * ((d >> 3) ^ L::vswz(vrow)) + 2 * (d & 7));
    }
  };

  float m_off = -INFINITY, l_run = 0.0f;
  f32x16 o[kDb];
#pragma unroll
  for (int i = 0; i < kDb; ++i) o[i] = f32x16{};
  f32x16 s0 = f32x16{}, s1 = f32x16{};  // S^T of the latest tile
  u32x4 pf[4];                          // P of the latest softmaxed tile
#pragma unroll
  for (int i = 0; i < 4; ++i) pf[i] = u32x4{};
  const float c = a.scale_log2;

  // MFMA block k: O += V(k-1)^T . P(k-1)^T (PV, k >= 1) and S(k) = K(k) . Q^T (SK, k < n_tiles),
  // as a compile-time schedule of steps: per d block db, two S steps (k-steps 2db, 2db+1: two
  // MFMAs on the K fragments of both key blocks) then four P.V steps (key steps js: one MFMA on one
  // V^T fragment). Every step's fragments take exactly two LDS read instructions (inline asm:
  // ordinary LDS reads would wait for the K/V loads of later tiles in flight), issued kLook steps
  // ahead into a ring of registers; before its MFMAs a step waits until at most 2 * (steps issued
  // after it) reads are outstanding (LDS reads complete in order), its registers tied to the wait.
  constexpr int kLook = 6, kRing = kLook + 2;
  auto mfma_block = [&](int k, auto pv_c, auto sk_c) {
    constexpr bool PV = decltype(pv_c)::value, SK = decltype(sk_c)::value;
    constexpr int kPerDb = (SK ? 2 : 0) + (PV ? 4 : 0), kSteps = kDb * kPerDb;
    const uint32_t vt = (uint32_t)((2 + ((k - 1) & 1)) * kTile);
    const uint32_t kslot = lds_addr(smem) + (uint32_t)((k & 1) * kTile);
    u32x4 ring[kRing][2];
    auto issue_reads = [&](auto sc) {
      constexpr int S = decltype(sc)::value, DB = S / kPerDb, W = S % kPerDb;
      constexpr bool IS_S = SK && W < 2;
      if constexpr (IS_S) {
        const uint32_t ka = kslot + kq(2 * DB + W);
        ring[S % kRing][0] = ds_read_b128_at<0>(ka);
        ring[S % kRing][1] = ds_read_b128_at<32 * kRowB>(ka);  // key block 1: 32 rows on
      } else {
        constexpr int JS = W - (SK ? 2 : 0);
        const uint32_t vb = vq(DB) + vt;
        const u32x2 w0 = ds_read_tr16_at<16 * kRowB * JS>(vb);
        const u32x2 w1 = ds_read_tr16_at<16 * kRowB * JS + 4 * kRowB>(vb);
        ring[S % kRing][0] = u32x4{w0.x, w0.y, w1.x, w1.y};
      }
    };
    if constexpr (SK) {
      s0 = f32x16{};  // S(k) accumulates in place: VALU block k-1 is done with S(k-1)
      s1 = f32x16{};
    }
    static_for<0, kLook>([&](auto sc) {
      if constexpr (decltype(sc)::value < kSteps) issue_reads(sc);
    });
    static_for<0, kSteps>([&](auto sc) {
      constexpr int S = decltype(sc)::value, DB = S / kPerDb, W = S % kPerDb;
      constexpr bool IS_S = SK && W < 2;
      if constexpr (S + kLook < kSteps) issue_reads(std::integral_constant<int, S + kLook>{});
      constexpr int kYounger = 2 * ((S + kLook < kSteps) ? kLook : (kSteps - 1 - S));
      asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(ring[S % kRing][0]), "+v"(ring[S % kRing][1]) : "i"(kYounger));
      if constexpr (IS_S) {
        s0 = mfma32x32x16<DT>(ring[S % kRing][0], qf[2 * DB + W], s0);
        s1 = mfma32x32x16<DT>(ring[S % kRing][1], qf[2 * DB + W], s1);
      } else {
        constexpr int JS = W - (SK ? 2 : 0);
        o[DB] = mfma32x32x16<DT>(ring[S % kRing][0], pf[JS], o[DB]);
      }
    });
  };
  // VALU block k: softmax bookkeeping and P(k)
  auto valu_block = [&](int k) {
    const int j0 = k * kBKV;
    if ((j0 + kBKV > a.S_kv) || (CAUSAL && j0 + kBKV - 1 > wave_q_min + diag)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr0 = (r < 8) ? (8 * g + r) : (16 + 8 * g + (r - 8));
        const int key0 = j0 + kr0, key1 = j0 + 32 + kr0;
        s0[r] = (key0 < a.S_kv && (!CAUSAL || key0 <= qi + diag)) ? s0[r] : -INFINITY;
        s1[r] = (key1 < a.S_kv && (!CAUSAL || key1 <= qi + diag)) ? s1[r] : -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = vmax3(mx, s0[r], s1[r]);
    mx = half_max(mx);
    const float m_tile = mx * c;
    float alpha = 1.0f;
    if (m_tile > m_off + kRescaleSlack) {
      alpha = __builtin_amdgcn_exp2f(m_off - m_tile);
      m_off = m_tile;
    }
    const float moff = m_off == -INFINITY ? 0.0f : m_off;
    l_run *= alpha;
    if (__any(alpha != 1.0f)) {
      // one accumulator block at a time: at most 16 values in flight through temporaries
#pragma unroll
      for (int i = 0; i < kDb; ++i) {
        o[i] *= alpha;
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    float psum = 0.0f;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
      const int r = 2 * ds;
      const float p00 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], c, -moff));
      const float p01 = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r + 1], c, -moff));
      const float p10 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], c, -moff));
      const float p11 = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r + 1], c, -moff));
      psum += (p00 + p01) + (p10 + p11);
      pf[r >> 3][(r & 7) >> 1] = pack2<DT>(p00, p01);
      pf[2 + (r >> 3)][(r & 7) >> 1] = pack2<DT>(p10, p11);
      __builtin_amdgcn_sched_barrier(0);  // few probabilities live at a time
    }
    l_run += psum;
  };

  if (n_tiles > 0) {
    issue_k(0);
    if (n_tiles > 1) issue_k(1);
    issue_v(0);
    wait_vmem();
    __syncthreads();
    const std::true_type T{};
    const std::false_type F{};
    // loads of slot 2k+2: K(k+2) and V(k+1); waited for before barrier 2k+3
    auto loads = [&](int k) {
      if (k + 2 < n_tiles) issue_k(k + 2);
      if (k + 1 < n_tiles) issue_v(k + 1);
    };
    // Both groups run 2 n_tiles + 1 barriers. Group 0: slot 2k = MFMA block k, slot 2k+1 = VALU
    // block k. Group 1: one slot later.
    if (grp == 0) {
      mfma_block(0, F, T);
      __syncthreads();  // 0
      for (int k = 0; k + 1 < n_tiles; ++k) {
        valu_block(k);
        if (k >= 1) wait_vmem();
        __syncthreads();  // 2k+1
        loads(k);
        mfma_block(k + 1, T, T);
        __syncthreads();  // 2k+2
      }
      valu_block(n_tiles - 1);
      if (n_tiles >= 2) wait_vmem();
      __syncthreads();  // 2N-1
      mfma_block(n_tiles, T, F);
      __syncthreads();  // 2N
    } else {
      __syncthreads();  // 0
      mfma_block(0, F, T);
      __syncthreads();  // 1
      for (int k = 0; k + 1 < n_tiles; ++k) {
        loads(k);
        valu_block(k);
        __syncthreads();  // 2k+2
        mfma_block(k + 1, T, T);
        wait_vmem();
        __syncthreads();  // 2k+3
      }
      valu_block(n_tiles - 1);
      __syncthreads();  // 2N
      mfma_block(n_tiles, T, F);
    }
  }

  const float l_tot = half_sum(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  store_lse(a, b, h, qi, g, m_off, l_tot);
  if (qi < a.S_q) {
    uint16_t *O = (uint16_t *)a.O;
    const size_t obase = (((size_t)b * a.S_q + qi) * a.H + h) * kD;
#pragma unroll
    for (int db = 0; db < kDb; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d = db * 32 + 8 * rq + 4 * g;
        const u32x2 v{pack2<DT>(o[db][4 * rq + 0] * inv, o[db][4 * rq + 1] * inv),
                      pack2<DT>(o[db][4 * rq + 2] * inv, o[db][4 * rq + 3] * inv)};
        *(u32x2 *)(O + obase + d) = v;
      }
  }
}

}  // namespace mtk

using namespace mtk;

MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_f16, DT_F16, false, 128, false, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_bf16, DT_BF16, false, 128, false, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_f16_causal, DT_F16, true, 128, false, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_bf16_causal, DT_BF16, true, 128, false, 2)

#define ATTN_PP_KERNEL(NAME, DT, CAUSAL, DP)                                                           \
  extern "C" __global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))        \
  NAME(const mtk_attn_kargs a) {                                                                       \
    attn_fwd_pp<DT, CAUSAL, DP>(a);                                                                    \
  }

ATTN_PP_KERNEL(mtk_attn_fwd_pp_f16, DT_F16, false, 128)
ATTN_PP_KERNEL(mtk_attn_fwd_pp_bf16, DT_BF16, false, 128)
ATTN_PP_KERNEL(mtk_attn_fwd_pp_f16_causal, DT_F16, true, 128)
ATTN_PP_KERNEL(mtk_attn_fwd_pp_bf16_causal, DT_BF16, true, 128)
ATTN_PP_KERNEL(mtk_attn_fwd_pp_d64_f16, DT_F16, false, 64)
ATTN_PP_KERNEL(mtk_attn_fwd_pp_d64_bf16, DT_BF16, false, 64)
ATTN_PP_KERNEL(mtk_attn_fwd_pp_d64_f16_causal, DT_F16, true, 64)
ATTN_PP_KERNEL(mtk_attn_fwd_pp_d64_bf16_causal, DT_BF16, true, 64)
