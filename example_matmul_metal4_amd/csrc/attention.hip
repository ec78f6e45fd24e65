// Flash-attention forward for gfx950 (head dim 128), fp16/bf16 in, fp32 softmax and accumulate.
//
// Replaces the reference's generated `attention` kernel (Sources/attention/attention.swift:133-380):
// O = softmax(Q K^T / sqrt(D)) V with base-2 online softmax (its dotScale = log2(e)/sqrt(D),
// attention.swift:24), per (batch, head), tensors laid out [B][S][H][D] (attention.swift:466-468
// with a batch dimension). Extensions: batch, causal mask (keys j <= i + S_kv - S_q), bf16.
//
// Work decomposition
//   * Workgroup = 4 wavefronts = 128 query rows of one (batch, head); each wave owns 32 queries.
//     K/V are streamed in tiles of 64 keys through two LDS stages (one barrier per tile).
//   * Scores are computed transposed, S^T = K . Q^T, on 32x32x16 MFMA: the accumulator column
//     (lane % 32) is the query, so each lane owns one query and the softmax row max / row sum are
//     in-register reductions plus one exchange with lane ^ 32.
//   * K rows are fed to the MFMA in a permuted order (MFMA row m reads key swap_bits_2_3(m)); with
//     that order accumulator register r of lane (i, g = lane/32) holds key 8g + r (r < 8) or
//     16 + 8g + (r - 8), which is exactly the B-operand layout of the P.V MFMA
//     (O^T = V^T . P^T). P therefore goes from the S accumulators to the next MFMA with only an
//     fp32 -> 16-bit conversion, never through LDS.
//   * V is transposed while staging to LDS (4x8 register transposes), so V^T fragments are
//     single 16-byte LDS reads. K rows (256 B) use a chunk ^ (row & 15) swizzle, V^T rows (128 B)
//     chunk ^ (row & 7) ^ ((row >> 3) & 7); both keep the fragment reads bank-conflict free.
//   * O is rescaled only when some lane's running max moved (wave-uniform branch).
//   * Global reads are raw buffer loads: rows past S (ragged tails) read zero, never fault.
//   * Causal: a workgroup stops at its last visible key tile; heavy query blocks are dispatched
//     first; query blocks of one (batch, head) are kept on one XCD for K/V reuse in L2.
#include "device.hpp"

namespace mtk {

constexpr int kD = 128;
constexpr int kBQ = 128;
constexpr int kBKV = 64;
constexpr int kStageBytes = 2 * kBKV * kD * 2;  // K tile + V^T tile

__device__ __forceinline__ int swap_bits_2_3(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

__device__ __forceinline__ uint32_t k_off(int row, int chunk) {  // 64 rows x 256 B
  return (uint32_t)(row * 256 + ((chunk ^ (row & 15)) << 4));
}
__device__ __forceinline__ uint32_t vt_off(int d, int chunk) {  // 128 rows x 128 B
  return (uint32_t)(kBKV * kD * 2 + d * 128 + ((chunk ^ (d & 7) ^ ((d >> 3) & 7)) << 4));
}

template <int DT>
__device__ __forceinline__ uint32_t half_of(const u32x4 &v, int e) {  // 16-bit element e of 8
  const uint32_t w = v[e >> 1];
  return (e & 1) ? (w >> 16) : (w & 0xffffu);
}

template <int DT, bool CAUSAL>
__device__ __forceinline__ void attn_fwd(const mtk_attn_kargs &a) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kStageBytes];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  // ---- staging: K as 4 chunks per thread, V as a 4-key x 8-dim block per thread
  const int kchunk = tid & 15;
  const int vjq = tid >> 4, vdb = tid & 15;
  u32x4 kr[4], vr[4];
  auto load_kv = [&](int t) {
    const int j0 = t * kBKV;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = j0 + (tid >> 4) + 16 * i;
      kr[i] = buf_load16(rk, key < a.S_kv ? kvbase + (uint32_t)key * rs + (uint32_t)kchunk * 16u : kOOB);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = j0 + 4 * vjq + i;
      vr[i] = buf_load16(rv, key < a.S_kv ? kvbase + (uint32_t)key * rs + (uint32_t)vdb * 16u : kOOB);
    }
  };
  auto store_kv = [&](int s) {
    char *st = smem + s * kStageBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) *(u32x4 *)(st + k_off((tid >> 4) + 16 * i, kchunk)) = kr[i];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = vdb * 8 + e;
      const uint32_t lo = half_of<DT>(vr[0], e) | (half_of<DT>(vr[1], e) << 16);
      const uint32_t hi = half_of<DT>(vr[2], e) | (half_of<DT>(vr[3], e) << 16);
      *(u32x2 *)(st + vt_off(d, vjq >> 1) + (vjq & 1) * 8) = u32x2{lo, hi};
    }
  };

  float m_run = -1e30f;  // running max of scaled logits (log2 domain)
  float l_run = 0.0f;    // this lane's half of the running row sum
  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};

  const int krow = swap_bits_2_3(col);
  const float c = a.scale_log2;
  const int wave_q_min = q0 + wave * 32;

  if (n_tiles > 0) {
    load_kv(0);
    store_kv(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int cur = t & 1;
    const bool more = t + 1 < n_tiles;
    if (more) load_kv(t + 1);
    const char *st = smem + cur * kStageBytes;

    // S^T for 64 keys: two 32-key blocks
    f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
      const int ch = 2 * ds + g;
      const u32x4 k0 = *(const u32x4 *)(st + k_off(krow, ch));
      const u32x4 k1 = *(const u32x4 *)(st + k_off(krow + 32, ch));
      s0 = mfma32x32x16<DT>(k0, qf[ds], s0);
      s1 = mfma32x32x16<DT>(k1, qf[ds], s1);
    }

    const int j0 = t * kBKV;
    const bool need_mask = (j0 + kBKV > a.S_kv) || (CAUSAL && j0 + kBKV - 1 > wave_q_min + diag);
    if (need_mask) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr0 = (r < 8) ? (8 * g + r) : (16 + 8 * g + (r - 8));
        const int key0 = j0 + kr0, key1 = j0 + 32 + kr0;
        const bool v0 = key0 < a.S_kv && (!CAUSAL || key0 <= qi + diag);
        const bool v1 = key1 < a.S_kv && (!CAUSAL || key1 <= qi + diag);
        s0[r] = v0 ? s0[r] : -INFINITY;
        s1[r] = v1 ? s1[r] : -INFINITY;
      }
    }

    // online softmax (base 2)
    float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx * c);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], c, -m_new));
      s1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], c, -m_new));
      psum += s0[r] + s1[r];
    }
    l_run = l_run * alpha + psum;
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] *= alpha;
    }

    // P^T as the B operand, 16 keys per MFMA k-step: js = 2 * block + half
    u32x4 pf[4];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      pf[hf] = u32x4{pack2<DT>(s0[8 * hf + 0], s0[8 * hf + 1]), pack2<DT>(s0[8 * hf + 2], s0[8 * hf + 3]),
                     pack2<DT>(s0[8 * hf + 4], s0[8 * hf + 5]), pack2<DT>(s0[8 * hf + 6], s0[8 * hf + 7])};
      pf[2 + hf] = u32x4{pack2<DT>(s1[8 * hf + 0], s1[8 * hf + 1]), pack2<DT>(s1[8 * hf + 2], s1[8 * hf + 3]),
                         pack2<DT>(s1[8 * hf + 4], s1[8 * hf + 5]), pack2<DT>(s1[8 * hf + 6], s1[8 * hf + 7])};
    }

    // O^T += V^T . P^T
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int vrow = db * 32 + col;
#pragma unroll
      for (int js = 0; js < 4; ++js) {
        const u32x4 vf = *(const u32x4 *)(st + vt_off(vrow, 2 * js + g));
        o[db] = mfma32x32x16<DT>(vf, pf[js], o[db]);
      }
    }

    if (more) store_kv(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O[qi][h][d] = O^T[d][qi] / l
  const float l_tot = l_run + __shfl_xor(l_run, 32);
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

}  // namespace mtk

using namespace mtk;

#define ATTN_KERNEL(NAME, DT, CAUSAL)                                                                  \
  extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))        \
  NAME(const mtk_attn_kargs a) {                                                                       \
    attn_fwd<DT, CAUSAL>(a);                                                                           \
  }

ATTN_KERNEL(mtk_attn_fwd_f16, DT_F16, false)
ATTN_KERNEL(mtk_attn_fwd_f16_causal, DT_F16, true)
ATTN_KERNEL(mtk_attn_fwd_bf16, DT_BF16, false)
ATTN_KERNEL(mtk_attn_fwd_bf16_causal, DT_BF16, true)
