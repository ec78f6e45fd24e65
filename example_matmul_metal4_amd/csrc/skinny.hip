// Skinny (decode-shaped) GEMM for gfx950: C[M <= 16][N] = A[M][K] . B[N][K]^T + bias, fp32 accumulate.
//
// The reference's generated GEMM handles M < BM only through its edge-tile path, which ignores
// split-K (Sources/matmul/matmul.swift:280-295). This kernel is the HBM-bound counterpart: B is
// streamed from HBM exactly once, straight into MFMA operands.
//
// Work decomposition
//   * Workgroup = split_k wavefronts; wavefront w owns K partition w for every column group the
//     workgroup processes. The grid is persistent (at most one workgroup per CU) and balanced:
//     workgroup b owns the contiguous columns [b * per, b * per + per), per = ceil(N / grid),
//     walked in groups of 16.
//   * 16x16x32 MFMA, lane (r = lane % 16, q = lane / 16). K step s of a partition covers 32
//     elements of K; lane (r, q) supplies elements 8q .. 8q+7 of that step, of A row r and of
//     B row (group column r), i.e. chunk 4s + q (8 elements) of the partition.
//   * Resident kernel (partitions of up to kSkinnyResident K steps): loads read whole cache lines.
//     Load instruction s reads row s of the group (or of A), 16 bytes per lane: chunk `lane` of
//     the partition, 1 KB contiguous per instruction. (Reading operand fragments directly, 64
//     bytes of each of 16 rows per instruction, streams B at ~4.4 TB/s against ~6.3 TB/s here.)
//     The wavefront transposes the 16 rows x 64 chunks through its own LDS region into fragment
//     layout: row s chunk c is parked in slot c ^ s, so both the parking writes and the fragment
//     reads of 16 lanes touch 16 distinct 16-byte bank groups. A is transposed once and kept in
//     registers; B loads are non-temporal (streamed once), the next group's issued before the
//     current group's MFMAs (two register buffers).
//   * Per group the partitions' fp32 16x16 results are parked in an LDS slot; every kSkinnySlots
//     groups (and after the last) the workgroup sums partitions 0, 1, ... in order, adds the bias
//     and stores: one barrier pair per kSkinnySlots groups instead of one barrier per group. With
//     at most kSkinnyFew groups per workgroup (and split-K >= 4) each group keeps its own slot and
//     the workgroup reduces once, at the end (mtk_skinny_few_*).
//   * The long kernel (longer partitions) loads fragments directly and reloads A per pass of
//     kSkinnyResident steps (L2-resident: A is M x K).
//   * Raw buffer loads: rows m >= M, columns n >= N and K past the partition read zero.
//   The arithmetic of every output is the same in both kernels and for any grid: per partition a
//   chain of MFMAs over its K steps in order from zero, partition sums added in partition order,
//   the bias last.
#include "device.hpp"

namespace mtk {

constexpr int kSkinnyResident = 16;  // K steps (x 32) a partition may keep resident: 512 K
constexpr int kSkinnySlots = 2;      // column groups parked in LDS between reductions
constexpr int kSkinnyFew = 4;        // groups per workgroup the one-reduction kernel handles

template <int DT, int KS>
struct SkinnyWave {
  // KS = K steps per pass over the partition (<= kSkinnyResident)
  u32x4 a[KS];
  uint32_t arow, k0, k_end;

  __device__ void load_a(rsrc_t ra, int kbase, int lane) {
    const int q = lane >> 4;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = kbase + 32 * s + 8 * q;
      a[s] = buf_load16(ra, k < (int)k_end ? arow + (uint32_t)k * 2u : kOOB);
    }
  }
  __device__ void load_b(rsrc_t rb, u32x4 (&b)[KS], int group, int N, int ldb, int kbase, int lane) const {
    const int n = group * 16 + (lane & 15), q = lane >> 4;
    const uint32_t brow = n < N ? (uint32_t)n * (uint32_t)ldb * 2u : kOOB;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = kbase + 32 * s + 8 * q;
      b[s] = buf_load16(rb, (k < (int)k_end && brow != kOOB) ? brow + (uint32_t)k * 2u : kOOB);
    }
  }
  __device__ f32x4 mma(const u32x4 (&b)[KS], f32x4 acc) const {
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma16x16x32<DT>(a[s], b[s], acc);
    return acc;
  }
};

// Workgroup barrier over LDS data only: this wavefront's LDS operations have completed
// (lgkmcnt(0)); its global loads stay in flight (__syncthreads' fence would wait for them, which
// drains the B stream at every reduction).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

// Partition results of one group are in LDS; after the barrier the workgroup (64 * split_k
// threads) sums them for the 256 outputs of the group.
template <int DT>
__device__ __forceinline__ void skinny_reduce_store(const mtk_skinny_args &p, float (*red)[256], int group, int tid) {
  for (int e = tid; e < 256; e += 64 * p.split_k) {
    const int m = e >> 4, c = e & 15;
    const int n = group * 16 + c;
    float s = red[0][e];
    for (int w = 1; w < p.split_k; ++w) s += red[w][e];
    if (m < p.M && n < p.N) {
      if (p.has_bias) s += from_bits<DT>(((const uint16_t *)p.bias)[n]);
      ((uint16_t *)p.C)[(size_t)m * p.ldc + n] = to_bits<DT>(s);
    }
  }
}

// Resident partitions (K per partition <= 32 * kSkinnyResident): whole-line loads transposed
// through LDS, balanced contiguous columns. R = kSkinnySlots: reductions every R groups, bias
// values parked in LDS. R = kSkinnyFew (workgroups of at most R groups): every group parked in
// its own LDS slot (160 KB with the transpose regions), one reduction at the end, each thread's
// bias values for it held in registers.
template <int DT, int R>
__device__ __forceinline__ void skinny_gemm_resident(const mtk_skinny_args &p) {
  constexpr int KS = kSkinnyResident;
  constexpr bool kFew = R == kSkinnyFew;
  static_assert(R == kSkinnySlots || kFew, "two slots, or one per group");
  // non-temporal B loads: each element of B is read once
  constexpr int kStreamPolicy = 2;
  __shared__ __attribute__((aligned(16))) float red[R][8][256];
  __shared__ __attribute__((aligned(16))) u32x4 tr[8][KS][64];  // per wavefront: 16 rows x 64 chunks
  // Bias values go through registers (kBiasRegs per thread, loads issued unconditionally:
  // out-of-range offsets read zeros). With reductions every two groups they are loaded right after
  // the first B group and parked in LDS once the wait for that group covers them: a global bias
  // load in a reduction would be the youngest vector-memory operation, and waiting for it
  // (vmcnt(0)) would also wait for the next group's B loads in flight, while loading the bias
  // before the B stream delays the stream by a memory round trip. With one reduction (at the end,
  // when no B load is left in flight) thread t loads the values of the outputs it sums there
  // (t, t + 64 split_k, ...) just before its barrier.
  constexpr int kBiasRegs = kFew ? 4 : 8;  // kFew: 4 x 256 outputs over >= 256 threads (split-K >= 4)
  __shared__ uint16_t bias_s[kFew ? 1 : kBiasRegs * 512];

  const int tid = threadIdx.x;
  const int nthr = 64 * p.split_k;  // the plan launches one wavefront per K partition
  const int lane = tid & 63, w = tid >> 6;
  const int per = (p.N + (int)gridDim.x - 1) / (int)gridDim.x;
  const int c0 = (int)blockIdx.x * per, c1 = min(p.N, c0 + per);
  const int ng = c1 > c0 ? (c1 - c0 + 15) / 16 : 0;  // workgroup-uniform
  const rsrc_t ra = make_rsrc(p.A, p.a_bytes);
  const rsrc_t rb = make_rsrc(p.B, p.b_bytes);
  const int k0 = w * p.k_per_split;
  const int k_end = min(p.K, k0 + p.k_per_split);
  const int kl = k0 + 8 * lane;  // the chunk this lane loads of every row
  const bool k_ok = kl < k_end;
  const int r = lane & 15, q = lane >> 4;
  u32x4(&t)[KS][64] = tr[w];
  const bool bias_cached = kFew || per <= kBiasRegs * nthr;

  // Row r of A or B is addressed by the scalar offset r * ld * 2 on top of the lane's fixed chunk
  // offset (out of range past the partition); rows past the end read through a descriptor of size 0
  // (zeros, no memory access). One address VGPR serves every load.
  const uint32_t voff = k_ok ? (uint32_t)kl * 2u : kOOB;
  const rsrc_t rnull = make_rsrc(p.B, 0);
  auto load_b = [&](u32x4 (&b)[KS], int col) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int n = col + s;
      b[s] = __builtin_amdgcn_raw_buffer_load_b128(n < c1 ? rb : rnull, voff, n < c1 ? (uint32_t)n * (uint32_t)p.ldb * 2u : 0u,
                                                   kStreamPolicy);
    }
  };

  // A: row s (s < M) -> slot lane ^ s, fragments read back once. The first B group's loads go out
  // before the transpose waits for A, so the B stream starts at once.
  u32x4 a[KS], b0[KS], b1[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    a[s] = __builtin_amdgcn_raw_buffer_load_b128(s < p.M ? ra : rnull, voff, s < p.M ? (uint32_t)s * (uint32_t)p.lda * 2u : 0u, 0);
  load_b(b0, c0);
  const rsrc_t rbias = make_rsrc(p.bias, (uint32_t)p.N * 2u);
  // kFew: output i of the reduction (group i / 256, column i % 16); else column c0 + i
  auto load_bias = [&](uint32_t (&br)[kBiasRegs]) {
#pragma unroll
    for (int j = 0; j < kBiasRegs; ++j) {
      const int i = j * nthr + tid;
      const int col = kFew ? c0 + 16 * (i >> 8) + (i & 15) : c0 + i;
      br[j] = buf_load2(rbias, (p.has_bias && bias_cached && col < c1 && (kFew || i < c1 - c0)) ? (uint32_t)col * 2u : kOOB);
    }
  };
  uint32_t bias_r[kBiasRegs];
  if constexpr (!kFew) load_bias(bias_r);
  // keep the A transpose (which waits for A) after the first B group's and the bias's issue: the
  // scheduler would otherwise sink those loads below it and start the B stream a round trip late
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < KS; ++s) t[s][lane ^ s] = a[s];
#pragma unroll
  for (int s = 0; s < KS; ++s) a[s] = t[r][(4 * s + q) ^ r];
  // LDS operations of one wavefront execute in order: the parking writes of a group follow the
  // fragment reads of the previous one.
  auto mma = [&](const u32x4 (&b)[KS]) {
#pragma unroll
    for (int s = 0; s < KS; ++s) t[s][lane ^ s] = b[s];
    f32x4 acc{};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma16x16x32<DT>(a[s], t[r][(4 * s + q) ^ r], acc);
    return acc;
  };
  // 16x16 accumulator layout: lane (c = lane % 16, g = lane / 16), register i -> row 4g + i, col c.
  auto park = [&](int slot, f32x4 acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[slot][w][(4 * q + i) * 16 + r] = acc[i];
  };
  // groups g0 .. g0 + n - 1 are parked in slots 0 .. n - 1
  auto flush = [&](int g0, int n) {
    if constexpr (kFew) {
      // The one reduction (g0 = 0): output e = tid + j * nthr with its bias value in bias_r[j],
      // loaded here (the B loads are complete; held from the start, the values' registers made
      // the compiler wait for the first B group before issuing the second) and waited for after
      // the barrier.
      load_bias(bias_r);
      lds_barrier();
#pragma unroll
      for (int j = 0; j < kBiasRegs; ++j) {
        const int e = tid + j * nthr;
        if (e < n * 256) {
          const int sl = e >> 8, o = e & 255, m = o >> 4;
          const int col = c0 + 16 * sl + (o & 15);
          float sum = red[sl][0][o];
          for (int ww = 1; ww < p.split_k; ++ww) sum += red[sl][ww][o];
          if (m < p.M && col < c1) {
            if (p.has_bias) sum += from_bits<DT>((uint16_t)bias_r[j]);
            ((uint16_t *)p.C)[(size_t)m * p.ldc + col] = to_bits<DT>(sum);
          }
        }
      }
      return;
    }
    lds_barrier();
    for (int e = tid; e < n * 256; e += nthr) {
      const int sl = e >> 8, o = e & 255, m = o >> 4;
      const int col = c0 + 16 * (g0 + sl) + (o & 15);
      float sum = red[sl][0][o];
      for (int ww = 1; ww < p.split_k; ++ww) sum += red[sl][ww][o];
      if (m < p.M && col < c1) {
        if (p.has_bias) sum += from_bits<DT>(bias_cached ? bias_s[col - c0] : ((const uint16_t *)p.bias)[col]);
        ((uint16_t *)p.C)[(size_t)m * p.ldc + col] = to_bits<DT>(sum);
      }
    }
    lds_barrier();
  };

  // The next group's loads are issued unconditionally (columns past c1 read zeros without touching
  // memory): with a branch around them the compiler's wait before each park would have to assume
  // either path and waits for the next group's loads as well, which serializes the stream.
  if constexpr (kFew) {
    // ng <= R: group g parked in slot g, the reduction after the loop (no path from it back to
    // the loop head, whose waits would otherwise have to cover its bias loads too)
    // (scheduling barriers: each group's loads go out before the previous group's transpose)
    for (int g = 0; g < ng; g += 2) {
      load_b(b1, c0 + 16 * (g + 1));
      __builtin_amdgcn_sched_barrier(0);
      park(g, mma(b0));
      if (g + 1 >= ng) break;
      load_b(b0, c0 + 16 * (g + 2));
      __builtin_amdgcn_sched_barrier(0);
      park(g + 1, mma(b1));
    }
    if (ng > 0) flush(0, ng);
    return;
  }
  for (int g = 0; g < ng; g += 2) {
    load_b(b1, c0 + 16 * (g + 1));
    if (g == 0 && bias_cached) {
      // the first reduction's barrier orders these writes before any read
#pragma unroll
      for (int j = 0; j < kBiasRegs; ++j)
        if (j * nthr < per) bias_s[j * nthr + tid] = (uint16_t)bias_r[j];
    }
    park(g % R, mma(b0));
    if (g % R == R - 1 || g + 1 == ng) flush(g - g % R, g % R + 1);
    if (g + 1 >= ng) break;
    load_b(b0, c0 + 16 * (g + 2));
    park((g + 1) % R, mma(b1));
    if ((g + 1) % R == R - 1 || g + 2 == ng) flush(g + 1 - (g + 1) % R, (g + 1) % R + 1);
  }
}

// Long partitions: passes of KS steps with fragments loaded directly and A reloaded per pass
// (L2-resident: A is M x K); groups b, b + grid, ...; one reduction per group.
template <int DT>
__device__ __forceinline__ void skinny_gemm_long(const mtk_skinny_args &p) {
  // two LDS buffers of [partition][16 x 16] fp32
  __shared__ __attribute__((aligned(16))) float red[2][8][256];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int groups = (p.N + 15) / 16;
  const rsrc_t ra = make_rsrc(p.A, p.a_bytes);
  const rsrc_t rb = make_rsrc(p.B, p.b_bytes);

  constexpr int KS = kSkinnyResident;
  SkinnyWave<DT, KS> sw;
  sw.arow = (lane & 15) < p.M ? (uint32_t)(lane & 15) * (uint32_t)p.lda * 2u : kOOB;
  sw.k0 = (uint32_t)(w * p.k_per_split);
  sw.k_end = (uint32_t)min(p.K, (int)sw.k0 + p.k_per_split);

  auto park = [&](int buf, f32x4 acc) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[buf][w][(4 * (lane >> 4) + r) * 16 + (lane & 15)] = acc[r];
  };
  int buf = 0;
  for (int g = blockIdx.x; g < groups; g += gridDim.x) {
    f32x4 acc = f32x4{};
    u32x4 b[KS];
    for (int kb = (int)sw.k0; kb < (int)sw.k_end; kb += 32 * KS) {
      sw.load_a(ra, kb, lane);
      sw.load_b(rb, b, g, p.N, p.ldb, kb, lane);
      acc = sw.mma(b, acc);
    }
    park(buf, acc);
    lds_barrier();
    skinny_reduce_store<DT>(p, red[buf], g, tid);
    buf ^= 1;
  }
}

// Partial-writing kernel for 16 < M <= 32 and long K, the shape of the reference's default run
// (f16 32 x 3072 x 80000, split-K 30; matmul.swift main()): one workgroup per (K partition,
// 64 columns), four wavefronts of 16 columns, two workgroups per CU. It writes the two-pass
// schedule's fp32 partials [split_k][M][N] (uniform partitions of k_per_split elements); the
// reduce kernel then adds them in partition order and the bias. Per 256-element chunk of the
// partition, loads two chunks ahead (three register buffers):
//   * every load instruction reads 512 bytes of each of two rows (whole cache lines): each
//     wavefront loads 8 of A's 32 rows and its own 16 B rows;
//   * the wavefronts write their A rows into the chunk's shared LDS buffer (three buffers; row m,
//     16-byte chunk c at slot c ^ (m & 15)), then a barrier; B goes through the wavefront's own
//     LDS region, transposed as in the decode kernel;
//   * 8 K steps of two 16x16x32 MFMAs (rows 0-15 and 16-31 of A) on one B fragment each.
// A is staged through registers rather than direct-to-LDS loads: with those in flight the
// compiler makes every LDS read wait for them (vmcnt(0)), which serializes the chunks.
// Rows m >= M, columns n >= N and K past the partition read zero.
template <int DT>
__device__ __forceinline__ void skinny_gemm_parts(const mtk_skinny_args &p) {
  constexpr int KS = 8;              // MFMA K steps (of 32) per chunk: 256 elements, 512 bytes a row
  constexpr int kStreamPolicy = 2;   // non-temporal B loads
  __shared__ __attribute__((aligned(1024))) u32x4 abuf[3][32][32];  // A chunks: 32 rows x 512 B
  __shared__ __attribute__((aligned(16))) u32x4 tr[4][16][32];      // per wavefront: 16 rows x 512 B

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int ncb = (p.N + 63) / 64;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int part = id / ncb, cb = id - part * ncb;
  const int k0 = part * p.k_per_split;
  const int k1 = min(p.K, k0 + p.k_per_split);
  const int nch = k1 > k0 ? (k1 - k0 + 32 * KS - 1) / (32 * KS) : 0;
  const int n0 = cb * 64 + 16 * w;
  const rsrc_t ra = make_rsrc(p.A, p.a_bytes);
  const rsrc_t rb = make_rsrc(p.B, p.b_bytes);
  const int r = lane & 15, q = lane >> 4;
  const int hl = lane >> 5, sl = lane & 31;  // load instruction lanes: row 2i + hl, 16-byte chunk sl
  u32x4(&t)[16][32] = tr[w];

  // A rows 8w + 2i + hl and B rows n0 + 2i + hl: chunk sl (16 bytes) of the chunk's 512 bytes
  auto load_a = [&](u32x4 (&ar)[4], int kc) {
    const int k = kc + 8 * sl;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 8 * w + 2 * i + hl;
      ar[i] = buf_load16(ra, (m < p.M && k < k1) ? (uint32_t)m * (uint32_t)p.lda * 2u + (uint32_t)k * 2u : kOOB);
    }
  };
  auto load_b = [&](u32x4 (&b)[8], int kc) {
    const int k = kc + 8 * sl;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int n = n0 + 2 * i + hl;
      b[i] = __builtin_amdgcn_raw_buffer_load_b128(
          rb, (n < p.N && k < k1) ? (uint32_t)n * (uint32_t)p.ldb * 2u + (uint32_t)k * 2u : kOOB, 0, kStreamPolicy);
    }
  };
  // row m, chunk c -> slot c ^ (m & 15)
  auto store_a = [&](const u32x4 (&ar)[4], int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 8 * w + 2 * i + hl;
      abuf[buf][m][sl ^ (m & 15)] = ar[i];
    }
  };
  f32x4 acc[2] = {f32x4{}, f32x4{}};
  auto mma = [&](const u32x4 (&b)[8], int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 2 * i + hl;
      t[row][sl ^ (row & 15)] = b[i];
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 bf = t[r][(4 * s + q) ^ r];
#pragma unroll
      for (int rb2 = 0; rb2 < 2; ++rb2) acc[rb2] = mfma16x16x32<DT>(abuf[buf][16 * rb2 + r][(4 * s + q) ^ r], bf, acc[rb2]);
    }
  };

  u32x4 a0[4], a1[4], a2[4], b0[8], b1[8], b2[8];
  // Chunk j: A (its wavefront's 8 rows) into LDS buffer j % 3, a raw barrier (LDS writes done:
  // lgkmcnt(0); __syncthreads' fence would also wait for the loads of chunks j + 1 and j + 2),
  // the loads of chunk j + 2, then the chunk's MFMAs. Loads are issued unconditionally (chunks
  // past the partition read zeros), so the compiler's waits for each register buffer are exact.
  auto step = [&](int j, const u32x4 (&ac)[4], const u32x4 (&bc)[8], int buf, u32x4 (&an)[4], u32x4 (&bn)[8]) {
    store_a(ac, buf);
    lds_barrier();
    load_a(an, k0 + 32 * KS * (j + 2));
    load_b(bn, k0 + 32 * KS * (j + 2));
    mma(bc, buf);
  };
  load_a(a0, k0);
  load_b(b0, k0);
  // chunk 0's loads ahead of chunk 1's: the wait at the loop head (for A of chunk j) is shared by
  // the entry and the back edge, so the entry's issue order sets it for every iteration
  __builtin_amdgcn_sched_barrier(0);
  load_a(a1, k0 + 32 * KS);
  load_b(b1, k0 + 32 * KS);
  // whole triples in a loop without exits (a break between steps gives the loop head a second
  // predecessor whose pending loads the compiler's waits there must also cover), then the rest
  int j = 0;
  for (; j + 3 <= nch; j += 3) {
    step(j, a0, b0, 0, a2, b2);
    step(j + 1, a1, b1, 1, a0, b0);
    step(j + 2, a2, b2, 2, a1, b1);
  }
  if (j < nch) step(j, a0, b0, 0, a2, b2);
  if (j + 1 < nch) step(j + 1, a1, b1, 1, a0, b0);
  wait_vmem();  // the chunks issued past the partition (zeros) land before the workgroup ends

  // 16x16 accumulator layout: lane (c = lane % 16, g = lane / 16), register i -> row 4g + i, col c
  float *P = p.partial + (size_t)part * p.M * p.N;
  const int n = n0 + r;
#pragma unroll
  for (int rb2 = 0; rb2 < 2; ++rb2)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * rb2 + 4 * q + i;
      if (m < p.M && n < p.N) P[(size_t)m * p.N + n] = acc[rb2][i];
    }
}

}  // namespace mtk

using namespace mtk;

#define SKINNY(NAME, DT, BODY) \
  extern "C" __global__ void __launch_bounds__(512) NAME(const mtk_skinny_args a) { BODY<DT>(a); }

#define SKINNY_RESIDENT(NAME, DT, R) \
  extern "C" __global__ void __launch_bounds__(512) NAME(const mtk_skinny_args a) { skinny_gemm_resident<DT, R>(a); }

SKINNY_RESIDENT(mtk_skinny_f16, DT_F16, kSkinnySlots)
SKINNY_RESIDENT(mtk_skinny_bf16, DT_BF16, kSkinnySlots)
SKINNY_RESIDENT(mtk_skinny_few_f16, DT_F16, kSkinnyFew)
SKINNY_RESIDENT(mtk_skinny_few_bf16, DT_BF16, kSkinnyFew)
SKINNY(mtk_skinny_f16_long, DT_F16, skinny_gemm_long)
SKINNY(mtk_skinny_bf16_long, DT_BF16, skinny_gemm_long)

extern "C" __global__ void __launch_bounds__(256) mtk_skinny_parts_f16(const mtk_skinny_args a) {
  skinny_gemm_parts<DT_F16>(a);
}
extern "C" __global__ void __launch_bounds__(256) mtk_skinny_parts_bf16(const mtk_skinny_args a) {
  skinny_gemm_parts<DT_BF16>(a);
}
