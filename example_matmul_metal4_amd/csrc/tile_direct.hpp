// Pipelined MFMA tile kernel with direct-to-LDS staging, parameterised by operand policies.
//
// C[M][N] (+ bias) = A . B with A and B given by policies:
//   A: OpRows  (A [M][lda] row-major, the reference GEMM)            -> LDS [BM][64]
//      OpConv  (implicit-GEMM gather of an NDHWC activation, C%64==0) -> LDS [BM][64]
//      OpColsT (A [K][lda]: the reference's transpose.left)           -> LDS [64][BM]
//   B: OpRows  (B [N][ldb], the reference's default transpose.right)  -> LDS [BN][64]
//      OpColsT (B [K][ldb]: GEMM B [K][N], DHWIO conv weights [K][O])  -> LDS [64][BN]
//
// Staging: gfx950 direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds). One wave instruction
// writes 1 KB of LDS, lane l to byte 16*l; each policy hands every lane the global address of the
// 16 bytes that belong at that slot, so swizzles are applied on the global side. Out-of-range
// offsets read as zero and are written to LDS as zero: rows past M/N, rows past K of a K-major
// operand and convolution padding cost nothing but an offset select. A partial last K-tile of a
// K-contiguous operand is loaded whole and its fragments are masked at K in registers; it runs in
// the same pipeline as the full tiles.
//
// Fragments: [rows][64] tiles use ds_read_b128 with the chunk swizzle chunk ^ (row&7) ^ ((row>>3)&7);
// the [64][cols] tile uses two ds_read_b64_tr_b16 per fragment: in each 16-lane group, lane s
// addresses row k0 + s/4, columns 4*(s%4).. of a 16-column block, and the transposed read hands
// lane s column s of that block at k0 .. k0+3 — exactly the 32x32x16 MFMA B-operand layout.
// Chunk swizzle there: chunk ^ 4*(row%4), which spreads the 8 rows one read touches over 16
// distinct 16-byte bank groups.
//
// Pipeline: two LDS stages, one barrier per 64-deep K-tile, in its middle; fragments are read two
// k-steps ahead into a ring of four k-step buffers, and the loads of K-tile kt + 2 go into the
// stage of K-tile kt during its last two k-steps. Each k-step's MFMAs are interleaved in groups with
// those loads and the fragment reads (scheduling fences keep the compiler from regrouping them).
#pragma once

#include "tile_gemm.hpp"



namespace mtk {

// ---------------------------------------------------------------- operand policies

// Every policy stages its share of a K-tile with NW wavefronts: 1 KB blocks per wavefront.

// Row-major operand, K contiguous: A [M][lda] or B [N][ldb]. LDS tile [ROWS][64].
template <int ROWS, int NW = 4>
struct OpRows {
  static constexpr int kWaves = NW;
  static constexpr bool kIsConv = false;
  static constexpr int kLoads = ROWS / (8 * NW);  // 1 KB blocks per wave per K-tile
  static constexpr bool kNeedsTail = true;  // the last K-tile's fragments are masked at K
  static constexpr int kReadsPerFrag = 1;
  uint32_t off[kLoads];
  int blk0;
  int ld;

  __device__ void init(const mtk_tile_args &, int wave, int lane, int row0, int nrows, int ld_) {
    ld = ld_;
    blk0 = wave * kLoads;
    const int cbase = (lane & 7) ^ (lane >> 3);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int b = blk0 + i, row = row0 + 8 * b + (lane >> 3);
      off[i] = row < nrows ? (uint32_t)row * (uint32_t)ld * 2u + 16u * (uint32_t)(cbase ^ (b & 7)) : kOOB;
    }
  }
  __device__ __forceinline__ void issue(rsrc_t r, char *lds, int q, int kt) const {
    lds_direct16(r, lds + (blk0 + q) * 1024, off[q] + (uint32_t)kt * 128u);
  }
  // The last K-tile of a K that is not a multiple of 64 is loaded whole (chunks past K hold the
  // next row's elements, or zeros past the operand); its fragments are masked before use. A
  // fragment holds the 8 elements k0 .. k0+7 of one row.
  __device__ static __forceinline__ u32x4 mask(u32x4 v, int k0, int K) {
    const int n = K - k0;  // valid elements in this chunk
    u32x4 r;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t keep = 2 * d + 1 < n ? 0xffffffffu : (2 * d < n ? 0x0000ffffu : 0u);
      r[d] = v[d] & keep;
    }
    return r;
  }
  // K offset of the fragment a lane reads for k-step ks of K-tile kt
  __device__ static __forceinline__ int frag_k0(int kt, int ks, int lane) { return kt * kBK + 16 * ks + 8 * (lane >> 5); }
  // (the two-ahead ring measured 2-3 % faster with this form of the offset; the one-ahead loop's
  // in-place reads below needed the registers frag_off saves)
  __device__ __forceinline__ u32x4 frag(const char *lds, int rowblk, int ks, int lane) const {
    return ds_read_b128_at<0>(lds_addr(lds) + lds_off(rowblk + (lane & 31), 2 * ks + (lane >> 5)));
  }
  __device__ __forceinline__ void frag_to(u32x4 &dst, const char *lds, int rowblk, int ks, int lane) const {
    ds_read_b128_into<0>(dst, lds_addr(lds) + frag_off(rowblk, ks, lane));
  }
};

// Implicit-GEMM gather of an NDHWC activation (C % 64 == 0, filter extents <= 10): tile row m is
// output pixel (n, oz, oh, ow); a 64-wide K-tile is one filter tap (kd, kh, kw) and 64 channels.
// Per tile row the lane keeps the element offset of (n, oz*SZ-PF, oh*SY-PT, ow*SX-PL, 0) plus its
// chunk, and the in-range taps as three bit masks packed in one word (10 bits each).
template <int ROWS, int NW = 4>
struct OpConv {
  static constexpr int kWaves = NW;
  static constexpr bool kIsConv = true;
  static constexpr int kLoads = ROWS / (8 * NW);
  static constexpr bool kNeedsTail = false;  // K = taps * C is a multiple of 64
  static constexpr int kReadsPerFrag = 1;
  int pb8[kLoads];
  uint32_t pm[kLoads];
  int blk0;

  __device__ void init(const mtk_tile_args &a, int wave, int lane, int row0, int, int) {
    blk0 = wave * kLoads;
    const int cbase = (lane & 7) ^ (lane >> 3);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int b = blk0 + i;
      const int m = row0 + 8 * b + (lane >> 3);
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
      pb8[i] = base + 8 * (cbase ^ (b & 7));
      pm[i] = z | (h << 10) | (w << 20);
    }
  }
  // Tap decode for K-tile kt (uniform across the workgroup).
  struct Tap {
    int elems;  // element offset of the tap and the tile's first channel
    int kd, kh, kw;
  };
  __device__ __forceinline__ Tap tap(const mtk_tile_args &a, int kt) const {
    const int k0 = kt * kBK;
    const int t = k0 / a.cC;
    Tap r;
    r.kw = t % a.cKW;
    r.kh = (t / a.cKW) % a.cKH;
    r.kd = t / (a.cKW * a.cKH);
    r.elems = ((r.kd * a.cDZ * a.cH + r.kh * a.cDY) * a.cW + r.kw * a.cDX) * a.cC + (k0 - t * a.cC);
    return r;
  }
  // The same decode for the channel-block-major K order (all filter taps of channels 0..63, then of
  // 64..127, ...), walked one K-tile at a time: tap t = (kd KH + kh) KW + kw and channel block cb
  // advance with scalar compares, where tap() takes five run-time divisions per K-tile. K-tile
  // t C / 64 + cb of the tap-major operand order gives the same Tap.
  struct TapWalk {
    int kd = 0, kh = 0, kw = 0, t = 0, cb = 0;
  };
  __device__ __forceinline__ static void advance(const mtk_tile_args &a, TapWalk &w) {
    ++w.t;
    if (++w.kw == a.cKW) {
      w.kw = 0;
      if (++w.kh == a.cKH) {
        w.kh = 0;
        if (++w.kd == a.cKD) {
          w.kd = 0;
          w.t = 0;
          ++w.cb;
        }
      }
    }
  }
  // ... and for the tap-major order (all channel blocks of tap 0, then of tap 1, ...)
  __device__ __forceinline__ static void advance_tap_major(const mtk_tile_args &a, TapWalk &w) {
    if (++w.cb == a.cC / kBK) {
      w.cb = 0;
      ++w.t;
      if (++w.kw == a.cKW) {
        w.kw = 0;
        if (++w.kh == a.cKH) {
          w.kh = 0;
          ++w.kd;
        }
      }
    }
  }
  __device__ __forceinline__ static Tap tap_at(const mtk_tile_args &a, const TapWalk &w) {
    Tap r;
    r.kd = w.kd;
    r.kh = w.kh;
    r.kw = w.kw;
    r.elems = ((w.kd * a.cDZ * a.cH + w.kh * a.cDY) * a.cW + w.kw * a.cDX) * a.cC + w.cb * kBK;
    return r;
  }
  __device__ __forceinline__ void issue(rsrc_t r, char *lds, int q, const Tap &tp) const {
    const bool ok = (pm[q] >> tp.kd) & (pm[q] >> (10 + tp.kh)) & (pm[q] >> (20 + tp.kw)) & 1u;
    lds_direct16(r, lds + (blk0 + q) * 1024, ok ? (uint32_t)(pb8[q] + tp.elems) * 2u : kOOB);
  }
  __device__ __forceinline__ u32x4 frag(const char *lds, int rowblk, int ks, int lane) const {
    return ds_read_b128_at<0>(lds_addr(lds) + lds_off(rowblk + (lane & 31), 2 * ks + (lane >> 5)));
  }
  __device__ __forceinline__ void frag_to(u32x4 &dst, const char *lds, int rowblk, int ks, int lane) const {
    ds_read_b128_into<0>(dst, lds_addr(lds) + frag_off(rowblk, ks, lane));
  }
};

// [K][ld] operand (N contiguous): GEMM B [K][N], conv weights DHWIO = [K][O]. LDS tile [64][COLS]
// (row = k), 16-byte chunk c of row k stored at chunk c ^ 4*(k%4).
template <int COLS, int NW = 4>
struct OpColsT {
  static constexpr int kWaves = NW;
  static constexpr bool kIsConv = false;
  static constexpr int kRowBytes = COLS * 2;
  static constexpr int kLoads = COLS / (8 * NW);  // 64 rows x kRowBytes / 1 KB / NW waves
  static constexpr bool kNeedsTail = false;  // rows k >= K are past the operand: read as zero
  static constexpr int kReadsPerFrag = 2;  // two transposed 8-byte reads
  uint32_t off[kLoads];
  int blk0;
  uint32_t kstride;  // bytes per K-tile (64 rows)

  __device__ void init(const mtk_tile_args &, int wave, int lane, int col0, int, int ld) {
    blk0 = wave * kLoads;
    kstride = (uint32_t)ld * 2u * kBK;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int byte = (blk0 + i) * 1024 + lane * 16;
      const int row = byte / kRowBytes;
      const int pc = (byte % kRowBytes) / 16;
      const int lc = pc ^ (4 * (row & 3));
      off[i] = ((uint32_t)row * (uint32_t)ld + (uint32_t)(col0 + 8 * lc)) * 2u;
    }
  }
  __device__ __forceinline__ void issue(rsrc_t r, char *lds, int q, int kt) const {
    lds_direct16(r, lds + (blk0 + q) * 1024, off[q] + (uint32_t)kt * kstride);
  }
  __device__ __forceinline__ void frag_to(u32x4 &dst, const char *lds, int colblk, int ks, int lane) const {
    dst = frag(lds, colblk, ks, lane);
  }
  __device__ __forceinline__ u32x4 frag(const char *lds, int colblk, int ks, int lane) const {
    const int s = lane & 15, h = lane >> 4;
    const int col = colblk + 16 * (h & 1) + 4 * (s & 3);
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int row = 16 * ks + 8 * (h >> 1) + 4 * e + (s >> 2);
      const int lc = col >> 3;
      const char *p = lds + row * kRowBytes + 16 * (lc ^ (4 * (row & 3))) + 2 * (col & 7);
      const u32x2 w = ds_read_tr16(p);
      v[2 * e] = w.x;
      v[2 * e + 1] = w.y;
    }
    return v;
  }
};

// ---------------------------------------------------------------- waits

// vmcnt(N): at most N vector-memory operations of this wave outstanding (direct-to-LDS loads
// included); LDS reads are not waited for.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// Wave issue priority around a k-step's MFMA groups, for 128x128 tiles (two workgroups per CU, so
// the two wavefronts of a SIMD belong to different workgroups and drift apart): the one in its
// MFMA groups issues first, the other's loads and reads fill the gaps. 128x128 convolution 3 %
// faster; the 256x256 tiles (both wavefronts of a SIMD in one workgroup, in step at its barriers)
// measured no gain per k-step and 2-3 % slower per MFMA group.
template <int P>
__device__ __forceinline__ void mfma_priority() {
  __builtin_amdgcn_s_setprio(P);
}

// Fragments filled by inline-asm LDS reads are handed to their consumers through empty asm
// statements that take them as in/out operands: no use can be scheduled above the wait before it.
template <int TA, int TB>
__device__ __forceinline__ void frag_tie(u32x4 (&fa)[TA], u32x4 (&fb)[TB]) {
#pragma unroll
  for (int i = 0; i < TA; ++i) asm volatile("" : "+v"(fa[i]));
#pragma unroll
  for (int j = 0; j < TB; ++j) asm volatile("" : "+v"(fb[j]));
}

// lgkmcnt(N): at most N LDS reads of this wave outstanding (they complete in issue order), then
// the fragments of the k-step about to run are tied to the wait.
template <int N, int TA, int TB>
__device__ __forceinline__ void frag_wait(u32x4 (&fa)[TA], u32x4 (&fb)[TB]) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
  frag_tie(fa, fb);
}

// ---------------------------------------------------------------- the kernel body

// SERIAL (GEMM split-K on a tile grid that already fills the chip, at most 4 partitions): one
// workgroup per output tile runs the K partitions one after another through one continuous
// pipeline. At the end of each partition but the last its fp32 sum is added to the tile's running
// sum (part in the workspace, part in registers, one accumulator block per wavefront in LDS) and
// the accumulators restart from zero; the epilogue adds the running sum and the last partition,
// then the bias. The arithmetic is the two-pass split-K's: every partition accumulates from zero
// over the same K-tiles, partition sums are added in partition order, the bias last.
template <int DT, int BM, int BN, int WAVES_M, int WAVES_N, typename AOP, typename BOP, bool SERIAL = false>
__device__ __forceinline__ void tile_direct(const mtk_tile_args &a) {
  constexpr int NW = WAVES_M * WAVES_N;
  static_assert(NW == 4 || NW == 8, "4 or 8 wavefronts per workgroup");
  static_assert(AOP::kWaves == NW && BOP::kWaves == NW, "operand policies staged by the same wavefronts");
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= TN, "fragment reads are paired per row block");
  constexpr int kStage = (BM + BN) * 128;
  constexpr int PA = AOP::kLoads, PB = BOP::kLoads;
  // The loads of K-tile kt + 2 go out in the MFMA groups of k-steps 2 and 3 of K-tile kt; the
  // barrier in the middle of K-tile kt + 1 waits for them.
  constexpr int kLoadGroups = 2 * TM;
  constexpr int kPerGroup = (PA + PB + kLoadGroups - 1) / kLoadGroups;
  constexpr int kReadsPerGroup = (TM + TN + TM - 1) / TM;  // next k-step's fragment reads per MFMA group

  // The K loop: fragments two k-steps ahead through a ring of four k-step buffers, or (256x256
  // convolution and split-K) one k-step ahead through two.
  constexpr bool kOneAhead = BM == 256 && (AOP::kIsConv || SERIAL);
  // SERIAL: where each wavefront's running sum lives, by accumulator block b = i + TM * j: blocks
  // b < kSlotBlocks in the workspace slot, the next kRegBlocks in registers (the registers the
  // fragments leave free: three blocks at 256x256 with the one-ahead loop, two at 128x128), the last
  // one, (TM - 1, TN - 1), in LDS past the two stages (4 KB per wavefront: 32 KB at 256x256, which
  // fills the 160 KB of LDS).
  constexpr int kLdsBlocks = SERIAL ? 1 : 0;
  constexpr int kRegBlocks = SERIAL ? (BM == 256 ? 3 : 2) : 0;
  constexpr int kSlotBlocks = SERIAL ? TM * TN - kLdsBlocks - kRegBlocks : 0;
  static_assert(kSlotBlocks >= 0, "running-sum blocks");
  constexpr int kLdsRun = kLdsBlocks * NW * 4096;
  static_assert(2 * kStage + kLdsRun <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage + kLdsRun];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave_m = wave / WAVES_N, wave_n = wave % WAVES_N;

  const int tiles = a.tiles_m * a.tiles_n;
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int split = SERIAL ? 0 : id / tiles;
  const int t = id - split * tiles;
  const int group = kGroupM * a.tiles_n;
  const int first_m = (t / group) * kGroupM;
  const int gm = min(a.tiles_m - first_m, kGroupM);
  const int tm = first_m + (t % group) % gm;
  const int tn = (t % group) / gm;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kt0 = SERIAL ? 0 : split_first_tile(a, split, t);
  const int kt1 = SERIAL ? a.k_tiles : split_first_tile(a, split + 1, t);
  constexpr bool kAnyTail = AOP::kNeedsTail || BOP::kNeedsTail;
  const bool tail_here = kAnyTail && (a.K % kBK) != 0 && kt1 == a.k_tiles && kt0 < kt1;
  const int kfull = tail_here ? kt1 - 1 : kt1;

  const rsrc_t ra = make_rsrc(a.A, a.a_bytes);
  const rsrc_t rb = make_rsrc(a.B, a.b_bytes);
  AOP opa;
  BOP opb;
  opa.init(a, wave, lane, m0, a.M, a.lda);
  opb.init(a, wave, lane, n0, a.N, a.ldb);

  // one K-tile's loads into stage base `st`
  auto issue_all = [&](char *st, int kt) {
    if constexpr (AOP::kIsConv) {
      const auto tp = opa.tap(a, kt);
#pragma unroll
      for (int q = 0; q < PA; ++q) opa.issue(ra, st, q, tp);
    } else {
#pragma unroll
      for (int q = 0; q < PA; ++q) opa.issue(ra, st, q, kt);
    }
#pragma unroll
    for (int q = 0; q < PB; ++q) opb.issue(rb, st + BM * 128, q, kt);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

  // SERIAL: the running sum of the finished partitions of this workgroup's tile lives in the
  // tile's slot of the workspace ([tiles][MTK_SERIAL_SLOT_BYTES(BM)]), in accumulator order (wave,
  // block b = i + TM * j, register quad, lane): each lane moves 16 bytes per instruction, one
  // instruction covers 1 KB of contiguous memory, and only this lane reads back what it wrote.
  // Only the blocks b < kSlotBlocks live there (the others below). The first boundary stores
  // partition 0; later ones add the finished partition to the slot ((p0 + p1) + p2 ...); the
  // epilogue adds the slot in front of the last partition. Slot loads bypass L1 (device scope), so
  // a line read at one boundary is never served stale at the next. The last block (TM - 1, TN - 1)
  // of every wavefront keeps its running sum in the LDS left over by the two stages instead, and
  // the kRegBlocks blocks before it in registers (the same additions in the same order): at
  // 256x256 half of the running sum never leaves the CU (config 2 split-K 4: 196.7 us with all of
  // it in the slot, 191.0 with the LDS block, 176.4 with three register blocks as well and the
  // one-ahead loop; medians, one process, same bits).
  constexpr uint32_t kSlotBytes = NW * kSlotBlocks * 4096;
  static_assert(!SERIAL || (BM == BN && kSlotBytes == MTK_SERIAL_SLOT_BYTES(BM)), "slot size shared with the host");
  // Slot traffic is streamed: nt on stores and loads alike, which keeps it from displacing the A/B
  // panels the other tiles of the XCD are reading (measured: 183 us vs 201 us with sc1 alone at
  // config 2), and sc1 on loads (device scope: served by L2, never by a possibly stale L1 line; a
  // lane reads back only what it wrote itself, through the same XCD's L2). Stores without sc1
  // measured 1.5-2 % faster with three register blocks (two sweeps of eight interleaved rounds;
  // sc1 on loads only, sc0 or no policy on stores, sc1 alone: no faster).
  constexpr int kStorePolicy = 2;
  constexpr int kLoadPolicy = 16 | 2;
  constexpr int kSlotRing = 2;  // accumulator blocks of the slot in flight (deeper rings spill)
  const rsrc_t rslot = make_rsrc(SERIAL ? a.partial + (size_t)t * (kSlotBytes / 4) : nullptr, SERIAL ? kSlotBytes : 0u);
  // LDS byte address of this lane's part of the LDS-resident running-sum block
  auto lds_run_at = [&]() {
    int l = lane_id();
    asm volatile("" : "+v"(l));
    return lds_addr(smem) + (uint32_t)(2 * kStage + wave * 4096 + l * 16);
  };
  // this lane's first slot byte (recomputed where used, so it is not held across the K loop)
  auto slot_lane_at = [&]() {
    int l = lane_id();
    asm volatile("" : "+v"(l));
    return (uint32_t)(wave * (kSlotBlocks * 1024) + l * 4) * 4u;
  };
  // Loads: the block's byte offset within the wave's part of the slot goes in the scalar offset
  // operand (it exceeds the 12-bit immediate): the lane part stays one register. Per-block lane
  // offsets were otherwise held in 32 registers across the K loop, and spilled.
  // Stores: the block offset is added to the lane offset (one VALU add per store) and the scalar
  // offset is 0. The compiler's hazard check takes a 16-byte buffer store whose scalar offset is a
  // register to need no wait states before its data registers are rewritten; on this hardware a
  // VALU write of them in the very next instruction corrupted the stored data (measured: one such
  // instruction pair in a build of this kernel, that block's values non-repeatable in 31 of 256
  // tiles). With a constant scalar offset the compiler inserts the wait states itself.
  auto slot_blk = [](int i, int j, int q) { return (i + TM * j) * 4096 + q * 1024; };  // slot blocks only
  auto slot_load = [&](uint32_t slot_lane, int i, int j, int q) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rslot, slot_lane, slot_blk(i, j, q), kLoadPolicy));
  };
  auto slot_store = [&](f32x4 v, uint32_t slot_lane, int i, int j, int q) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rslot, slot_lane + (uint32_t)slot_blk(i, j, q), 0,
                                           kStorePolicy);
  };
  int split_end = SERIAL ? split_first_tile(a, 1, t) : 0;  // SERIAL: first K-tile of the next partition
  int parked = 0;                                           // SERIAL: partitions parked so far
  constexpr int kSlotStores = kSlotBlocks * 4;  // slot store instructions per wavefront and boundary
  static_assert(!SERIAL || kSlotStores < 64, "vmcnt range");
  // SERIAL: running sums of the register-resident accumulator blocks (set at the first boundary,
  // read only after one)
  f32x16 run[kRegBlocks > 0 ? kRegBlocks : 1];

  // SERIAL, at a partition boundary (every LDS read of the loop waited for): running sum += the
  // finished partition's sum (partition 0's sum as it is), accumulators back to zero.
  auto park = [&]() {
    const uint32_t slot_lane = slot_lane_at();
    // the LDS-resident block (TM - 1, TN - 1), in place (inline asm: ordinary LDS accesses would
    // wait for the next partition's K-tile loads in flight)
    if constexpr (kLdsBlocks > 0) {
      const uint32_t la = lds_run_at();
      constexpr int I = TM - 1, J = TN - 1;
      if (parked > 0) {
        // one register quad at a time (the boundary is where registers are scarcest)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          u32x4 prev = lds_rd128(la + 1024u * q);
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(prev));
          const f32x4 v = __builtin_bit_cast(f32x4, prev) +
                          f32x4{acc[I][J][4 * q], acc[I][J][4 * q + 1], acc[I][J][4 * q + 2], acc[I][J][4 * q + 3]};
          lds_wr128(la + 1024u * q, __builtin_bit_cast(u32x4, v));
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          lds_wr128(la + 1024u * q, __builtin_bit_cast(u32x4, f32x4{acc[I][J][4 * q], acc[I][J][4 * q + 1],
                                                                    acc[I][J][4 * q + 2], acc[I][J][4 * q + 3]}));
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // the register-resident blocks
#pragma unroll
    for (int r = 0; r < kRegBlocks; ++r) {
      const int b = kSlotBlocks + r;
      run[r] = parked > 0 ? run[r] + acc[b % TM][b / TM] : acc[b % TM][b / TM];
    }
    // the slot blocks
    if (parked == 0) {
#pragma unroll
      for (int b = 0; b < kSlotBlocks; ++b)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x16 &s = acc[b % TM][b / TM];
          slot_store(f32x4{s[4 * q], s[4 * q + 1], s[4 * q + 2], s[4 * q + 3]}, slot_lane, b % TM, b / TM, q);
        }
    } else {
      // one register quad (16 bytes per lane) at a time, the next kAheadQ quads' loads in flight
      constexpr int kQuads = kSlotBlocks * 4, kAheadQ = 3;
      auto quad_load = [&](int x) { return slot_load(slot_lane, (x / 4) % TM, (x / 4) / TM, x % 4); };
      f32x4 ring[kAheadQ + 1];
#pragma unroll
      for (int x = 0; x < kAheadQ && x < kQuads; ++x) ring[x] = quad_load(x);
#pragma unroll
      for (int x = 0; x < kQuads; ++x) {
        const int i = (x / 4) % TM, j = (x / 4) / TM, q = x % 4;
        if (x + kAheadQ < kQuads) ring[(x + kAheadQ) % (kAheadQ + 1)] = quad_load(x + kAheadQ);
        const f32x4 v = ring[x % (kAheadQ + 1)] +
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        slot_store(v, slot_lane, i, j, q);
      }
    }
    ++parked;
    split_end = split_first_tile(a, parked + 1, t);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};
  };
  // SERIAL: the K loop runs once per partition (the pipeline carries on across the boundary).
  // Partition boundaries lie strictly inside K (at most split_k-1 of them); the K loop ends anywhere
  // else (or at K itself) after the last partition. Only boundaries park, so every slot written is
  // one of this tile's split_k-1.
  auto at_boundary = [&](int kt) { return kt == split_end && split_end < a.k_tiles && parked < a.split_k - 1; };

  if constexpr (!kOneAhead) {
    // Fragments: a ring of four k-step buffers (slot s holds k-step s of a K-tile), read two k-steps
    // ahead. The reads are inline asm, which the compiler does not track: it would otherwise make
    // every LDS read wait for the direct-to-LDS loads in flight, and at the loop's back edge for
    // every read. Each k-step waits for its own reads only (lgkmcnt counts them in issue order).
    constexpr int kStepReads = TM * AOP::kReadsPerFrag + TN * BOP::kReadsPerFrag;
    static_assert(kStepReads <= 15, "lgkmcnt range");
    u32x4 fa[4][TM], fb[4][TN];
    auto read_step = [&](auto s_c, const char *st) {
      constexpr int S = decltype(s_c)::value;
  #pragma unroll
      for (int i = 0; i < TM; ++i) fa[S][i] = opa.frag(st, wave_m * WTM + i * 32, S, lane);
  #pragma unroll
      for (int j = 0; j < TN; ++j) fb[S][j] = opb.frag(st + BM * 128, wave_n * WTN + j * 32, S, lane);
    };

    // Convolutions (tap-major K order, kt0 = 0): the tap walk at the K-tile whose loads go out next.
    typename std::conditional<AOP::kIsConv, typename OpConv<BM, NW>::TapWalk, int>::type walk{};
    auto issue_walk = [&](char *st) {
      if constexpr (AOP::kIsConv) {
        const auto tp = OpConv<BM, NW>::tap_at(a, walk);
#pragma unroll
        for (int q = 0; q < PA; ++q) opa.issue(ra, st, q, tp);
#pragma unroll
        for (int q = 0; q < PB; ++q) opb.issue(rb, st + BM * 128, q, walk.t * (a.cC / kBK) + walk.cb);
      }
    };
    // Prologue: K-tiles kt0 and kt0 + 1 into the two stages, the first two k-steps' fragments.
    if (kt0 < kt1) {
      if constexpr (AOP::kIsConv) {
        issue_walk(smem);
        if (kt0 + 1 < kt1) OpConv<BM, NW>::advance_tap_major(a, walk);
        issue_walk(smem + kStage);
      } else {
        issue_all(smem, kt0);
        issue_all(smem + kStage, min(kt0 + 1, kt1 - 1));
      }
      vm_wait<PA + PB>();  // the first K-tile's loads (the second's may still be in flight)
      __builtin_amdgcn_s_barrier();
      read_step(std::integral_constant<int, 0>{}, smem);
      read_step(std::integral_constant<int, 1>{}, smem);
    }
    // Asm reads land in their registers asynchronously, unseen by the compiler: wherever code it
    // schedules freely follows (here, the loop entry; the partition boundary; the end), the reads in
    // flight are waited for first, so a register copy or spill never takes a value before it lands.
    frag_wait<0>(fa[0], fb[0]);
    frag_tie(fa[1], fb[1]);

    // One K-tile: four k-steps of TM groups of TN MFMAs. K-steps 0 and 1 read k-steps 2 and 3 of this
    // K-tile's stage; the barrier before k-step 2 (every wave done reading the stage, K-tile kt + 1
    // landed) frees the stage, so k-steps 2 and 3 read k-steps 0 and 1 of the next K-tile and load
    // K-tile kt + 2 into this stage, which the barrier of the next K-tile waits for. Past the end the
    // last K-tile is reloaded (L2 hits, never computed) instead of a branch. PRE (SERIAL only): the
    // first K-tile after a partition boundary, whose wait leaves the boundary's slot stores in flight
    // (vector memory operations complete in issue order; the next K-tile's loads went out before
    // them).
    auto ktile = [&](const int kt, auto pre_c) {
      constexpr bool PRE = decltype(pre_c)::value;
      const int cur = (kt - kt0) & 1;
      char *sc = smem + cur * kStage;
      const char *sn = smem + (cur ^ 1) * kStage;
      int kn = min(kt + 2, kt1 - 1);
      typename std::conditional<AOP::kIsConv, typename OpConv<BM, NW>::Tap, int>::type tp{};
      if constexpr (AOP::kIsConv) {
        // K-tile min(kt + 2, kt1 - 1) (past the end the last one is reloaded)
        if (kt + 2 < kt1) OpConv<BM, NW>::advance_tap_major(a, walk);
        kn = walk.t * (a.cC / kBK) + walk.cb;
        tp = OpConv<BM, NW>::tap_at(a, walk);
      }
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, kBK / 16>([&](auto k_c) {
        constexpr int ks = decltype(k_c)::value;
        constexpr int kr = (ks + 2) & 3;  // the k-step read during this one (ring slot)
        if constexpr (ks == 2) {
          frag_wait<0>(fa[2], fb[2]);
          frag_tie(fa[3], fb[3]);
          if constexpr (PRE)
            vm_wait<kSlotStores>();
          else
            vm_wait<0>();
          __builtin_amdgcn_s_barrier();
        } else {
          frag_wait<kStepReads>(fa[ks], fb[ks]);
        }
        const char *src = ks < 2 ? sc : sn;
        if constexpr (BM == 128) mfma_priority<1>();
  #pragma unroll
        for (int i = 0; i < TM; ++i) {
  #pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16<DT>(fa[ks][i], fb[ks][j], acc[i][j]);
          if constexpr (ks >= 2) {
  #pragma unroll
            for (int u = 0; u < kPerGroup; ++u) {
              const int q = ((ks - 2) * TM + i) * kPerGroup + u;
              if (q < PA) {
                if constexpr (AOP::kIsConv)
                  opa.issue(ra, sc, q, tp);
                else
                  opa.issue(ra, sc, q, kn);
              } else if (q < PA + PB) {
                opb.issue(rb, sc + BM * 128, q - PA, kn);
              }
            }
          }
          // The next k-step's first MFMA group needs every B fragment and only A fragment 0, later
          // groups one more A fragment each: read the B fragments in the first groups, then A.
  #pragma unroll
          for (int u = 0; u < kReadsPerGroup; ++u) {
            const int slot = i * kReadsPerGroup + u;
            if (slot < TN)
              fb[kr][slot] = opb.frag(src + BM * 128, wave_n * WTN + slot * 32, kr, lane);
            else if (slot < TN + TM)
              fa[kr][slot - TN] = opa.frag(src, wave_m * WTM + (slot - TN) * 32, kr, lane);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (BM == 128) mfma_priority<0>();
      });
    };

    int kt = kt0;
    bool pre = false;
    for (;;) {
      const int kstop = SERIAL ? min(split_end, kfull) : kfull;
      if constexpr (SERIAL) {
        if (pre && kt < kstop) ktile(kt++, std::true_type{});
        pre = false;
      }
      for (; kt < kstop; ++kt) ktile(kt, std::false_type{});
      if constexpr (!SERIAL) {
        break;
      } else {
        if (!at_boundary(kt)) break;
        pre = true;
        frag_wait<0>(fa[0], fb[0]);
        frag_tie(fa[1], fb[1]);
        park();
      }
    }
    // The reads of the last K-tile's k-steps 2 and 3 (fragments of the partial last K-tile, or of a
    // K-tile that is never computed) may still be in flight.
    frag_wait<0>(fa[0], fb[0]);
    frag_tie(fa[1], fb[1]);
    if constexpr (kAnyTail) {
      if (tail_here) {
        // The partial last K-tile, already in LDS (loaded as a next K-tile by the loop, or by the
        // prologue when it is the only one) with its first two k-steps' fragments in slots 0 and 1:
        // the same k-steps, fragments masked at K.
        const char *st = smem + ((kfull - kt0) & 1) * kStage;
        static_for<0, kBK / 16>([&](auto k_c) {
          constexpr int ks = decltype(k_c)::value;
          frag_wait<(ks < 2 ? kStepReads : 0)>(fa[ks], fb[ks]);
          if constexpr (AOP::kNeedsTail) {
  #pragma unroll
            for (int i = 0; i < TM; ++i) fa[ks][i] = AOP::mask(fa[ks][i], AOP::frag_k0(kfull, ks, lane), a.K);
          }
          if constexpr (BOP::kNeedsTail) {
  #pragma unroll
            for (int j = 0; j < TN; ++j) fb[ks][j] = BOP::mask(fb[ks][j], BOP::frag_k0(kfull, ks, lane), a.K);
          }
  #pragma unroll
          for (int i = 0; i < TM; ++i) {
  #pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16<DT>(fa[ks][i], fb[ks][j], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
          }
          if constexpr (ks < 2) read_step(std::integral_constant<int, ks + 2>{}, st);
        });
      }
    }
  } else {
    // 256x256 convolution and 256x256 in-workgroup split-K GEMM: fragments one k-step ahead; the
    // loads of K-tile kt + 1 go out in the first MFMA groups of K-tile kt and are waited for at one
    // barrier before its last k-step. Convolution: the two-ahead ring measured 2-5 % slower on this
    // gather, whose loads of K-tile kt + 2 then come in the second half of K-tile kt (on the 128x128
    // convolution it is 1-2 % faster). Split-K: the ring's fragments take 96 registers per lane,
    // these 36, and the registers freed hold three accumulator blocks' running sums (so half of each
    // wavefront's running sum never leaves the CU).
    // Fragment registers: B fragments double-buffered by k-step parity; A fragment i of the next
    // k-step is read into A fragment i's own register right after MFMA group i (the last use of
    // it), so A takes TM registers plus one: A fragment TM - 1 of the last k-step of a K-tile goes
    // to the spare (its regular register is still in use by group TM - 1 when the read is issued,
    // in group TM - 2, early enough to be waited for with the barrier), and the next K-tile's
    // A fragment TM - 1 goes back to its regular register in the last k-step's group 0. Each group
    // waits (counted lgkmcnt, reads complete in issue order) for the reads it uses only.
    // Convolution K-tiles are visited channel-block-major: all filter taps of channels 0..63, then
    // of 64..127, and so on (K-tile kt of the visit is tap kt % T of channel block kt / T, i.e.
    // K-tile (kt % T) * (C / 64) + kt / T of the tap-major K order the operands are laid out in).
    // The gather's reuse distance is shorter than tap-major (neighbouring taps read overlapping
    // pixel windows one after the other): conv2d 177.9 -> 172.1 us, the reference's 512-channel
    // conv2d profile shape 336.8 -> 324.8 us. (With 128 channels, as at config 4b's 128x128 tiles,
    // tap-major measured faster: both halves of a pixel's 256-byte channel row are then read back
    // to back.)
    static_assert(!AOP::kIsConv || (!SERIAL && !kAnyTail), "convolutions never split K and have whole K-tiles");
    constexpr int kLast = kBK / 16 - 1;  // k-steps per K-tile - 1
    static_assert(TM >= 3 && kLast == 3, "fragment schedule");
    int taps = 1, cblocks = 1;
    if constexpr (AOP::kIsConv) {
      taps = a.cKD * a.cKH * a.cKW;
      cblocks = a.cC / kBK;
    }
    auto kmap = [&](int kt) { return AOP::kIsConv ? (kt % taps) * cblocks + kt / taps : kt; };
    // convolutions: the tap walk at the K-tile whose loads go out next (kt0 = 0: no split-K)
    typename std::conditional<AOP::kIsConv, typename OpConv<BM, NW>::TapWalk, int>::type walk{};
    constexpr int kGroups1 = (kBK / 16) * TM;
    constexpr int kLoadGroups1 = 8 < kGroups1 - TM ? 8 : kGroups1 - TM;
    constexpr int kPerGroup1 = (PA + PB + kLoadGroups1 - 1) / kLoadGroups1;

    // the register of k-step ks's A fragment i
    constexpr auto areg = [](int ks, int i) { return ks == kLast && i == TM - 1 ? TM : i; };
    // LDS read instructions issued by k-step p in MFMA group g (the fragments of k-step p + 1, the
    // B fragments first in group 0)
    constexpr int RA = AOP::kReadsPerFrag, RB = BOP::kReadsPerFrag;
    constexpr auto nreads = [](int p, int g) {
      if (p == kLast) return g == 0 ? TN * RB + 2 * RA : (g < TM - 1 ? RA : 0);
      if (p == kLast - 1) return g == 0 ? TN * RB + RA : (g < TM - 2 ? RA : (g == TM - 2 ? 2 * RA : 0));
      return g == 0 ? TN * RB + RA : RA;
    };
    // read instructions k-step p issues after the last one of k-step p + 1's A fragment i
    constexpr auto later = [](int p, int i) {
      const int slot = p == kLast ? (i == 0 ? 0 : (i == TM - 1 ? 1 : i + 1)) : i;  // A reads before it
      return (TM - 1 - slot) * RA;
    };
    // lgkmcnt before MFMA group g of k-step c: the reads issued after the last one the group uses
    // (B fragments and A fragment 0 in group 0, A fragment g later), by k-step c - 1 and by k-step
    // c's earlier groups
    constexpr auto wcount = [=](int c, int g) {
      int n = later((c + kLast) % (kLast + 1), g);
      for (int h = 0; h < g; ++h) n += nreads(c, h);
      return n;
    };
    static_assert(wcount(0, TM - 1) <= 15 && wcount(1, TM - 1) <= 15, "lgkmcnt range");

    u32x4 ga[TM + 1] = {}, gb[2][TN] = {};
    auto tie = [](u32x4 &v) { asm volatile("" : "+v"(v)); };
    auto tie_all = [&]() {
#pragma unroll
      for (int i = 0; i <= TM; ++i) tie(ga[i]);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        tie(gb[0][j]);
        tie(gb[1][j]);
      }
    };
    // the reads k-step p issues in MFMA group g: fragments of k-step p + 1, at k-step index ksn of
    // the stage at st
    auto reads = [&](auto p_c, auto g_c, const char *st, int ksn) {
      constexpr int p = decltype(p_c)::value, g = decltype(g_c)::value;
      constexpr int n = (p + 1) % (kLast + 1);
      auto rd_a = [&](int i) { opa.frag_to(ga[areg(n, i)], st, wave_m * WTM + i * 32, ksn, lane); };
      if constexpr (g == 0) {
#pragma unroll
        for (int j = 0; j < TN; ++j) opb.frag_to(gb[n & 1][j], st + BM * 128, wave_n * WTN + j * 32, ksn, lane);
        rd_a(0);
        if constexpr (p == kLast) rd_a(TM - 1);
      } else if constexpr (p == kLast) {
        if constexpr (g < TM - 1) rd_a(g);
      } else if constexpr (p == kLast - 1) {
        if constexpr (g < TM - 1) rd_a(g);
        if constexpr (g == TM - 2) rd_a(TM - 1);
      } else {
        rd_a(g);
      }
    };

    if constexpr (AOP::kIsConv) {
      if (kt0 < kt1) {
        const auto tp0 = OpConv<BM, NW>::tap_at(a, walk);
#pragma unroll
        for (int q = 0; q < PA; ++q) opa.issue(ra, smem, q, tp0);
#pragma unroll
        for (int q = 0; q < PB; ++q) opb.issue(rb, smem + BM * 128, q, walk.t * cblocks + walk.cb);
      }
    } else {
      if (kt0 < kt1) issue_all(smem, kmap(kt0));
    }
    wait_vmem();
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN; ++j) gb[0][j] = opb.frag(smem + BM * 128, wave_n * WTN + j * 32, 0, lane);
#pragma unroll
    for (int i = 0; i < TM; ++i) ga[i] = opa.frag(smem, wave_m * WTM + i * 32, 0, lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    tie_all();

    // One K-tile (TAIL: the partial last K-tile, with its first k-step's fragments read: masked at
    // K, no loads, no reads past its last k-step). The barrier before the last k-step also waits
    // for all of this K-tile's fragment reads (the next K-tile's loads overwrite its stage), and,
    // after a partition boundary, for the slot stores issued before the loads. Past the end the
    // last K-tile is reloaded (L2 hits, never computed) instead of a branch.
    auto ktile1 = [&](const int kt, auto tail_c) {
      constexpr bool TAIL = decltype(tail_c)::value;
      const int cur = (kt - kt0) & 1;
      char *nxt = smem + (cur ^ 1) * kStage;
      int kn;
      const char *sa = smem + cur * kStage;
      typename std::conditional<AOP::kIsConv, typename OpConv<BM, NW>::Tap, int>::type tp{};
      if constexpr (AOP::kIsConv) {
        // K-tile min(kt + 1, kt1 - 1) of the visit (past the end the last one is reloaded)
        if (kt + 1 < kt1) OpConv<BM, NW>::advance(a, walk);
        kn = walk.t * cblocks + walk.cb;
        tp = OpConv<BM, NW>::tap_at(a, walk);
      } else {
        kn = kmap(min(kt + 1, kt1 - 1));
      }
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, kLast + 1>([&](auto k_c) {
        constexpr int ks = decltype(k_c)::value;
        constexpr int c = ks & 1;
        const char *rs = ks < kLast ? sa : nxt;
        constexpr int ksn = ks < kLast ? ks + 1 : 0;
        static_for<0, TM>([&](auto i_c) {
          constexpr int i = decltype(i_c)::value;
          constexpr int ar = areg(ks, i);
          if constexpr (TAIL) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            // the lane index taken afresh in each group: the masks are computed where they are used,
            // not all at once ahead of the K-tile (which holds 16 more registers)
            int ln = lane_id();
            asm volatile("" : "+v"(ln));
            tie(ga[ar]);
            if constexpr (AOP::kNeedsTail) ga[ar] = AOP::mask(ga[ar], AOP::frag_k0(kt, ks, ln), a.K);
            if constexpr (i == 0) {
#pragma unroll
              for (int j = 0; j < TN; ++j) {
                tie(gb[c][j]);
                if constexpr (BOP::kNeedsTail) gb[c][j] = BOP::mask(gb[c][j], BOP::frag_k0(kt, ks, ln), a.K);
              }
            }
          } else if constexpr (ks == kLast) {
            if constexpr (i == 0) {
              // the next K-tile has landed and every wave is done reading this K-tile's stage
              asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
              tie_all();
              wait_vmem();
              __syncthreads();
            }
          } else {
            asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(wcount(ks, i)));
            tie(ga[ar]);
            if constexpr (i == 0) {
#pragma unroll
              for (int j = 0; j < TN; ++j) tie(gb[c][j]);
            }
          }
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mfma32x32x16<DT>(ga[ar], gb[c][j], acc[i][j]);
          if constexpr (!TAIL) {
#pragma unroll
            for (int u = 0; u < kPerGroup1; ++u) {
              const int q = (ks * TM + i) * kPerGroup1 + u;
              if (q < PA) {
                if constexpr (AOP::kIsConv)
                  opa.issue(ra, nxt, q, tp);
                else
                  opa.issue(ra, nxt, q, kn);
              } else if (q < PA + PB) {
                opb.issue(rb, nxt + BM * 128, q - PA, kn);
              }
            }
          }
          if constexpr (!TAIL || ks < kLast) reads(k_c, i_c, TAIL ? sa : rs, ksn);
          __builtin_amdgcn_sched_barrier(0);
        });
      });
    };

    int kt = kt0;
    for (;;) {
      const int kstop = SERIAL ? min(split_end, kfull) : kfull;
      for (; kt < kstop; ++kt) ktile1(kt, std::false_type{});
      if constexpr (!SERIAL) {
        break;
      } else {
        if (!at_boundary(kt)) break;
        // The next K-tile's first fragments (in flight) are read again after the boundary: no
        // fragment register is held across it (they hold slot traffic there instead).
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        park();
        const char *st = smem + ((kt - kt0) & 1) * kStage;
        // the lane index taken afresh: addresses shared with the prologue's reads would otherwise
        // be kept (and spilled) across the K loop
        int ln = lane_id();
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          gb[0][j] = opb.frag(st + BM * 128, wave_n * WTN + j * 32, 0, ln);
          asm volatile("" : "=v"(gb[1][j]));  // a fresh value (overwritten before use)
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) ga[i] = opa.frag(st, wave_m * WTM + i * 32, 0, ln);
        asm volatile("" : "=v"(ga[TM]));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        tie_all();
      }
    }
    // the last prefetch (of the partial last K-tile, or of a K-tile never computed) may still be in
    // flight
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    tie_all();
    if constexpr (kAnyTail) {
      // the partial last K-tile, already in LDS (loaded as a next K-tile by the loop, or by the
      // prologue when it is the only one) with its first k-step's fragments read
      if (tail_here) ktile1(kfull, std::true_type{});
    }
  }

  // ---- epilogue. 32x32 accumulator layout: lane l, register r holds row 8*(r/4) + 4*(l/32) + r%4,
  // column l%32 of its block. Adjacent lanes swap one value of each register pair (DPP quad_perm
  // [1,0,3,2]) so every lane then holds two adjacent columns of one row: even lanes row R, odd
  // lanes row R+1. Half the store instructions, each 4 bytes (f16/bf16) or 8 bytes (fp32 partial).
  // The epilogue takes the lane index afresh: nothing it derives from it (columns, bias values,
  // LDS addresses) is computed before the K loop and held, or spilled, across it.
  int lane_e = lane_id();
  asm volatile("" : "+v"(lane_e));
  const bool odd = lane_e & 1;
  const int col_l = (lane_e & 31) & ~1;
  const int row_l = 4 * (lane_e >> 5) + (odd ? 1 : 0);
  const int mw = m0 + wave_m * WTM + row_l, nw = n0 + wave_n * WTN + col_l;
  auto pair = [&](float x0, float x1, float &lo, float &hi) {
    const float send = odd ? x0 : x1;
    const float recv =
        __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, false));
    lo = odd ? recv : x0;
    hi = odd ? x1 : recv;
  };
  // Split-K partials: GEMM only (convolution plans never split K).
  constexpr bool kPartials = !SERIAL && !AOP::kIsConv;
  if (kPartials && a.partial != nullptr) {
    float *P = a.partial + (size_t)split * a.M * a.N;
    const bool vec = (a.N & 1) == 0;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = nw + j * 32;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          float lo, hi;
          pair(acc[i][j][r], acc[i][j][r + 1], lo, hi);
          const int row = mw + i * 32 + 8 * (r >> 2) + (r & 3);
          if (row < a.M) {
            // partials are streamed out once and read once by the second pass: non-temporal
            if (vec && col + 1 < a.N) {
              __builtin_nontemporal_store(f32x2{lo, hi}, (f32x2 *)(P + (size_t)row * a.N + col));
            } else {
              if (col < a.N) __builtin_nontemporal_store(lo, P + (size_t)row * a.N + col);
              if (col + 1 < a.N) __builtin_nontemporal_store(hi, P + (size_t)row * a.N + col + 1);
            }
          }
        }
    }
  } else {
    // The C tile goes through LDS (free after the main loop): each wave parks its WTM x WTN
    // sub-tile there as paired 4-byte writes, then reads it back along rows and stores 16 bytes
    // per lane, so one store instruction writes whole 256-byte row segments (two cache lines)
    // instead of sixteen half lines.
    constexpr int kRowB = WTN * 2;       // bytes per sub-tile row
    constexpr int kChunks = kRowB / 16;  // 16-byte chunks per row
    static_assert(kChunks == 16 || kChunks == 8, "sub-tile width");
    static_assert(NW * WTM * kRowB <= 2 * kStage, "C tile fits the LDS stages");
    // chunk swizzle: the four rows one paired write instruction touches land on disjoint banks
    auto swz = [](int rr) { return kChunks == 16 ? 4 * ((rr & 1) | ((rr >> 1) & 2)) : 4 * ((rr >> 2) & 1); };
    // The last K-tile's loop reloads a K-tile past the end into the idle stage: those loads must
    // have landed before the stages hold the C tile (explicit, not left to the fence's own wait).
    wait_vmem();
    __syncthreads();  // every wave is done reading the last K-tile's fragments
    char *ct = smem + wave * (WTM * kRowB);
    const uint16_t *bias = (const uint16_t *)a.bias;
    // SERIAL: the running sum of the earlier partitions (slot and LDS blocks loaded one accumulator
    // block ahead, register blocks as they are), added in front of the last partition's sum.
    const bool has_slot = SERIAL && parked > 0;
    const uint32_t slot_lane = SERIAL ? slot_lane_at() : 0u;
    f32x4 ring[kSlotRing][4];
    auto in_regs = [](int b) { return b >= kSlotBlocks && b < kSlotBlocks + kRegBlocks; };
    auto fetch = [&](int s, int i, int j) {
      if (has_slot && !in_regs(i + TM * j)) {
        if (kLdsBlocks > 0 && i == TM - 1 && j == TN - 1) {
          // the LDS-resident block (no loads in flight here: ordinary LDS reads)
          const char *lr = smem + 2 * kStage + wave * 4096 + lane_e * 16;
#pragma unroll
          for (int q = 0; q < 4; ++q) ring[s][q] = *(const f32x4 *)(lr + 1024 * q);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) ring[s][q] = slot_load(slot_lane, i, j, q);
        }
      }
    };
    if constexpr (SERIAL) {
#pragma unroll
      for (int b = 0; b + 1 < kSlotRing; ++b) fetch(b, b % TM, b / TM);
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int own = nw + j * 32 + (odd ? 1 : 0);  // the column this lane's accumulators belong to
      const float bv = (a.has_bias && own < a.N) ? from_bits<DT>(bias[own]) : 0.0f;
      const int cc = col_l + j * 32;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int b = j * TM + i;  // block index (fetch order)
        float x[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = acc[i][j][r];
        if constexpr (SERIAL) {
          constexpr int kAhead = kSlotRing - 1;
          if (b + kAhead < TM * TN) fetch((b + kAhead) % kSlotRing, (b + kAhead) % TM, (b + kAhead) / TM);
          if (has_slot && in_regs(b)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) x[r] = run[b - kSlotBlocks][r] + x[r];
          } else if (has_slot) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 v = ring[b % kSlotRing][q];
#pragma unroll
              for (int e = 0; e < 4; ++e) x[4 * q + e] = v[e] + x[4 * q + e];
            }
          }
        }
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          float lo, hi;
          pair(x[r] + bv, x[r + 1] + bv, lo, hi);
          const int rr = row_l + i * 32 + 8 * (r >> 2) + (r & 3);
          *(uint32_t *)(ct + rr * kRowB + (((cc >> 3) ^ swz(rr)) << 4) + (cc & 7) * 2) = pack2<DT>(lo, hi);
        }
        if constexpr (SERIAL) __builtin_amdgcn_sched_barrier(0);
      }
    }
    uint16_t *C = (uint16_t *)a.C;
    const bool v16 = (a.ldc & 7) == 0 && ((uintptr_t)a.C & 15) == 0;
    const int gr0 = m0 + wave_m * WTM, gc0 = n0 + wave_n * WTN;
    constexpr int kRowsPerInst = 64 / kChunks;
#pragma unroll 4
    for (int it = 0; it < WTM / kRowsPerInst; ++it) {
      const int rr = it * kRowsPerInst + lane_e / kChunks, ch = lane_e % kChunks;
      const u32x4 v = *(const u32x4 *)(ct + rr * kRowB + ((ch ^ swz(rr)) << 4));
      const int grow = gr0 + rr, gcol = gc0 + 8 * ch;
      if (grow < a.M) {
        uint16_t *dst = C + (size_t)grow * a.ldc + gcol;
        if (v16 && gcol + 8 <= a.N) {
          *(u32x4 *)dst = v;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = v[e >> 1];
            if (gcol + e < a.N) dst[e] = (uint16_t)((e & 1) ? (w >> 16) : (w & 0xffffu));
          }
        }
      }
    }
  }
}

}  // namespace mtk
