// Device-side helpers shared by the gfx950 kernels: vector types, raw buffer
// loads (out-of-range offsets read as zero, never fault), MFMA wrappers and
// fp16/bf16 packing. CDNA4 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kargs.h"

// Every code object records the kernel-argument contract it was built against; the runtime
// refuses to load one whose version differs from its own (a stale build would read its argument
// blocks and workspaces with the wrong layout).
extern "C" __attribute__((used)) __device__ const int32_t mtk_kargs_version = MTK_KARGS_VERSION;

namespace mtk {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Note: __builtin_bit_cast applied directly to a vector element (v.y, w[2]) reads element 0 with
// this compiler (ROCm 7.2 clang); copy the element to a scalar first or load a vector of the
// wanted element type.

enum { DT_F16 = 0, DT_BF16 = 1 };

// A byte offset that is past every buffer range this library creates (ranges are
// capped at 2^31 - 256 bytes on the host), so a load from it returns zeros.
constexpr uint32_t kOOB = 0x7fffff00u;

// Word 3 of a gfx9-family buffer descriptor: raw (untyped) 32-bit data format.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, kRsrcWord3);
}

__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ u32x2 buf_load8(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load2(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// 32x32x16 MFMA, fp32 accumulate. The operands carry 8 packed 16-bit values per lane.
template <int DT>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == DT_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == DT_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
}

// fp32 -> 16-bit storage, round to nearest even (hardware conversions).
template <int DT>
__device__ __forceinline__ uint16_t to_bits(float x) {
  if constexpr (DT == DT_F16) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  } else {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
}

template <int DT>
__device__ __forceinline__ float from_bits(uint32_t h) {
  if constexpr (DT == DT_F16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  } else {
    return __builtin_bit_cast(float, h << 16);
  }
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  // written as one vector conversion: gfx950's v_cvt_pk_{f16,bf16}_f32 (round to nearest even,
  // as to_bits) converts the pair in one instruction
  if constexpr (DT == DT_F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, h2{(_Float16)lo, (_Float16)hi});
  } else {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, b2{(__bf16)lo, (__bf16)hi});
  }
}

// max(a, b, c) in one gfx950 v_maximum3_f32 (IEEE maximum: a NaN operand gives NaN). fmaxf on
// values the compiler cannot prove canonical (MFMA results) is lowered with a quieting
// v_max_f32 x, x per operand before v_max3_f32. A compiler-visible operation, not inline asm: the
// compiler must see the read of MFMA results to insert the wait states it needs.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// v_perm_b32 byte selectors: low 16 bits of x, y -> (x.lo | y.lo << 16); high halves likewise.
__device__ __forceinline__ uint32_t pack_lo(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x05040100u); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t x, uint32_t y) { return __builtin_amdgcn_perm(y, x, 0x07060302u); }

// ---------------------------------------------------------------- LDS staging and reads

// gfx950 direct-to-LDS load (buffer_load_dwordx4 ... lds): lane l of the wave writes the 16 bytes
// at buffer offset `off` to LDS byte lds + 16 * l (one instruction fills 1 KB). Out-of-range
// offsets write zeros.
__device__ __forceinline__ void lds_direct16(rsrc_t r, char *lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, off, 0, 0, 0);
}

// This lane's index in its wavefront, computed afresh (mbcnt), not derived from threadIdx: code
// after a long loop that takes it from here holds nothing lane-specific across the loop. Inline
// asm, so that the compiler neither merges the calls into one value (which it then kept, and
// spilled, across the loop) nor hoists them.
__device__ __forceinline__ int lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Wait until every vector-memory load of this wave has completed, direct-to-LDS ones included.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const char *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}

// ds_read_b64_tr_b16 as inline asm. The compiler's wait insertion cannot tell the transposed-read
// builtin apart from in-flight direct-to-LDS writes and would wait for all of them (vmcnt(0))
// before every read; callers of this form wait for the read themselves with lgkm_wait0.
// In each 16-lane group, lane s addresses row k0 + s/4, columns 4*(s%4) .. of a 16-column block of
// 16-bit elements; lane s receives column s of that block at rows k0 .. k0+3.
__device__ __forceinline__ u32x2 ds_read_tr16(const char *p) {
  u32x2 w;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(w) : "v"(lds_addr(p)));
  return w;
}

// The same read at LDS byte address addr + OFF (OFF folded into the instruction's offset field).
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr16_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x2 w;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(w) : "v"(addr), "i"(OFF));
  return w;
}

// ds_read_b128 as inline asm at LDS byte address addr + OFF: like the transposed reads above, for
// code that keeps direct-to-LDS loads in flight while it reads other LDS data (the compiler would
// otherwise make every read wait for them); the caller waits with lgkm_wait0.
template <int OFF>
__device__ __forceinline__ u32x4 ds_read_b128_at(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x4 w;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(w) : "v"(addr), "i"(OFF));
  return w;
}

// The same read into the registers that hold dst (an in/out operand: the compiler keeps the new
// value where the old one was, e.g. a fragment re-read right after its last use).
template <int OFF>
__device__ __forceinline__ void ds_read_b128_into(u32x4 &dst, uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "+v"(dst) : "v"(addr), "i"(OFF));
}

// 16-byte LDS read / write as inline asm at a byte address (the caller waits for the read with an
// lgkmcnt wait that carries its registers), for code that keeps direct-to-LDS loads in flight.
__device__ __forceinline__ u32x4 lds_rd128(uint32_t addr) {
  u32x4 w;
  asm volatile("ds_read_b128 %0, %1" : "=v"(w) : "v"(addr));
  return w;
}
__device__ __forceinline__ void lds_wr128(uint32_t addr, u32x4 v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

// Direct-to-LDS load with a uniform scalar offset added to the per-lane offset. The buffer range
// check does not cover the scalar part: only for ranges known to lie inside the buffer.
__device__ __forceinline__ void lds_direct16_s(rsrc_t r, char *lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voff, soff, 0, 0);
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = B .. E-1.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Wait for every outstanding LDS read and hand registers filled by inline-asm reads on to their
// consumers through this wait: they are in/out operands, so no use can be scheduled above it.
template <int N>
__device__ __forceinline__ void lgkm_wait0(u32x4 (&f)[N]) {
  if constexpr (N == 1) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]));
  } else if constexpr (N == 2) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]));
  } else if constexpr (N == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));
  } else {
    static_assert(N == 8, "fragment count");
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]),
                   "+v"(f[7]));
  }
}

// Workgroup id remap so that consecutive logical ids share an XCD: hardware hands
// workgroup b to XCD (b % 8); XCD x receives its ids in order, so logical id =
// (ids owned by XCDs before x) + (b / 8). A bijection on [0, n).
// Combine a lane's value with lane ^ 32's without going through LDS (v_permlane32_swap: the two
// halves of the wave trade places). Both halves compute (lower half's value) op (upper half's), so
// they get identical results. The elements are copied to scalars before the bit casts (see the
// note on __builtin_bit_cast above).
__device__ __forceinline__ void half_swap(float x, float &lo, float &hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  const uint32_t r0 = r[0], r1 = r[1];  // lanes < 32: (x, x[lane + 32]); lanes >= 32: (x[lane - 32], x)
  lo = __builtin_bit_cast(float, r0);
  hi = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float half_max(float x) {
  float lo, hi;
  half_swap(x, lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float half_sum(float x) {
  float lo, hi;
  half_swap(x, lo, hi);
  return lo + hi;
}

__device__ __forceinline__ int xcd_remap(int b, int n) {
  const int q = n >> 3, r = n & 7, x = b & 7;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + (b >> 3);
}

// Causal attention grids: blocks of unequal work (query blocks near the end of the sequence see
// more keys; key blocks near its start are seen by more queries). Workgroup id (after xcd_remap,
// so an XCD holds a contiguous id range) -> (batch-head pair bh, rank), rank 0 = the pair's
// heaviest block. Ids run over groups of kCausalGroup pairs, each group's blocks heaviest first
// and interleaved across its pairs: each XCD then starts its longest blocks first (list
// scheduling in that order balances the unequal blocks) while it works on the K/V of about
// kCausalGroup pairs at a time (L2 reuse). With every pair's blocks heaviest first but pair after
// pair, an XCD's last pairs started late and ran their longest blocks alone at the end.
// Groups of 4 measured best (2 and 8: the same or slower; 16: 13 % slower).
constexpr int kCausalGroup = 4;
__device__ __forceinline__ void causal_order(int id, int nblk, int nbh, int &bh, int &rank) {
  const int g0 = (id / (kCausalGroup * nblk)) * kCausalGroup;
  const int gn = min(kCausalGroup, nbh - g0);
  const int r = id - g0 * nblk;
  bh = g0 + r % gn;
  rank = r / gn;
}

}  // namespace mtk
