// Host runtime behind include/mtk.h: device/context, code-object modules, kernel-select
// (plans), launches through hipModuleLaunchKernel, event timing and error reporting.
//
// The reference builds a Metal pipeline per shape by generating MSL source and JIT compiling it
// (Sources/matmul/matmul.swift:364-390). Here every kernel is compiled ahead of time by
// `hipcc --genco --offload-arch=gfx950` into mtk_*.hsaco code objects; a plan picks one of the
// template instantiations by name and fixes its grid and argument block.
//
// Plans may be created with ctx == NULL ("dry" plans): the descriptor is validated and the
// kernel-select is made, but nothing is resolved on a device. That keeps the selection logic
// testable on machines without a GPU; running a dry plan is an error.
#include <dirent.h>
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/mtk.h"
#include "kargs.h"
#include "scratch.h"

namespace {

thread_local std::string g_last_error = "no error";

int fail(int status, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

#define HIP_TRY(expr)                                                                       \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess) return fail(MTK_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

constexpr uint64_t kMaxOperandBytes = (1ull << 31) - 256;  // buffer-resource ranges (see device.hpp)
constexpr int kAutoKStagger = 16;  // in-workgroup split-K: boundary offsets span up to 16 K-tiles
constexpr int kMaxHeadDim = MTK_ATTN_MAX_HEAD_DIM;  // largest padded head dimension compiled (512)

}  // namespace

struct mtk_ctx {
  int device = 0;
  hipDeviceProp_t prop{};
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  std::vector<hipModule_t> modules;
  std::map<std::string, hipFunction_t> functions;

  int function(const std::string &name, hipFunction_t *f) {
    auto it = functions.find(name);
    if (it != functions.end()) {
      *f = it->second;
      return MTK_OK;
    }
    for (hipModule_t m : modules) {
      hipFunction_t fn = nullptr;
      if (hipModuleGetFunction(&fn, m, name.c_str()) == hipSuccess && fn) {
        functions[name] = fn;
        *f = fn;
        return MTK_OK;
      }
      // a miss in one module is expected; leave no sticky error for the caller's next HIP call
      (void)hipGetLastError();
    }
    return fail(MTK_ERR_MODULE, "kernel %s not found in the loaded code objects", name.c_str());
  }
};

namespace {

enum PlanKind { PLAN_GEMM = 1, PLAN_ATTN = 2, PLAN_CONV = 3, PLAN_ATTN_BWD = 4, PLAN_PERMUTE = 5 };

enum LaunchRole { ROLE_MAIN = 0, ROLE_REDUCE = 1, ROLE_PERMUTE = 2 };

struct Launch {
  std::string name;
  hipFunction_t fn = nullptr;
  unsigned grid = 1, block = 256;
  LaunchRole role = ROLE_MAIN;
  std::vector<char> args;  // kernel argument block (one struct, by value)
};

}  // namespace

struct mtk_plan {
  mtk_ctx *ctx = nullptr;
  PlanKind kind = PLAN_GEMM;
  mtk_gemm_desc gemm{};
  mtk_attn_desc attn{};
  mtk_conv_desc conv{};
  mtk_permute_desc perm{};
  std::vector<Launch> launches;
  size_t workspace = 0;
  size_t weight_bytes = 0;            // conv: exact byte extent of w (its workspace copy is rounded up)
  bool serial_split = false;          // GEMM split-K run in-workgroup (C written by the main kernel)
  unsigned align_a = 2, align_b = 2;  // required operand alignments (bytes)
  double flops = 0, bytes = 0;
  std::string description;
};

namespace {

int resolve(mtk_plan *p) {
  if (!p->ctx) return MTK_OK;
  for (auto &l : p->launches) {
    int s = p->ctx->function(l.name, &l.fn);
    if (s != MTK_OK) return s;
  }
  return MTK_OK;
}

template <typename T>
void set_args(Launch &l, const T &a) {
  l.args.resize(sizeof(T));
  memcpy(l.args.data(), &a, sizeof(T));
}

template <typename T>
T &args_of(Launch &l) {
  return *reinterpret_cast<T *>(l.args.data());
}

int launch_all(const mtk_plan *p, std::vector<Launch> &ls, hipEvent_t *evs) {
  hipStream_t s = p->ctx->stream;
  if (evs) HIP_TRY(hipEventRecord(evs[0], s));
  for (size_t i = 0; i < ls.size(); ++i) {
    Launch &l = ls[i];
    void *params[] = {l.args.data()};
    hipError_t e = hipModuleLaunchKernel(l.fn, l.grid, 1, 1, l.block, 1, 1, 0, s, params, nullptr);
    if (e != hipSuccess) return fail(MTK_ERR_LAUNCH, "launch of %s failed: %s", l.name.c_str(), hipGetErrorString(e));
    if (evs) HIP_TRY(hipEventRecord(evs[i + 1], s));
  }
  return MTK_OK;
}

int pow2_vec(std::initializer_list<long long> values) {
  for (int v : {8, 4, 2}) {
    bool ok = true;
    for (long long x : values) ok = ok && (x % v == 0);
    if (ok) return v == 2 ? 1 : v;  // 2-wide loads are served by the scalar path
  }
  return 1;
}

bool aligned(const void *p, unsigned a) { return ((uintptr_t)p % a) == 0; }

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  if (exp == 0) return (sign ? -1.0f : 1.0f) * std::ldexp((float)mant, -24);
  const uint32_t u = exp == 31 ? (sign | 0x7f800000u | (mant << 13)) : (sign | ((exp + 112u) << 23) | (mant << 13));
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// ------------------------------------------------------------------ GEMM planning

int plan_gemm(mtk_ctx *ctx, const mtk_gemm_desc *d_in, mtk_plan **out) {
  if (!d_in || !out) return fail(MTK_ERR_INVALID, "null descriptor or output");
  mtk_gemm_desc d = *d_in;
  if (d.M <= 0 || d.N <= 0 || d.K <= 0) return fail(MTK_ERR_INVALID, "M, N, K must be positive (got %d, %d, %d)", d.M, d.N, d.K);
  if (d.dtype != MTK_F16 && d.dtype != MTK_BF16) return fail(MTK_ERR_INVALID, "GEMM dtype must be MTK_F16 or MTK_BF16");
  d.trans_a = d.trans_a ? 1 : 0;
  if (d.lda == 0) d.lda = d.trans_a ? d.M : d.K;
  if (d.ldb == 0) d.ldb = d.trans_b ? d.K : d.N;
  if (d.ldc == 0) d.ldc = d.N;
  if (d.lda < (d.trans_a ? d.M : d.K)) return fail(MTK_ERR_INVALID, "lda (%d) too small", d.lda);
  if (d.trans_a && d.lda % 2 != 0)
    return fail(MTK_ERR_UNSUPPORTED, "trans_a needs an even lda (4-byte aligned rows of A [K][lda])");
  if (d.ldb < (d.trans_b ? d.K : d.N)) return fail(MTK_ERR_INVALID, "ldb (%d) too small", d.ldb);
  if (d.ldc < d.N) return fail(MTK_ERR_INVALID, "ldc (%d) < N (%d)", d.ldc, d.N);
  if (d.split_k < 0) return fail(MTK_ERR_INVALID, "split_k must be >= 0");
  if (d.tile != 0 && d.tile != 128 && d.tile != 256) return fail(MTK_ERR_INVALID, "tile must be 0, 128 or 256");
  if (d.k_stagger < -1) return fail(MTK_ERR_INVALID, "k_stagger must be >= -1 (got %d)", d.k_stagger);
  if (d.split_mode < MTK_SPLIT_AUTO || d.split_mode > MTK_SPLIT_SERIAL)
    return fail(MTK_ERR_INVALID, "split_mode must be MTK_SPLIT_AUTO, MTK_SPLIT_TWO_PASS or MTK_SPLIT_SERIAL");
  // Buffer ranges end on a whole dword: raw buffer loads range-check per dword, so a last element
  // in the low half of a straddling dword would read as zero. The at most 2 extra bytes lie in the
  // same aligned dword (same page) as the operand's last element; they are masked in the kernels.
  const uint64_t a_rows = d.trans_a ? d.K : d.M, a_cols = d.trans_a ? d.M : d.K;
  const uint64_t a_bytes = (((a_rows - 1) * (uint64_t)d.lda + a_cols) * 2 + 3) & ~3ull;
  const uint64_t b_rows = d.trans_b ? d.N : d.K, b_cols = d.trans_b ? d.K : d.N;
  const uint64_t b_bytes = (((b_rows - 1) * (uint64_t)d.ldb + b_cols) * 2 + 3) & ~3ull;
  if (a_bytes > kMaxOperandBytes || b_bytes > kMaxOperandBytes)
    return fail(MTK_ERR_UNSUPPORTED, "operands above 2 GiB are not supported by this build");

  mtk_plan *p = new mtk_plan();
  p->ctx = ctx;
  p->kind = PLAN_GEMM;
  p->gemm = d;
  const char *dt = d.dtype == MTK_F16 ? "f16" : "bf16";
  const int k_tiles = (d.K + 63) / 64;
  p->flops = 2.0 * d.M * d.N * d.K;
  p->bytes = 2.0 * ((double)d.M * d.K + (double)d.N * d.K + (double)d.M * d.N + (d.has_bias ? d.N : 0));

  // Decode-shaped problems (M <= 16, B [N][K]) go to the HBM-streaming skinny kernel; its
  // split-K partitions are wavefronts of one workgroup, reduced on chip with the bias fused. The
  // grid is persistent: one workgroup per CU walking the 16-column groups. Partitions longer than
  // the 512 K whose A fragments stay in registers go, when K >= 2048 and there are at least two,
  // to the partial-writing kernel below with the same partition count (16 x 4096 x 14336, split-K
  // 8: 25 us there against 41 us on the long-partition kernel, which remains for the rest).
  int decode_parts_split = 0;
  if (d.M <= 16 && !d.trans_a && d.trans_b && d.tile == 0 && d.K % 8 == 0 && d.lda % 8 == 0 && d.ldb % 8 == 0) {
    int split = d.split_k == 0 ? (d.K >= 1024 ? 8 : std::max(1, d.K / 128)) : d.split_k;
    split = std::max(1, std::min(split, 8));
    int kps = ((d.K + split - 1) / split + 31) / 32 * 32;
    split = (d.K + kps - 1) / kps;
    if (kps > 512 && split >= 2 && d.K >= 2048 && d.split_mode != MTK_SPLIT_SERIAL) decode_parts_split = split;
  }
  if (d.M <= 16 && !decode_parts_split && !d.trans_a && d.trans_b && d.tile == 0 && d.K % 8 == 0 && d.lda % 8 == 0 &&
      d.ldb % 8 == 0) {
    int split = d.split_k == 0 ? (d.K >= 1024 ? 8 : std::max(1, d.K / 128)) : d.split_k;
    split = std::max(1, std::min(split, 8));
    int kps = ((d.K + split - 1) / split + 31) / 32 * 32;
    split = (d.K + kps - 1) / kps;
    const long long groups = (d.N + 15) / 16;
    const int cus = ctx ? ctx->prop.multiProcessorCount : 256;
    Launch g;
    // partitions of up to 512 K keep their A fragments in registers for the whole kernel; with at
    // most four 16-column groups per workgroup and split-K >= 4 every group keeps its own LDS slot
    // and the workgroup reduces once, at the end ("few")
    g.grid = (unsigned)std::min<long long>(groups, cus);
    const long long per_wg = (d.N + g.grid - 1) / g.grid;
    const bool few = kps <= 512 && split >= 4 && (per_wg + 15) / 16 <= 4;
    g.name = std::string("mtk_skinny_") + (few ? "few_" : "") + dt + (kps <= 512 ? "" : "_long");
    g.block = (unsigned)(64 * split);
    mtk_skinny_args a{};
    a.M = d.M;
    a.N = d.N;
    a.K = d.K;
    a.lda = d.lda;
    a.ldb = d.ldb;
    a.ldc = d.ldc;
    a.a_bytes = (uint32_t)a_bytes;
    a.b_bytes = (uint32_t)b_bytes;
    a.split_k = split;
    a.k_per_split = kps;
    a.has_bias = d.has_bias ? 1 : 0;
    set_args(g, a);
    p->launches.push_back(g);
    p->align_a = p->align_b = 16;
    char desc[256];
    snprintf(desc, sizeof desc,
             "gemm %s skinny M=%d N=%d K=%d split_k=%d (k/split=%d, reduced in LDS, bias fused) grid=%u block=%u", dt,
             d.M, d.N, d.K, split, kps, g.grid, g.block);
    p->description = desc;
    int s = resolve(p);
    if (s != MTK_OK) {
      delete p;
      return s;
    }
    *out = p;
    return MTK_OK;
  }

  // 16 < M <= 32 with long K (the reference's default run, 32 x 3072 x 80000, split-K 30), and
  // M <= 16 with partitions longer than 512 K (above): B streamed once by the partial-writing
  // skinny kernel, one workgroup per (K partition, 64 columns), then the two-pass reduce. Same partition layout as the two-pass tile schedule
  // (uniform partitions of whole 64-element K-tiles); needs split_k >= 2 after the plan's choice.
  if ((decode_parts_split || (d.M > 16 && d.M <= 32)) && !d.trans_a && d.trans_b && d.tile == 0 &&
      d.split_mode != MTK_SPLIT_SERIAL && d.K >= 2048 && d.K % 8 == 0 && d.lda % 8 == 0 && d.ldb % 8 == 0) {
    const int cus = ctx ? ctx->prop.multiProcessorCount : 256;
    const long long ncb = (d.N + 63) / 64;
    int split = decode_parts_split ? decode_parts_split : d.split_k;
    if (split == 0)  // about four workgroups per CU, partitions of at least 8 K-tiles
      split = (int)std::min<long long>(std::max<long long>(2, (4LL * cus + ncb - 1) / ncb), std::max(1, k_tiles / 8));
    split = std::min(split, k_tiles);
    const int kps = (k_tiles + split - 1) / split;
    split = (k_tiles + kps - 1) / kps;
    if (split >= 2) {
      Launch g;
      g.name = std::string("mtk_skinny_parts_") + dt;
      g.grid = (unsigned)(ncb * split);
      g.block = 256;
      mtk_skinny_args a{};
      a.M = d.M;
      a.N = d.N;
      a.K = d.K;
      a.lda = d.lda;
      a.ldb = d.ldb;
      a.ldc = d.ldc;
      a.a_bytes = (uint32_t)a_bytes;
      a.b_bytes = (uint32_t)b_bytes;
      a.split_k = split;
      a.k_per_split = kps * 64;
      a.has_bias = d.has_bias ? 1 : 0;
      set_args(g, a);
      p->launches.push_back(g);
      p->workspace = (size_t)split * d.M * d.N * sizeof(float);
      Launch r;
      r.role = ROLE_REDUCE;
      r.name = std::string("mtk_splitk_reduce_") + dt;
      mtk_reduce_args ra{};
      ra.M = d.M;
      ra.N = d.N;
      ra.ldc = d.ldc;
      ra.split_k = split;
      ra.has_bias = a.has_bias;
      // more than 8 partials over an output of fewer than 4 x 256 elements per CU: one output per
      // thread, so that more workgroups keep partial loads in flight (the reference's run: 30
      // partials of 32 x 3072, the scalar reduce ~2 us faster than four outputs per thread)
      const bool few_outputs = split > 8 && (long long)d.M * d.N < 4LL * 256 * cus;
      ra.vec4 = (d.N % 4 == 0 && d.ldc % 4 == 0 && !few_outputs) ? 1 : 0;
      const long long work = ra.vec4 ? (long long)d.M * d.N / 4 : (long long)d.M * d.N;
      r.grid = (unsigned)std::min<long long>((work + 255) / 256, 65535);
      set_args(r, ra);
      p->launches.push_back(r);
      p->align_a = p->align_b = 16;
      char desc[256];
      snprintf(desc, sizeof desc,
               "gemm %s skinny partials M=%d N=%d K=%d split_k=%d k_tiles/split=%d grid=%u block=256 + splitk_reduce", dt,
               d.M, d.N, d.K, split, kps, g.grid);
      p->description = desc;
      int st = resolve(p);
      if (st != MTK_OK) {
        delete p;
        return st;
      }
      *out = p;
      return MTK_OK;
    }
  }

  int tile = d.tile;
  int split = d.split_k;
  if (tile == 0) {
    // 256x256 tiles when there are enough of them (with the requested split) to fill most of the
    // device, unless M or N fits a 128 tile: a 256 tile would then compute mostly padding. Below
    // that, 128x128 tiles at two workgroups per CU (one box, split-K 1, K = 4096: 128 tiles of
    // 256x256, 2048x4096, 91.4 us on 256x256 against 79.9 us on 128x128; 192 tiles 115.4 against
    // 127.8 us; 64 tiles 144.3 against 95.3 us).
    const long long t256 = (long long)((d.M + 255) / 256) * ((d.N + 255) / 256);
    tile = (t256 * std::max(split, 1) >= 160 && d.M > 128 && d.N > 128) ? 256 : 128;
  }
  const int tiles_m = (d.M + tile - 1) / tile, tiles_n = (d.N + tile - 1) / tile;
  const long long tiles = (long long)tiles_m * tiles_n;
  if (split == 0) {  // fill about one wave of 256 CUs with split-K when the tile grid is small
    split = 1;
    if (tiles < 192) split = (int)std::min<long long>(std::max<long long>(1, 256 / tiles), std::max(1, k_tiles / 4));
    split = std::min(split, 16);
  }
  split = std::min(split, k_tiles);
  const int kps = (k_tiles + split - 1) / split;
  split = (k_tiles + kps - 1) / kps;  // no empty splits

  // Operand rows 4-byte aligned (even leading dimensions): the direct-to-LDS pipeline, with B
  // [N][K] read as row fragments or B [K][N] read through transposed LDS loads (16-byte loads
  // need only dword alignment; a K tail that is not a multiple of 8 is loaded element-wise).
  // Odd leading dimensions: the register-staged kernel with 2-byte loads.
  const bool direct = d.lda % 2 == 0 && d.ldb % 2 == 0;
  p->align_a = p->align_b = direct ? 4 : 2;

  // Split-K scheduling. In-workgroup ("serial"): one workgroup per tile walks the partitions in
  // sequence and parks split-1 fp32 partition sums per tile; worth it when the tile grid alone
  // fills the device (every CU busy without extra partition workgroups), and it saves the second
  // kernel and 1/split of the partial traffic.
  bool serial = false;
  if (split > 1) {
    const int cus = ctx ? ctx->prop.multiProcessorCount : 256;
    if (d.split_mode == MTK_SPLIT_SERIAL) {
      if (split > 4 || !direct) {
        delete p;
        return fail(MTK_ERR_UNSUPPORTED, "in-workgroup split-K needs split_k <= 4 and even leading dimensions");
      }
      serial = true;
    } else if (d.split_mode == MTK_SPLIT_AUTO) {
      serial = direct && split <= 4 && tiles * 4 >= 3LL * cus;
    }
  }
  p->serial_split = serial;

  Launch g;
  char name[96];
  // operand letters: A [M][K] 'n' / [K][M] 't', B [N][K] 't' / [K][N] 'n'
  snprintf(name, sizeof name, "mtk_gemm_%s_%c%c_%dx%d_%s", dt, d.trans_a ? 't' : 'n', d.trans_b ? 't' : 'n', tile, tile,
           serial ? "s" : direct ? "d" : "v1");
  g.name = name;
  if (tile == 256 && direct) g.block = 512;  // 256x256 direct-to-LDS tiles run 8 wavefronts
  g.grid = (unsigned)(serial ? tiles : tiles * split);
  mtk_tile_args a{};
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  a.a_bytes = (uint32_t)a_bytes;
  a.b_bytes = (uint32_t)b_bytes;
  a.tiles_m = tiles_m;
  a.tiles_n = tiles_n;
  a.k_tiles = k_tiles;
  a.k_tiles_per_split = kps;
  a.split_k = split;
  a.has_bias = d.has_bias ? 1 : 0;
  // Staggered partition boundaries (per-tile offsets in [-S/2, S/2)): with every tile ending a
  // partition at the same K-tile, all workgroups of the in-workgroup schedule write their running
  // sums in one burst. The span keeps the first partition and the last (which may be shorter)
  // non-empty. The two-pass schedule keeps uniform partitions by default: there every partition
  // is its own workgroup and uneven ones would unbalance the grid.
  if (split > 1 && d.k_stagger >= 0) {
    const int last = k_tiles - (split - 1) * kps;
    int span = std::min(2 * (kps - 1), 2 * last);
    span = std::min(span, d.k_stagger > 0 ? d.k_stagger : serial ? kAutoKStagger : 0);
    a.k_stagger = span >= 2 ? span & ~1 : 0;
  }
  set_args(g, a);
  p->launches.push_back(g);
  if (serial) {
    p->workspace = (size_t)tiles * MTK_SERIAL_SLOT_BYTES(tile);  // each tile's running-sum slot
  } else if (split > 1) {
    p->workspace = (size_t)split * d.M * d.N * sizeof(float);
    Launch r;
    r.role = ROLE_REDUCE;
    r.name = std::string("mtk_splitk_reduce_") + dt;
    mtk_reduce_args ra{};
    ra.M = d.M;
    ra.N = d.N;
    ra.ldc = d.ldc;
    ra.split_k = split;
    ra.has_bias = a.has_bias;
    // as for the partial-writing kernel: many partials over a small output, one output per thread
    const int cus_r = ctx ? ctx->prop.multiProcessorCount : 256;
    const bool few_outputs = split > 8 && (long long)d.M * d.N < 4LL * 256 * cus_r;
    ra.vec4 = (d.N % 4 == 0 && d.ldc % 4 == 0 && !few_outputs) ? 1 : 0;
    const long long work = ra.vec4 ? (long long)d.M * d.N / 4 : (long long)d.M * d.N;
    r.grid = (unsigned)std::min<long long>((work + 255) / 256, 65535);
    set_args(r, ra);
    p->launches.push_back(r);
  }
  char desc[320];
  snprintf(desc, sizeof desc,
           "gemm %s %s %s M=%d N=%d K=%d tile=%dx%d split_k=%d k_tiles/split=%d k_stagger=%d %s grid=%u%s", dt,
           d.trans_a ? "A[K][M]" : "A[M][K]", d.trans_b ? "B[N][K]" : "B[K][N]", d.M, d.N, d.K, tile, tile, split, kps,
           a.k_stagger, direct ? "direct-to-LDS" : "2-byte loads", g.grid,
           serial ? " (partitions in sequence per tile, summed in the epilogue)" : split > 1 ? " + splitk_reduce" : "");
  p->description = desc;
  int s = resolve(p);
  if (s != MTK_OK) {
    delete p;
    return s;
  }
  *out = p;
  return MTK_OK;
}

// Attention backward: D-term pass, then dK/dV (one workgroup per 128 keys) and dQ (one per 256
// queries), all reading the forward's lse; the D vector lives in the plan's workspace.
int plan_attn_bwd(mtk_ctx *ctx, const mtk_attn_desc *d_in, mtk_plan **out) {
  if (!d_in || !out) return fail(MTK_ERR_INVALID, "null descriptor or output");
  mtk_attn_desc d = *d_in;
  if (d.B <= 0 || d.H <= 0 || d.S_q <= 0 || d.S_kv <= 0) return fail(MTK_ERR_INVALID, "B, H, S_q, S_kv must be positive");
  if (d.H_kv == 0) d.H_kv = d.H;
  if (d.H_kv < 0 || d.H % d.H_kv != 0)
    return fail(MTK_ERR_INVALID, "H_kv must divide H (got H=%d, H_kv=%d)", d.H, d.H_kv);
  if (d.D <= 0 || d.D > 256 || d.D % 8 != 0)
    return fail(MTK_ERR_UNSUPPORTED, "backward head dimension must be a multiple of 8 up to 256 (got %d)", d.D);
  // D <= 128: the 32-key / 32-query wavefront kernels, laid out for 64 (D <= 64) or 128 (chunks
  // past D are zeros); 128 < D <= 256: the 16-key / 16-query wavefront kernels laid out for 256
  const bool wide = d.D > 128;
  const char *lay = d.D <= 64 ? "d64_" : "";
  if (d.dtype != MTK_F16 && d.dtype != MTK_BF16) return fail(MTK_ERR_INVALID, "attention dtype must be MTK_F16 or MTK_BF16");
  if (d.q_rows != 0) return fail(MTK_ERR_INVALID, "the backward plan chooses its own blocking (q_rows must be 0)");
  const uint64_t q_bytes = (uint64_t)d.B * d.S_q * d.H * d.D * 2;
  const uint64_t kv_bytes = (uint64_t)d.B * d.S_kv * d.H_kv * d.D * 2;
  if (q_bytes > kMaxOperandBytes || kv_bytes > kMaxOperandBytes)
    return fail(MTK_ERR_UNSUPPORTED, "operands above 2 GiB are not supported by this build");
  mtk_plan *p = new mtk_plan();
  p->ctx = ctx;
  p->kind = PLAN_ATTN_BWD;
  p->attn = d;
  p->align_a = p->align_b = 16;
  const char *dt = d.dtype == MTK_F16 ? "f16" : "bf16";
  const char *cz = d.causal ? "_causal" : "";
  mtk_attn_bwd_kargs a{};
  a.B = d.B;
  a.H = d.H;
  a.H_kv = d.H_kv;
  a.S_q = d.S_q;
  a.S_kv = d.S_kv;
  a.q_blocks = wide ? (d.S_q + 63) / 64 : (d.S_q + 255) / 256;
  a.k_blocks = wide ? (d.S_kv + 63) / 64 : (d.S_kv + 127) / 128;
  a.causal = d.causal ? 1 : 0;
  a.scale = (float)(1.0 / std::sqrt((double)d.D));
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)d.D));
  a.q_bytes = (uint32_t)q_bytes;
  a.kv_bytes = (uint32_t)kv_bytes;
  a.D = d.D;
  Launch pre, kv, q;
  pre.name = std::string("mtk_attn_bwd_pre_") + dt;
  pre.grid = (unsigned)(((long long)d.B * d.S_q * d.H + 15) / 16);
  kv.name = std::string(wide ? "mtk_attn_bwd256_dkdv_" : "mtk_attn_bwd_dkdv_") + (wide ? "" : lay) + dt + cz;
  kv.grid = (unsigned)((long long)a.k_blocks * d.B * d.H_kv);  // per K/V head: sums over its query heads
  q.name = std::string(wide ? "mtk_attn_bwd256_dq_" : "mtk_attn_bwd_dq_") + (wide ? "" : lay) + dt + cz;
  q.grid = (unsigned)((long long)a.q_blocks * d.B * d.H);
  q.block = wide ? 256 : 512;
  for (Launch *l : {&pre, &kv, &q}) {
    set_args(*l, a);
    p->launches.push_back(*l);
  }
  // workspace: the scaled D-term, then the base-2 lse, [B][H][S_q] fp32 each
  p->workspace = 2 * (((size_t)d.B * d.H * d.S_q * sizeof(float) + 255) & ~(size_t)255);
  double pairs = (double)d.S_q * d.S_kv;
  if (d.causal) {
    pairs = 0;
    for (long long i = 0; i < d.S_q; ++i) {
      long long lim = i + (d.S_kv - d.S_q) + 1;
      pairs += (double)std::max(0ll, std::min<long long>(lim, d.S_kv));
    }
  }
  // five products of 2 * pairs * D flops each (S, dP, dV, dK, dQ; the dQ kernel's recomputation of
  // S and dP is not counted); bytes: Q, K, V, O, dO read, dQ, dK, dV written, lse and D
  p->flops = 10.0 * d.B * d.H * d.D * pairs;
  p->bytes = 4.0 * (double)q_bytes + 4.0 * (double)kv_bytes + 3.0 * 4.0 * d.B * d.H * d.S_q;
  char desc[256];
  snprintf(desc, sizeof desc, "attention bwd %s B=%d H=%d H_kv=%d S_q=%d S_kv=%d D=%d causal=%d grids=%u/%u/%u", dt,
           d.B, d.H, d.H_kv, d.S_q, d.S_kv, d.D, d.causal, pre.grid, kv.grid, q.grid);
  p->description = desc;
  int s = resolve(p);
  if (s != MTK_OK) {
    delete p;
    return s;
  }
  *out = p;
  return MTK_OK;
}

// OIDHW -> DHWIO weight re-layout: a tiled transpose of src viewed as [O][C*T] (one workgroup per
// 64 x 64 tile); 16-byte accesses when C*T and O are multiples of 8 (alignment checked at run).
int plan_permute(mtk_ctx *ctx, const mtk_permute_desc *d_in, mtk_plan **out) {
  if (!d_in || !out) return fail(MTK_ERR_INVALID, "null descriptor or output");
  const mtk_permute_desc d = *d_in;
  if (d.O <= 0 || d.C <= 0 || d.KD <= 0 || d.KH <= 0 || d.KW <= 0)
    return fail(MTK_ERR_INVALID, "O, C, KD, KH, KW must be positive");
  const long long T = (long long)d.KD * d.KH * d.KW, CT = T * d.C;
  const uint64_t bytes = (uint64_t)d.O * CT * 2;
  if (bytes > kMaxOperandBytes || CT >= (1ll << 31))
    return fail(MTK_ERR_UNSUPPORTED, "operands above 2 GiB are not supported by this build");
  mtk_plan *p = new mtk_plan();
  p->ctx = ctx;
  p->kind = PLAN_PERMUTE;
  p->perm = d;
  const bool vec = CT % 8 == 0 && d.O % 8 == 0;
  p->align_a = p->align_b = vec ? 16 : 2;
  Launch g;
  g.name = vec ? "mtk_permute_oidhw_dhwio_v8" : "mtk_permute_oidhw_dhwio_v1";
  g.grid = (unsigned)(((d.O + 63) / 64) * ((CT + 63) / 64));
  mtk_permute_args a{};
  a.O = d.O;
  a.C = d.C;
  a.T = (int)T;
  set_args(g, a);
  p->launches.push_back(g);
  p->flops = 0;
  p->bytes = 2.0 * (double)bytes;
  char desc[160];
  snprintf(desc, sizeof desc, "permute OIDHW->DHWIO O=%d C=%d KD=%d KH=%d KW=%d %s grid=%u", d.O, d.C, d.KD, d.KH, d.KW,
           vec ? "16-byte" : "2-byte", g.grid);
  p->description = desc;
  int s = resolve(p);
  if (s != MTK_OK) {
    delete p;
    return s;
  }
  *out = p;
  return MTK_OK;
}

// ------------------------------------------------------------------ conv planning

int conv_out(const mtk_conv_desc *d, int *od, int *oh, int *ow) {
  *od = (d->D + d->pad_front + d->pad_back - ((d->KD - 1) * d->dil_d + 1)) / d->stride_d + 1;
  *oh = (d->H + d->pad_top + d->pad_bottom - ((d->KH - 1) * d->dil_h + 1)) / d->stride_h + 1;
  *ow = (d->W + d->pad_left + d->pad_right - ((d->KW - 1) * d->dil_w + 1)) / d->stride_w + 1;
  return MTK_OK;
}

int normalise_conv(const mtk_conv_desc *in, mtk_conv_desc *d) {
  if (!in) return fail(MTK_ERR_INVALID, "null descriptor");
  *d = *in;
  if (d->rank == 2) {
    d->D = 1;
    d->KD = 1;
    d->stride_d = d->stride_d > 0 ? d->stride_d : 1;
    d->dil_d = d->dil_d > 0 ? d->dil_d : 1;
    if (d->pad_front || d->pad_back) return fail(MTK_ERR_INVALID, "rank-2 convolution has no depth padding");
  } else if (d->rank != 3) {
    return fail(MTK_ERR_INVALID, "rank must be 2 or 3 (got %d)", d->rank);
  }
  if (d->N <= 0 || d->D <= 0 || d->H <= 0 || d->W <= 0 || d->C <= 0 || d->O <= 0)
    return fail(MTK_ERR_INVALID, "N, D, H, W, C, O must be positive");
  if (d->KD <= 0 || d->KH <= 0 || d->KW <= 0) return fail(MTK_ERR_INVALID, "kernel extents must be positive");
  if (d->KD > 32 || d->KH > 32 || d->KW > 32) return fail(MTK_ERR_UNSUPPORTED, "kernel extents above 32 are not supported");
  if (d->stride_d <= 0 || d->stride_h <= 0 || d->stride_w <= 0) return fail(MTK_ERR_INVALID, "strides must be positive");
  if (d->dil_d <= 0 || d->dil_h <= 0 || d->dil_w <= 0) return fail(MTK_ERR_INVALID, "dilations must be positive");
  if (d->pad_front < 0 || d->pad_back < 0 || d->pad_top < 0 || d->pad_bottom < 0 || d->pad_left < 0 || d->pad_right < 0)
    return fail(MTK_ERR_INVALID, "padding must be non-negative");
  if (d->dtype != MTK_F16) return fail(MTK_ERR_INVALID, "convolution dtype must be MTK_F16");
  if (d->weight_layout != MTK_WEIGHTS_DHWIO && d->weight_layout != MTK_WEIGHTS_OIDHW)
    return fail(MTK_ERR_INVALID, "weight_layout must be MTK_WEIGHTS_DHWIO or MTK_WEIGHTS_OIDHW (got %d)",
                d->weight_layout);
  int od, oh, ow;
  conv_out(d, &od, &oh, &ow);
  if (d->D + d->pad_front + d->pad_back < (d->KD - 1) * d->dil_d + 1 || d->H + d->pad_top + d->pad_bottom < (d->KH - 1) * d->dil_h + 1 ||
      d->W + d->pad_left + d->pad_right < (d->KW - 1) * d->dil_w + 1 || od <= 0 || oh <= 0 || ow <= 0)
    return fail(MTK_ERR_INVALID, "kernel larger than the padded input");
  return MTK_OK;
}

int plan_conv(mtk_ctx *ctx, const mtk_conv_desc *d_in, mtk_plan **out) {
  if (!out) return fail(MTK_ERR_INVALID, "null output");
  mtk_conv_desc d;
  int s = normalise_conv(d_in, &d);
  if (s != MTK_OK) return s;
  int od, oh, ow;
  conv_out(&d, &od, &oh, &ow);
  const long long M = (long long)d.N * od * oh * ow;
  const long long K = (long long)d.KD * d.KH * d.KW * d.C;
  const uint64_t x_bytes = (uint64_t)d.N * d.D * d.H * d.W * d.C * 2;
  const uint64_t w_bytes = (uint64_t)K * d.O * 2;
  const uint64_t y_elems = (uint64_t)M * d.O;
  if (x_bytes > kMaxOperandBytes || w_bytes > kMaxOperandBytes || M >= (1ll << 31) || y_elems >= (1ull << 40))
    return fail(MTK_ERR_UNSUPPORTED, "operands above 2 GiB are not supported by this build");

  mtk_plan *p = new mtk_plan();
  p->ctx = ctx;
  p->kind = PLAN_CONV;
  p->conv = d;
  // C % 64 == 0 (every 64-wide K-tile is one filter tap), even O and filter extents <= 10: the
  // direct-to-LDS pipeline (gather with padding as out-of-range loads, weights read transposed).
  // Anything else: the register-staged generic gather.
  const bool fast = (d.C % 64) == 0 && d.O % 2 == 0 && d.KD <= 10 && d.KH <= 10 && d.KW <= 10;
  int va, bm, bn;
  if (fast) {
    va = 8;
    // Fewer than 256 output channels: 128x128 tiles, two workgroups per CU whose K loops run out
    // of phase with each other (config 4b: 71 us against 80 us for one 256x128 workgroup of 4 or
    // 8 wavefronts per CU, same bits).
    if (d.O >= 256) {
      bm = 256;
      bn = 256;
    } else {
      bm = 128;
      bn = 128;
    }
    // Fewer than ~140 tiles of 256x256: 128x128 at two workgroups per CU (one box: 128 tiles,
    // conv2d 2x128x128x256 3x3, 66.2 us on 256x256 against 51.3 us; 144 tiles 124.4 against
    // 140.4 us; 192 tiles 72.4 against 82.5 us).
    if ((M + bm - 1) / bm * ((d.O + bn - 1) / bn) < 140) bm = bn = 128;
  } else {
    va = pow2_vec({d.C, d.O});
    bm = bn = 128;
  }
  p->align_a = fast ? 16 : 2 * va;
  p->align_b = fast ? 4 : 2 * va;
  const char *kind = fast ? "fast" : "gen";
  // OIDHW weights (the reference's PermuteThenTensorOpSession3D, ConvolutionShared.swift:1676-1857):
  // the re-layout kernel writes DHWIO weights into the plan's workspace and the convolution reads
  // them there, both in one run. The weights' own alignment is then the re-layout kernel's.
  const bool oidhw = d.weight_layout == MTK_WEIGHTS_OIDHW;
  if (oidhw) {
    const long long ct = K;  // C * KD * KH * KW
    const bool vec = ct % 8 == 0 && d.O % 8 == 0;
    Launch pm;
    pm.name = vec ? "mtk_permute_oidhw_dhwio_v8" : "mtk_permute_oidhw_dhwio_v1";
    pm.grid = (unsigned)(((d.O + 63) / 64) * ((ct + 63) / 64));
    pm.role = ROLE_PERMUTE;
    mtk_permute_args pa{};
    pa.O = d.O;
    pa.C = d.C;
    pa.T = d.KD * d.KH * d.KW;
    set_args(pm, pa);
    p->launches.push_back(pm);
    p->align_b = vec ? 16 : 2;
    p->workspace = ((size_t)w_bytes + 255) & ~(size_t)255;
  }
  p->weight_bytes = (size_t)w_bytes;
  Launch g;
  char name[96];
  if (fast)
    snprintf(name, sizeof name, "mtk_conv_f16_fast_%dx%d_d", bm, bn);
  else
    snprintf(name, sizeof name, "mtk_conv_f16_gen_%dx%d_v%d", bm, bn, va);
  g.name = name;
  if (fast && bm == 256 && bn == 256) g.block = 512;  // 8 wavefronts
  mtk_tile_args a{};
  a.M = (int)M;
  a.N = d.O;
  a.K = (int)K;
  a.lda = 0;
  a.ldb = d.O;
  a.ldc = d.O;
  a.a_bytes = (uint32_t)x_bytes;
  a.b_bytes = (uint32_t)w_bytes;
  a.tiles_m = (int)((M + bm - 1) / bm);
  a.tiles_n = (d.O + bn - 1) / bn;
  a.k_tiles = (int)((K + 63) / 64);
  a.k_tiles_per_split = a.k_tiles;
  a.split_k = 1;
  a.has_bias = d.has_bias ? 1 : 0;
  a.cN = d.N;
  a.cD = d.D;
  a.cH = d.H;
  a.cW = d.W;
  a.cC = d.C;
  a.cKD = d.KD;
  a.cKH = d.KH;
  a.cKW = d.KW;
  a.cSZ = d.stride_d;
  a.cSY = d.stride_h;
  a.cSX = d.stride_w;
  a.cDZ = d.dil_d;
  a.cDY = d.dil_h;
  a.cDX = d.dil_w;
  a.cPF = d.pad_front;
  a.cPT = d.pad_top;
  a.cPL = d.pad_left;
  a.cOD = od;
  a.cOH = oh;
  a.cOW = ow;
  g.grid = (unsigned)((long long)a.tiles_m * a.tiles_n);
  set_args(g, a);
  p->launches.push_back(g);
  p->flops = 2.0 * (double)M * d.O * (double)K;
  p->bytes = (double)x_bytes + (double)w_bytes + 2.0 * (double)y_elems + (d.has_bias ? 2.0 * d.O : 0) +
             (oidhw ? 2.0 * (double)w_bytes : 0.0);  // the re-layout reads and writes the weights once
  char desc[288];
  snprintf(desc, sizeof desc, "conv%dd f16 implicit-GEMM M=%lld N=%d K=%lld out=%dx%dx%d tile=%dx%d gather=%s grid=%u%s",
           d.rank, M, d.O, K, od, oh, ow, bm, bn, kind, g.grid,
           oidhw ? " weights OIDHW (re-laid out in the workspace)" : "");
  p->description = desc;
  s = resolve(p);
  if (s != MTK_OK) {
    delete p;
    return s;
  }
  *out = p;
  return MTK_OK;
}

// ------------------------------------------------------------------ attention planning

int plan_attn(mtk_ctx *ctx, const mtk_attn_desc *d_in, mtk_plan **out) {
  if (!d_in || !out) return fail(MTK_ERR_INVALID, "null descriptor or output");
  mtk_attn_desc d = *d_in;
  if (d.B <= 0 || d.H <= 0 || d.S_q <= 0 || d.S_kv <= 0) return fail(MTK_ERR_INVALID, "B, H, S_q, S_kv must be positive");
  if (d.H_kv == 0) d.H_kv = d.H;
  if (d.H_kv < 0 || d.H % d.H_kv != 0)
    return fail(MTK_ERR_INVALID, "H_kv must divide H (got H=%d, H_kv=%d)", d.H, d.H_kv);
  if (d.D < 1 || d.D > kMaxHeadDim)
    return fail(MTK_ERR_UNSUPPORTED, "head dimension must be 1..%d (got %d)", kMaxHeadDim, d.D);
  // above 256: the 16-query wavefront kernel laid out for 512 (16-byte aligned rows only)
  const bool wide = d.D > 256;
  if (wide && d.D % 8 != 0)
    return fail(MTK_ERR_UNSUPPORTED, "head dimensions above 256 must be multiples of 8 (got %d)", d.D);
  if (wide && d.q_rows != 0)
    return fail(MTK_ERR_UNSUPPORTED, "head dimensions above 256 run 64 query rows per workgroup (q_rows must be 0)");
  if (d.dtype != MTK_F16 && d.dtype != MTK_BF16) return fail(MTK_ERR_INVALID, "attention dtype must be MTK_F16 or MTK_BF16");
  if (d.q_rows != 0 && d.q_rows != 128 && d.q_rows != 256)
    return fail(MTK_ERR_INVALID, "q_rows must be 0, 128 or 256 (got %d)", d.q_rows);
  if (d.q_rows == 256 && d.D != 128 && d.D != 64)
    return fail(MTK_ERR_UNSUPPORTED, "q_rows 256 (the ping-pong kernel) needs head dimension 128 or 64 (got %d)", d.D);
  const uint64_t q_bytes = (uint64_t)d.B * d.S_q * d.H * d.D * 2;
  const uint64_t kv_bytes = (uint64_t)d.B * d.S_kv * d.H_kv * d.D * 2;
  if (q_bytes > kMaxOperandBytes || kv_bytes > kMaxOperandBytes)
    return fail(MTK_ERR_UNSUPPORTED, "operands above 2 GiB are not supported by this build");
  mtk_plan *p = new mtk_plan();
  p->ctx = ctx;
  p->kind = PLAN_ATTN;
  p->attn = d;
  // Head dimension: the kernels are compiled for a padded head dimension DP of 64, 128 or 256 and
  // run any D <= DP. D % 8 == 0 keeps every row 16-byte aligned (direct-to-LDS staging, 16-byte
  // loads); other D use the element-staged kernels (2-byte aligned rows).
  const int dp = d.D <= 64 ? 64 : d.D <= 128 ? 128 : d.D <= 256 ? 256 : 512;
  const bool gen = d.D % 8 != 0;
  p->align_a = p->align_b = gen ? 2 : 16;
  // Query rows per workgroup: 256 (the ping-pong kernel: 8 wavefronts in two groups alternating MFMA
  // and softmax blocks, one workgroup per CU) for non-causal D = 128 and D = 64 grids that still fill
  // the device (config 5, one box: 526.5 us against 546.5 us for 128 rows; at D = 64 368.8 against
  // 412.4 us); 128 (4 wavefronts, two workgroups
  // per CU) otherwise, causal included (config 5 causal, one box: 298.7 us against 305.3 us for the
  // ping-pong kernel, both in the kernels' balanced causal dispatch order).
  int rows = d.q_rows;
  if (rows == 0) {
    const int cus = ctx ? ctx->prop.multiProcessorCount : 256;
    rows = ((d.D == 128 || d.D == 64) && !d.causal && (long long)d.B * d.H * ((d.S_q + 255) / 256) >= cus) ? 256 : 128;
    if (wide) rows = 64;
  }
  Launch g;
  std::string family;
  if (rows == 256)
    family = dp == 128 ? "pp_" : "pp_d64_";  // D = 128 or 64 exactly
  else if (gen)
    family = "g" + std::to_string(dp) + "_";
  else if (dp != 128)
    family = "d" + std::to_string(dp) + "_";
  g.name = "mtk_attn_fwd_" + family + (d.dtype == MTK_F16 ? "f16" : "bf16") + (d.causal ? "_causal" : "");
  if (rows == 256) g.block = 512;  // 8 wavefronts: two groups of 4 in ping-pong
  mtk_attn_kargs a{};
  a.B = d.B;
  a.H = d.H;
  a.H_kv = d.H_kv;
  a.S_q = d.S_q;
  a.S_kv = d.S_kv;
  a.q_blocks = (d.S_q + rows - 1) / rows;
  a.causal = d.causal ? 1 : 0;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)d.D));
  a.q_bytes = (uint32_t)q_bytes;
  a.kv_bytes = (uint32_t)kv_bytes;
  a.D = d.D;
  g.grid = (unsigned)((long long)a.q_blocks * d.B * d.H);
  set_args(g, a);
  p->launches.push_back(g);
  double pairs = (double)d.S_q * d.S_kv;
  if (d.causal) {  // exact count of unmasked (i, j): j <= i + (S_kv - S_q)
    pairs = 0;
    for (long long i = 0; i < d.S_q; ++i) {
      long long lim = i + (d.S_kv - d.S_q) + 1;
      pairs += (double)std::max(0ll, std::min<long long>(lim, d.S_kv));
    }
  }
  p->flops = 4.0 * d.B * d.H * d.D * pairs;
  p->bytes = 2.0 * (double)q_bytes + 2.0 * (double)kv_bytes;
  char desc[256];
  snprintf(desc, sizeof desc, "attention fwd %s B=%d H=%d H_kv=%d S_q=%d S_kv=%d D=%d causal=%d rows/wg=%d grid=%u",
           d.dtype == MTK_F16 ? "f16" : "bf16", d.B, d.H, d.H_kv, d.S_q, d.S_kv, d.D, d.causal, rows, g.grid);
  p->description = desc;
  int s = resolve(p);
  if (s != MTK_OK) {
    delete p;
    return s;
  }
  *out = p;
  return MTK_OK;
}

// ------------------------------------------------------------------ binding run-time pointers

int check_gemm_args(const mtk_plan *p, const mtk_gemm_args *g) {
  if (!g || !g->A || !g->B || !g->C) return fail(MTK_ERR_INVALID, "A, B and C must be non-null");
  if (p->gemm.has_bias && !g->bias) return fail(MTK_ERR_INVALID, "plan has a bias but bias is null");
  if (!aligned(g->A, p->align_a) || !aligned(g->B, p->align_b))
    return fail(MTK_ERR_INVALID, "A/B must be %u-byte aligned for this plan", p->align_a);
  if (!aligned(g->C, 4)) return fail(MTK_ERR_INVALID, "C must be 4-byte aligned");
  return MTK_OK;
}

// Writes the run-time pointers of one GEMM launch into `block`, a copy of that launch's argument
// block; `ws` is the workspace (the caller's, or the static scratch).
void patch_gemm(const mtk_plan *p, const Launch &l, char *block, const mtk_gemm_args *g, void *ws) {
  if (l.name.rfind("mtk_skinny_", 0) == 0) {
    mtk_skinny_args *k = (mtk_skinny_args *)block;
    k->A = g->A;
    k->B = g->B;
    k->bias = g->bias;
    k->C = g->C;
    k->partial = p->workspace ? (float *)ws : nullptr;  // the partial-writing kernel's output
    return;
  }
  const bool two_pass = p->workspace != 0 && !p->serial_split;
  if (l.role == ROLE_MAIN) {
    mtk_tile_args *a = (mtk_tile_args *)block;
    a->A = g->A;
    a->B = g->B;
    a->bias = g->bias;
    a->C = two_pass ? nullptr : g->C;
    a->partial = p->workspace ? (float *)ws : nullptr;
  } else if (l.role == ROLE_REDUCE) {
    mtk_reduce_args *r = (mtk_reduce_args *)block;
    r->partial = (const float *)ws;
    r->bias = g->bias;
    r->C = g->C;
    r->vec4 = r->vec4 && aligned(g->C, 8) && (!g->bias || aligned(g->bias, 8));
  }
}

int bind_args(const mtk_plan *p, const void *argset, std::vector<Launch> &ls) {
  ls = p->launches;
  if (p->kind == PLAN_GEMM) {
    const mtk_gemm_args *g = (const mtk_gemm_args *)argset;
    int s = check_gemm_args(p, g);
    if (s != MTK_OK) return s;
    if (p->workspace && (!g->workspace || !aligned(g->workspace, 16)))
      return fail(MTK_ERR_INVALID, "this plan needs a 16-byte aligned workspace of %zu bytes", p->workspace);
    for (Launch &l : ls) patch_gemm(p, l, l.args.data(), g, g->workspace);
  } else if (p->kind == PLAN_CONV) {
    const mtk_conv_args *c = (const mtk_conv_args *)argset;
    if (!c || !c->x || !c->w || !c->y) return fail(MTK_ERR_INVALID, "x, w and y must be non-null");
    if (p->conv.has_bias && !c->bias) return fail(MTK_ERR_INVALID, "plan has a bias but bias is null");
    if (!aligned(c->x, p->align_a) || !aligned(c->w, p->align_b))
      return fail(MTK_ERR_INVALID, "x must be %u-byte and w %u-byte aligned for this plan", p->align_a, p->align_b);
    if (p->workspace && (!c->workspace || !aligned(c->workspace, 16)))
      return fail(MTK_ERR_INVALID, "this plan needs a 16-byte aligned workspace of %zu bytes", p->workspace);
    if (p->workspace) {
      const char *w0 = (const char *)c->w, *s0 = (const char *)c->workspace;
      if (w0 < s0 + p->workspace && s0 < w0 + p->weight_bytes) return fail(MTK_ERR_INVALID, "w and workspace overlap");
    }
    for (Launch &l : ls) {
      if (l.role == ROLE_PERMUTE) {
        mtk_permute_args &pa = args_of<mtk_permute_args>(l);
        pa.src = c->w;
        pa.dst = c->workspace;
        continue;
      }
      mtk_tile_args &a = args_of<mtk_tile_args>(l);
      a.A = c->x;
      a.B = p->workspace ? c->workspace : c->w;
      a.bias = c->bias;
      a.C = c->y;
      a.partial = nullptr;
    }
  } else if (p->kind == PLAN_PERMUTE) {
    const mtk_permute_run_args *t = (const mtk_permute_run_args *)argset;
    if (!t || !t->src || !t->dst) return fail(MTK_ERR_INVALID, "src and dst must be non-null");
    if (!aligned(t->src, p->align_a) || !aligned(t->dst, p->align_b))
      return fail(MTK_ERR_INVALID, "src and dst must be %u-byte aligned for this plan", p->align_a);
    const size_t n = (size_t)p->perm.O * p->perm.C * p->perm.KD * p->perm.KH * p->perm.KW * 2;
    const char *s0 = (const char *)t->src, *d0 = (const char *)t->dst;
    if (s0 < d0 + n && d0 < s0 + n) return fail(MTK_ERR_INVALID, "src and dst overlap");
    mtk_permute_args &a = args_of<mtk_permute_args>(ls[0]);
    a.src = t->src;
    a.dst = t->dst;
  } else if (p->kind == PLAN_ATTN_BWD) {
    const mtk_attn_bwd_args *t = (const mtk_attn_bwd_args *)argset;
    if (!t || !t->Q || !t->K || !t->V || !t->O || !t->dO || !t->lse || !t->dQ || !t->dK || !t->dV)
      return fail(MTK_ERR_INVALID, "Q, K, V, O, dO, lse, dQ, dK and dV must be non-null");
    for (const void *x : {t->Q, t->K, t->V, t->O, t->dO, (const void *)t->dQ, (const void *)t->dK, (const void *)t->dV})
      if (!aligned(x, 16)) return fail(MTK_ERR_INVALID, "attention tensors must be 16-byte aligned");
    if (!aligned(t->lse, 4)) return fail(MTK_ERR_INVALID, "lse must be 4-byte aligned");
    if (!t->workspace || !aligned(t->workspace, 16))
      return fail(MTK_ERR_INVALID, "this plan needs a 16-byte aligned workspace of %zu bytes", p->workspace);
    for (Launch &l : ls) {
      mtk_attn_bwd_kargs &a = args_of<mtk_attn_bwd_kargs>(l);
      a.Q = t->Q;
      a.K = t->K;
      a.V = t->V;
      a.O = t->O;
      a.dO = t->dO;
      a.lse = t->lse;
      a.Dt = (float *)t->workspace;
      a.Lt = (float *)((char *)t->workspace + p->workspace / 2);
      a.dQ = t->dQ;
      a.dK = t->dK;
      a.dV = t->dV;
    }
  } else {
    const mtk_attn_args *t = (const mtk_attn_args *)argset;
    if (!t || !t->Q || !t->K || !t->V || !t->O) return fail(MTK_ERR_INVALID, "Q, K, V and O must be non-null");
    const unsigned al = p->align_a;
    if (!aligned(t->Q, al) || !aligned(t->K, al) || !aligned(t->V, al) || !aligned(t->O, al))
      return fail(MTK_ERR_INVALID, "Q, K, V, O must be %u-byte aligned for this plan", al);
    if (t->lse && !aligned(t->lse, 4)) return fail(MTK_ERR_INVALID, "lse must be 4-byte aligned");
    mtk_attn_kargs &a = args_of<mtk_attn_kargs>(ls[0]);
    a.Q = t->Q;
    a.K = t->K;
    a.V = t->V;
    a.O = t->O;
    a.lse = t->lse;
  }
  return MTK_OK;
}

size_t argset_size(const mtk_plan *p) {
  switch (p->kind) {
    case PLAN_GEMM:
      return sizeof(mtk_gemm_args);
    case PLAN_CONV:
      return sizeof(mtk_conv_args);
    case PLAN_ATTN_BWD:
      return sizeof(mtk_attn_bwd_args);
    case PLAN_PERMUTE:
      return sizeof(mtk_permute_run_args);
    default:
      return sizeof(mtk_attn_args);
  }
}

int run_plan(const mtk_plan *p, const void *argset) {
  if (!p) return fail(MTK_ERR_INVALID, "null plan");
  if (!p->ctx) return fail(MTK_ERR_INVALID, "plan was created without a context (dry plan)");
  std::vector<Launch> ls;
  int s = bind_args(p, argset, ls);
  if (s != MTK_OK) return s;
  HIP_TRY(hipSetDevice(p->ctx->device));
  return launch_all(p, ls, nullptr);
}

std::string self_dir() {
  Dl_info info;
  if (dladdr((void *)&mtk_init, &info) && info.dli_fname) {
    std::string f = info.dli_fname;
    size_t k = f.rfind('/');
    if (k != std::string::npos) return f.substr(0, k);
  }
  return ".";
}

}  // namespace

// ====================================================================== C ABI

extern "C" {

const char *mtk_last_error(void) { return g_last_error.c_str(); }

const char *mtk_status_string(int s) {
  switch (s) {
    case MTK_OK:
      return "MTK_OK";
    case MTK_ERR_INVALID:
      return "MTK_ERR_INVALID";
    case MTK_ERR_NO_DEVICE:
      return "MTK_ERR_NO_DEVICE";
    case MTK_ERR_UNSUPPORTED:
      return "MTK_ERR_UNSUPPORTED";
    case MTK_ERR_MODULE:
      return "MTK_ERR_MODULE";
    case MTK_ERR_OOM:
      return "MTK_ERR_OOM";
    case MTK_ERR_LAUNCH:
      return "MTK_ERR_LAUNCH";
    case MTK_ERR_HIP:
      return "MTK_ERR_HIP";
    default:
      return "unknown status";
  }
}

int mtk_device_count(int *count) {
  if (!count) return fail(MTK_ERR_INVALID, "null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    *count = 0;
    return fail(MTK_ERR_NO_DEVICE, "no HIP device: %s", hipGetErrorString(e));
  }
  *count = n;
  return MTK_OK;
}

int mtk_init(int device, const char *code_object_dir, mtk_ctx **out) {
  if (!out) return fail(MTK_ERR_INVALID, "null output");
  *out = nullptr;
  int n = 0;
  int s = mtk_device_count(&n);
  if (s != MTK_OK) return s;
  if (n <= 0) return fail(MTK_ERR_NO_DEVICE, "no HIP device");
  if (device < 0 || device >= n) return fail(MTK_ERR_INVALID, "device %d out of range (%d devices)", device, n);
  mtk_ctx *ctx = new mtk_ctx();
  ctx->device = device;
  auto bail = [&](int status) {
    mtk_destroy(ctx);
    return status;
  };
  if (hipSetDevice(device) != hipSuccess) return bail(fail(MTK_ERR_HIP, "hipSetDevice(%d) failed", device));
  if (hipGetDeviceProperties(&ctx->prop, device) != hipSuccess) return bail(fail(MTK_ERR_HIP, "hipGetDeviceProperties failed"));
  if (strncmp(ctx->prop.gcnArchName, "gfx950", 6) != 0)
    return bail(fail(MTK_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950 (MI355X)", device, ctx->prop.gcnArchName));
  // the static scratch of mtk_gemm_run_noalloc: its device address on this device, taken once
  // (a failure is reported by that entry point; nothing else uses the scratch)
  (void)mtk_scratch::setup(device);
  if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess)
    return bail(fail(MTK_ERR_HIP, "hipStreamCreate failed"));
  ctx->stream = ctx->own_stream;
  std::string dir;
  if (code_object_dir && *code_object_dir)
    dir = code_object_dir;
  else if (const char *env = getenv("MTK_CODE_OBJECT_DIR"))
    dir = env;
  else
    dir = self_dir();
  DIR *dp = opendir(dir.c_str());
  if (!dp) return bail(fail(MTK_ERR_MODULE, "code object directory %s not readable", dir.c_str()));
  std::vector<std::string> files;
  while (dirent *e = readdir(dp)) {
    std::string f = e->d_name;
    if (f.size() > 10 && f.rfind("mtk_", 0) == 0 && f.substr(f.size() - 6) == ".hsaco") files.push_back(f);
  }
  closedir(dp);
  std::sort(files.begin(), files.end());
  if (files.empty()) return bail(fail(MTK_ERR_MODULE, "no mtk_*.hsaco code objects in %s", dir.c_str()));
  for (const std::string &f : files) {
    hipModule_t m = nullptr;
    std::string path = dir + "/" + f;
    hipError_t e = hipModuleLoad(&m, path.c_str());
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return bail(fail(MTK_ERR_MODULE, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e)));
    }
    // the code object's kernel-argument contract must be this library's
    hipDeviceptr_t gp = nullptr;
    size_t gsz = 0;
    int32_t version = -1;
    e = hipModuleGetGlobal(&gp, &gsz, m, "mtk_kargs_version");
    if (e == hipSuccess && gsz == sizeof version) e = hipMemcpyDtoH(&version, gp, sizeof version);
    if (e != hipSuccess || gsz != sizeof version || version != MTK_KARGS_VERSION) {
      (void)hipGetLastError();
      (void)hipModuleUnload(m);
      return bail(fail(MTK_ERR_MODULE, "%s was built for kernel-argument version %d, this library uses %d: rebuild it",
                       path.c_str(), version, MTK_KARGS_VERSION));
    }
    ctx->modules.push_back(m);
  }
  *out = ctx;
  return MTK_OK;
}

int mtk_destroy(mtk_ctx *ctx) {
  if (!ctx) return MTK_OK;
  if (ctx->own_stream) {
    (void)hipStreamSynchronize(ctx->own_stream);
    (void)hipStreamDestroy(ctx->own_stream);
  }
  for (hipModule_t m : ctx->modules) (void)hipModuleUnload(m);
  delete ctx;
  return MTK_OK;
}

int mtk_get_device_info(const mtk_ctx *ctx, mtk_device_info *info) {
  if (!ctx || !info) return fail(MTK_ERR_INVALID, "null argument");
  memset(info, 0, sizeof *info);
  snprintf(info->name, sizeof info->name, "%s", ctx->prop.name);
  snprintf(info->arch, sizeof info->arch, "%s", ctx->prop.gcnArchName);
  info->compute_units = ctx->prop.multiProcessorCount;
  info->clock_khz = ctx->prop.clockRate;
  info->lds_bytes_per_cu = (int)ctx->prop.maxSharedMemoryPerMultiProcessor;
  info->wavefront_size = ctx->prop.warpSize;
  info->global_mem_bytes = ctx->prop.totalGlobalMem;
  info->peak_f16_tflops = (double)info->compute_units * (info->clock_khz * 1e3) * 4096.0 / 1e12;
  return MTK_OK;
}

int mtk_alloc(mtk_ctx *ctx, size_t bytes, void **dptr) {
  if (!ctx || !dptr) return fail(MTK_ERR_INVALID, "null argument");
  *dptr = nullptr;
  HIP_TRY(hipSetDevice(ctx->device));
  hipError_t e = hipMalloc(dptr, bytes ? bytes : 1);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(MTK_ERR_OOM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
  }
  return MTK_OK;
}

int mtk_free(mtk_ctx *ctx, void *dptr) {
  if (!ctx) return fail(MTK_ERR_INVALID, "null context");
  if (!dptr) return MTK_OK;
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipFree(dptr));
  return MTK_OK;
}

int mtk_upload(mtk_ctx *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(MTK_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return MTK_OK;
}

int mtk_download(mtk_ctx *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(MTK_ERR_INVALID, "null argument");
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return MTK_OK;
}

int mtk_fill_u16(mtk_ctx *ctx, void *dst, uint16_t value, size_t count) {
  if (!ctx || (!dst && count)) return fail(MTK_ERR_INVALID, "null argument");
  if (!count) return MTK_OK;
  hipFunction_t f;
  int s = ctx->function("mtk_fill_u16", &f);
  if (s != MTK_OK) return s;
  mtk_fill_args a{dst, (uint64_t)count, value};
  void *params[] = {&a};
  unsigned grid = (unsigned)std::min<size_t>((count + 255) / 256, 4096);
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipModuleLaunchKernel(f, grid, 1, 1, 256, 1, 1, 0, ctx->stream, params, nullptr));
  return MTK_OK;
}

int mtk_sync(mtk_ctx *ctx) {
  if (!ctx) return fail(MTK_ERR_INVALID, "null context");
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return MTK_OK;
}

int mtk_set_stream(mtk_ctx *ctx, void *hip_stream) {
  if (!ctx) return fail(MTK_ERR_INVALID, "null context");
  ctx->stream = hip_stream ? (hipStream_t)hip_stream : ctx->own_stream;
  return MTK_OK;
}

int mtk_gemm_plan(mtk_ctx *ctx, const mtk_gemm_desc *desc, mtk_plan **out) { return plan_gemm(ctx, desc, out); }
int mtk_gemm_run(const mtk_plan *plan, const mtk_gemm_args *args) {
  if (plan && plan->kind != PLAN_GEMM) return fail(MTK_ERR_INVALID, "not a GEMM plan");
  return run_plan(plan, args);
}

int mtk_gemm_run_noalloc(const mtk_plan *plan, const mtk_gemm_args *args) {
  if (!plan) return fail(MTK_ERR_INVALID, "null plan");
  if (plan->kind != PLAN_GEMM) return fail(MTK_ERR_INVALID, "not a GEMM plan");
  if (!plan->ctx) return fail(MTK_ERR_INVALID, "plan was created without a context (dry plan)");
  int s = check_gemm_args(plan, args);
  if (s != MTK_OK) return s;
  if (args->workspace)
    return fail(MTK_ERR_INVALID, "mtk_gemm_run_noalloc works in the library's static scratch: workspace must be NULL");
  if (plan->workspace > (size_t)MTK_NOALLOC_MAX_WORKSPACE)
    return fail(MTK_ERR_UNSUPPORTED,
                "this plan needs a %zu-byte workspace, above the %zu bytes of mtk_gemm_run_noalloc's static scratch: "
                "use mtk_gemm_run with a caller workspace",
                plan->workspace, (size_t)MTK_NOALLOC_MAX_WORKSPACE);
  void *ws = nullptr;
  if (plan->workspace) {
    char err[256];
    if (mtk_scratch::address(plan->ctx->device, &ws, err, sizeof err) != 0) return fail(MTK_ERR_HIP, "%s", err);
  }
  // argument blocks on the stack: nothing is allocated, on the device or the host
  alignas(16) char block[512];
  HIP_TRY(hipSetDevice(plan->ctx->device));
  for (const Launch &l : plan->launches) {
    if (l.args.size() > sizeof block) return fail(MTK_ERR_INVALID, "argument block of %s too large", l.name.c_str());
    memcpy(block, l.args.data(), l.args.size());
    patch_gemm(plan, l, block, args, ws);
    void *params[] = {block};
    hipError_t e = hipModuleLaunchKernel(l.fn, l.grid, 1, 1, l.block, 1, 1, 0, plan->ctx->stream, params, nullptr);
    if (e != hipSuccess) return fail(MTK_ERR_LAUNCH, "launch of %s failed: %s", l.name.c_str(), hipGetErrorString(e));
  }
  return MTK_OK;
}

int mtk_attn_plan(mtk_ctx *ctx, const mtk_attn_desc *desc, mtk_plan **out) { return plan_attn(ctx, desc, out); }
int mtk_attn_run(const mtk_plan *plan, const mtk_attn_args *args) {
  if (plan && plan->kind != PLAN_ATTN) return fail(MTK_ERR_INVALID, "not an attention plan");
  return run_plan(plan, args);
}

int mtk_attn_bwd_plan(mtk_ctx *ctx, const mtk_attn_desc *desc, mtk_plan **out) {
  return plan_attn_bwd(ctx, desc, out);
}
int mtk_attn_bwd_run(const mtk_plan *plan, const mtk_attn_bwd_args *args) {
  if (plan && plan->kind != PLAN_ATTN_BWD) return fail(MTK_ERR_INVALID, "not an attention backward plan");
  return run_plan(plan, args);
}

int mtk_permute_plan(mtk_ctx *ctx, const mtk_permute_desc *desc, mtk_plan **out) {
  return plan_permute(ctx, desc, out);
}
int mtk_permute_run(const mtk_plan *plan, const mtk_permute_run_args *args) {
  if (plan && plan->kind != PLAN_PERMUTE) return fail(MTK_ERR_INVALID, "not a permutation plan");
  return run_plan(plan, args);
}

int mtk_conv_plan(mtk_ctx *ctx, const mtk_conv_desc *desc, mtk_plan **out) { return plan_conv(ctx, desc, out); }
int mtk_conv_out_shape(const mtk_conv_desc *desc, int *OD, int *OH, int *OW) {
  if (!desc || !OD || !OH || !OW) return fail(MTK_ERR_INVALID, "null argument");
  mtk_conv_desc d;
  int s = normalise_conv(desc, &d);
  if (s != MTK_OK) return s;
  return conv_out(&d, OD, OH, OW);
}
int mtk_conv_run(const mtk_plan *plan, const mtk_conv_args *args) {
  if (plan && plan->kind != PLAN_CONV) return fail(MTK_ERR_INVALID, "not a convolution plan");
  return run_plan(plan, args);
}

size_t mtk_plan_workspace_bytes(const mtk_plan *plan) { return plan ? plan->workspace : 0; }

int mtk_plan_describe(const mtk_plan *plan, char *buf, size_t len) {
  if (!plan || !buf || !len) return fail(MTK_ERR_INVALID, "null argument");
  std::string s = plan->description + " kernels:";
  for (const auto &l : plan->launches) s += " " + l.name;
  snprintf(buf, len, "%s", s.c_str());
  return MTK_OK;
}

int mtk_plan_work(const mtk_plan *plan, double *flops, double *bytes) {
  if (!plan) return fail(MTK_ERR_INVALID, "null plan");
  if (flops) *flops = plan->flops;
  if (bytes) *bytes = plan->bytes;
  return MTK_OK;
}

int mtk_plan_destroy(mtk_plan *plan) {
  delete plan;
  return MTK_OK;
}

struct mtk_graph {
  mtk_ctx *ctx = nullptr;
  hipStream_t stream = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

int mtk_graph_create(const mtk_plan *p, const void *arg_sets, int nsets, int steps, mtk_graph **out) {
  if (!p || !arg_sets || nsets <= 0 || steps <= 0 || !out) return fail(MTK_ERR_INVALID, "invalid graph arguments");
  if (!p->ctx) return fail(MTK_ERR_INVALID, "plan was created without a context (dry plan)");
  if (steps > 100000) return fail(MTK_ERR_INVALID, "steps above 100000");
  *out = nullptr;
  const size_t stride = argset_size(p);
  std::vector<std::vector<Launch>> bound((size_t)nsets);
  for (int i = 0; i < nsets; ++i) {
    int s = bind_args(p, (const char *)arg_sets + stride * i, bound[(size_t)i]);
    if (s != MTK_OK) return s;
  }
  HIP_TRY(hipSetDevice(p->ctx->device));
  hipStream_t st = p->ctx->stream;
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  int status = MTK_OK;
  for (int i = 0; i < steps && status == MTK_OK; ++i) status = launch_all(p, bound[(size_t)(i % nsets)], nullptr);
  hipGraph_t graph = nullptr;
  const hipError_t ec = hipStreamEndCapture(st, &graph);
  if (status != MTK_OK || ec != hipSuccess) {
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
    return status != MTK_OK ? status : fail(MTK_ERR_HIP, "stream capture failed: %s", hipGetErrorString(ec));
  }
  hipGraphExec_t exec = nullptr;
  const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (ei != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return fail(MTK_ERR_HIP, "graph instantiation failed: %s", hipGetErrorString(ei));
  }
  // Finish setting the graph up on the device now (kernel argument blocks and the launch packets
  // prepared), so that the first launch submits work instead of doing this set-up. No kernel runs.
  const hipError_t eu = hipGraphUpload(exec, st);
  if (eu == hipSuccess) {
    const hipError_t es = hipStreamSynchronize(st);
    if (es != hipSuccess) {
      (void)hipGraphExecDestroy(exec);
      (void)hipGraphDestroy(graph);
      return fail(MTK_ERR_HIP, "graph upload failed: %s", hipGetErrorString(es));
    }
  } else {
    (void)hipGetLastError();  // optional step: the first launch then does the set-up itself
  }
  mtk_graph *g = new mtk_graph();
  g->ctx = p->ctx;
  g->stream = st;
  g->graph = graph;
  g->exec = exec;
  *out = g;
  return MTK_OK;
}

int mtk_graph_launch(mtk_graph *g) {
  if (!g) return fail(MTK_ERR_INVALID, "null graph");
  HIP_TRY(hipSetDevice(g->ctx->device));
  HIP_TRY(hipGraphLaunch(g->exec, g->stream));
  return MTK_OK;
}

int mtk_graph_destroy(mtk_graph *g) {
  if (!g) return MTK_OK;
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
  return MTK_OK;
}

int mtk_profile(const mtk_plan *p, const void *arg_sets, int nsets, int warmup, int iters, mtk_timing *out) {
  if (!p || !arg_sets || nsets <= 0 || warmup < 0 || iters <= 0 || !out)
    return fail(MTK_ERR_INVALID, "invalid profile arguments");
  if (!p->ctx) return fail(MTK_ERR_INVALID, "plan was created without a context (dry plan)");
  if (iters > 100000) return fail(MTK_ERR_INVALID, "iters above 100000");
  memset(out, 0, sizeof *out);
  const size_t stride = argset_size(p);
  std::vector<std::vector<Launch>> bound((size_t)nsets);
  for (int i = 0; i < nsets; ++i) {
    int s = bind_args(p, (const char *)arg_sets + stride * i, bound[(size_t)i]);
    if (s != MTK_OK) return s;
  }
  HIP_TRY(hipSetDevice(p->ctx->device));
  for (int i = 0; i < warmup; ++i) {
    int s = launch_all(p, bound[(size_t)(i % nsets)], nullptr);
    if (s != MTK_OK) return s;
  }
  const size_t nk = p->launches.size();
  // Events created so far are destroyed on every exit path; a failed query fails the call (never
  // a silent 0 ms).
  std::vector<hipEvent_t> evs;
  evs.reserve((size_t)iters * (nk + 1));
  int status = MTK_OK;
  for (size_t i = 0; i < (size_t)iters * (nk + 1) && status == MTK_OK; ++i) {
    hipEvent_t e = nullptr;
    const hipError_t ec = hipEventCreate(&e);
    if (ec != hipSuccess)
      status = fail(MTK_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(ec));
    else
      evs.push_back(e);
  }
  for (int i = 0; i < iters && status == MTK_OK; ++i)
    status = launch_all(p, bound[(size_t)(i % nsets)], &evs[(size_t)i * (nk + 1)]);
  if (status == MTK_OK) {
    hipError_t e = hipStreamSynchronize(p->ctx->stream);
    if (e != hipSuccess) status = fail(MTK_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  }
  auto elapsed = [&](hipEvent_t a, hipEvent_t b, float *ms) {
    const hipError_t e = hipEventElapsedTime(ms, a, b);
    return e == hipSuccess ? MTK_OK : fail(MTK_ERR_HIP, "hipEventElapsedTime: %s", hipGetErrorString(e));
  };
  if (status == MTK_OK) {
    std::vector<double> per(nk, 0.0);
    for (int i = 0; i < iters && status == MTK_OK; ++i) {
      for (size_t k = 0; k < nk && status == MTK_OK; ++k) {
        float ms = 0;
        status = elapsed(evs[(size_t)i * (nk + 1) + k], evs[(size_t)i * (nk + 1) + k + 1], &ms);
        per[k] += ms;
      }
    }
    float total = 0;
    if (status == MTK_OK) status = elapsed(evs[0], evs[(size_t)(iters - 1) * (nk + 1) + nk], &total);
    out->total_ms = total / iters;
    out->n_kernels = (int)std::min<size_t>(nk, 4);
    for (size_t k = 0; k < nk && k < 4; ++k) {
      out->kernel_ms[k] = per[k] / iters;
      snprintf(out->kernel_names[k], sizeof out->kernel_names[k], "%s", p->launches[k].name.c_str());
    }
  }
  for (auto &e : evs) (void)hipEventDestroy(e);
  return status;
}

int mtk_validate_f16(const uint16_t *actual, int dtype, const float *expected, size_t n, double abs_tol, mtk_validation *out) {
  if ((!actual || !expected) && n) return fail(MTK_ERR_INVALID, "null argument");
  if (!out || (dtype != MTK_F16 && dtype != MTK_BF16)) return fail(MTK_ERR_INVALID, "invalid argument");
  double num = 0, den = 0, mx = 0;
  long long bad = 0;
  for (size_t i = 0; i < n; ++i) {
    const float v = dtype == MTK_BF16 ? bf16_to_f32(actual[i]) : f16_to_f32(actual[i]);
    const double diff = std::fabs((double)v - (double)expected[i]);
    num += diff * diff;
    den += (double)expected[i] * expected[i];
    mx = std::max(mx, diff);
    if (diff > abs_tol || std::isnan(v)) ++bad;
  }
  out->rel_frobenius = den > 0 ? std::sqrt(num / den) : std::sqrt(num);
  out->max_abs_error = mx;
  out->mismatches = bad;
  return MTK_OK;
}

}  // extern "C"
