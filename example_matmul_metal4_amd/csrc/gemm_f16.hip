// fp16 GEMM instantiations. Kernel names are what the runtime's kernel-select looks up.
//   *_nt_*_d   B [N][K] (the reference's default layout), direct-to-LDS pipeline
//   *_nn_*_d   B [K][N] (config 1 "C = A.B row-major"), direct-to-LDS + transposed LDS reads
//   *_tt_*_d, *_tn_*_d   A [K][M] (the reference's transpose.left) with B [N][K] / [K][N]
//   *_s        split-K with the partitions run in sequence by one workgroup per tile
//   *_v1       2-byte register-staged fallback for odd leading dimensions
// plus the split-K second pass.
#include "tile_direct.hpp"

using namespace mtk;

// 256x256 tiles: 8 wavefronts (2 x 4, 128 x 64 each, two per SIMD); 128x128: 4 (2 x 2).
#define DIRECT_KERNEL(NAME, DT, BM, BN, WM, WN, AOP, BOP, SER)                                      \
  extern "C" __global__ void __launch_bounds__(64 * WM * WN) NAME(const mtk_tile_args a) {        \
    tile_direct<DT, BM, BN, WM, WN, AOP, BOP, SER>(a);                                            \
  }

#define TILE_KERNEL(NAME, DT, BM, BN, WM, WN, AK, BKIND, VA, VB)                    \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_gemm<DT, BM, BN, WM, WN, AK, BKIND, VA, VB>(a);                          \
  }

using R256 = OpRows<256, 8>;
using C256 = OpColsT<256, 8>;
using R128 = OpRows<128, 4>;
using C128 = OpColsT<128, 4>;
DIRECT_KERNEL(mtk_gemm_f16_nt_256x256_d, DT_F16, 256, 256, 2, 4, R256, R256, false)
DIRECT_KERNEL(mtk_gemm_f16_nt_128x128_d, DT_F16, 128, 128, 2, 2, R128, R128, false)
DIRECT_KERNEL(mtk_gemm_f16_nt_256x256_s, DT_F16, 256, 256, 2, 4, R256, R256, true)
DIRECT_KERNEL(mtk_gemm_f16_nt_128x128_s, DT_F16, 128, 128, 2, 2, R128, R128, true)
DIRECT_KERNEL(mtk_gemm_f16_nn_256x256_d, DT_F16, 256, 256, 2, 4, R256, C256, false)
DIRECT_KERNEL(mtk_gemm_f16_nn_128x128_d, DT_F16, 128, 128, 2, 2, R128, C128, false)
DIRECT_KERNEL(mtk_gemm_f16_nn_256x256_s, DT_F16, 256, 256, 2, 4, R256, C256, true)
DIRECT_KERNEL(mtk_gemm_f16_nn_128x128_s, DT_F16, 128, 128, 2, 2, R128, C128, true)
DIRECT_KERNEL(mtk_gemm_f16_tt_256x256_d, DT_F16, 256, 256, 2, 4, C256, R256, false)
DIRECT_KERNEL(mtk_gemm_f16_tt_128x128_d, DT_F16, 128, 128, 2, 2, C128, R128, false)
DIRECT_KERNEL(mtk_gemm_f16_tt_256x256_s, DT_F16, 256, 256, 2, 4, C256, R256, true)
DIRECT_KERNEL(mtk_gemm_f16_tt_128x128_s, DT_F16, 128, 128, 2, 2, C128, R128, true)
DIRECT_KERNEL(mtk_gemm_f16_tn_256x256_d, DT_F16, 256, 256, 2, 4, C256, C256, false)
DIRECT_KERNEL(mtk_gemm_f16_tn_128x128_d, DT_F16, 128, 128, 2, 2, C128, C128, false)
DIRECT_KERNEL(mtk_gemm_f16_tn_256x256_s, DT_F16, 256, 256, 2, 4, C256, C256, true)
DIRECT_KERNEL(mtk_gemm_f16_tn_128x128_s, DT_F16, 128, 128, 2, 2, C128, C128, true)

TILE_KERNEL(mtk_gemm_f16_nt_256x256_v1, DT_F16, 256, 256, 2, 2, A_MK, B_NK, 1, 1)
TILE_KERNEL(mtk_gemm_f16_nt_128x128_v1, DT_F16, 128, 128, 2, 2, A_MK, B_NK, 1, 1)
TILE_KERNEL(mtk_gemm_f16_nn_256x256_v1, DT_F16, 256, 256, 2, 2, A_MK, B_KN, 1, 1)
TILE_KERNEL(mtk_gemm_f16_nn_128x128_v1, DT_F16, 128, 128, 2, 2, A_MK, B_KN, 1, 1)

extern "C" __global__ void __launch_bounds__(256) mtk_splitk_reduce_f16(const mtk_reduce_args a) {
  splitk_reduce<DT_F16>(a);
}
