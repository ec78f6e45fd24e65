// bf16 tile-GEMM instantiations: B stored [N][K] ("nt", the reference's default layout) or [K][N]
// ("nn"), plus the split-K second pass. Kernel names are what the runtime's kernel-select looks up.
//   *_d    direct-to-LDS staging, B [N][K], operand rows 4-byte aligned
//   *_vV   register-staged loads V halves wide (8, 4 or 1); for B [N][K] only the 2-byte
//          path remains (odd leading dimensions), everything else takes *_d
#include "tile_gemm.hpp"

using namespace mtk;

#define TILE_KERNEL(NAME, DT, BM, BN, WM, WN, AK, BKIND, VA, VB)                    \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_gemm<DT, BM, BN, WM, WN, AK, BKIND, VA, VB>(a);                          \
  }

#define DIRECT_KERNEL(NAME, DT, BM, BN, WM, WN)                                   \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_gemm_direct<DT, BM, BN, WM, WN>(a);                                      \
  }

DIRECT_KERNEL(mtk_gemm_bf16_nt_256x256_d, DT_BF16, 256, 256, 2, 2)
DIRECT_KERNEL(mtk_gemm_bf16_nt_128x128_d, DT_BF16, 128, 128, 2, 2)

TILE_KERNEL(mtk_gemm_bf16_nt_256x256_v1, DT_BF16, 256, 256, 2, 2, A_MK, B_NK, 1, 1)
TILE_KERNEL(mtk_gemm_bf16_nt_128x128_v1, DT_BF16, 128, 128, 2, 2, A_MK, B_NK, 1, 1)
TILE_KERNEL(mtk_gemm_bf16_nn_256x256_v8, DT_BF16, 256, 256, 2, 2, A_MK, B_KN, 8, 8)
TILE_KERNEL(mtk_gemm_bf16_nn_256x256_v4, DT_BF16, 256, 256, 2, 2, A_MK, B_KN, 4, 4)
TILE_KERNEL(mtk_gemm_bf16_nn_256x256_v1, DT_BF16, 256, 256, 2, 2, A_MK, B_KN, 1, 1)
TILE_KERNEL(mtk_gemm_bf16_nn_128x128_v8, DT_BF16, 128, 128, 2, 2, A_MK, B_KN, 8, 8)
TILE_KERNEL(mtk_gemm_bf16_nn_128x128_v4, DT_BF16, 128, 128, 2, 2, A_MK, B_KN, 4, 4)
TILE_KERNEL(mtk_gemm_bf16_nn_128x128_v1, DT_BF16, 128, 128, 2, 2, A_MK, B_KN, 1, 1)

extern "C" __global__ void __launch_bounds__(256) mtk_splitk_reduce_bf16(const mtk_reduce_args a) {
  splitk_reduce<DT_BF16>(a);
}
