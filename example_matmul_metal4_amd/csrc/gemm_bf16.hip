// bf16 GEMM instantiations. Kernel names are what the runtime's kernel-select looks up.
//   *_nt_*_d   B [N][K] (the reference's default layout), direct-to-LDS pipeline
//   *_nn_*_d   B [K][N] (config 1 "C = A.B row-major"), direct-to-LDS + transposed LDS reads
//   *_tt_*_d, *_tn_*_d   A [K][M] (the reference's transpose.left) with B [N][K] / [K][N]
//   *_s        split-K with the partitions run in sequence by one workgroup per tile
//   *_v1       2-byte register-staged fallback for odd leading dimensions
// plus the split-K second pass.
#include "tile_direct.hpp"

using namespace mtk;

#define DIRECT_KERNEL(NAME, DT, BM, BN, AOP, BOP)                                   \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_direct<DT, BM, BN, 2, 2, AOP, BOP>(a);                                   \
  }

#define SERIAL_KERNEL(NAME, DT, BM, BN, AOP, BOP)                                   \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_direct<DT, BM, BN, 2, 2, AOP, BOP, true>(a);                             \
  }

#define TILE_KERNEL(NAME, DT, BM, BN, WM, WN, AK, BKIND, VA, VB)                    \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_gemm<DT, BM, BN, WM, WN, AK, BKIND, VA, VB>(a);                          \
  }

DIRECT_KERNEL(mtk_gemm_bf16_nt_256x256_d, DT_BF16, 256, 256, OpRows<256>, OpRows<256>)
DIRECT_KERNEL(mtk_gemm_bf16_nt_128x128_d, DT_BF16, 128, 128, OpRows<128>, OpRows<128>)
DIRECT_KERNEL(mtk_gemm_bf16_nn_256x256_d, DT_BF16, 256, 256, OpRows<256>, OpColsT<256>)
DIRECT_KERNEL(mtk_gemm_bf16_nn_128x128_d, DT_BF16, 128, 128, OpRows<128>, OpColsT<128>)
DIRECT_KERNEL(mtk_gemm_bf16_tt_256x256_d, DT_BF16, 256, 256, OpColsT<256>, OpRows<256>)
DIRECT_KERNEL(mtk_gemm_bf16_tt_128x128_d, DT_BF16, 128, 128, OpColsT<128>, OpRows<128>)
DIRECT_KERNEL(mtk_gemm_bf16_tn_256x256_d, DT_BF16, 256, 256, OpColsT<256>, OpColsT<256>)
DIRECT_KERNEL(mtk_gemm_bf16_tn_128x128_d, DT_BF16, 128, 128, OpColsT<128>, OpColsT<128>)

SERIAL_KERNEL(mtk_gemm_bf16_nt_256x256_s, DT_BF16, 256, 256, OpRows<256>, OpRows<256>)
SERIAL_KERNEL(mtk_gemm_bf16_nt_128x128_s, DT_BF16, 128, 128, OpRows<128>, OpRows<128>)
SERIAL_KERNEL(mtk_gemm_bf16_nn_256x256_s, DT_BF16, 256, 256, OpRows<256>, OpColsT<256>)
SERIAL_KERNEL(mtk_gemm_bf16_nn_128x128_s, DT_BF16, 128, 128, OpRows<128>, OpColsT<128>)
SERIAL_KERNEL(mtk_gemm_bf16_tt_256x256_s, DT_BF16, 256, 256, OpColsT<256>, OpRows<256>)
SERIAL_KERNEL(mtk_gemm_bf16_tt_128x128_s, DT_BF16, 128, 128, OpColsT<128>, OpRows<128>)
SERIAL_KERNEL(mtk_gemm_bf16_tn_256x256_s, DT_BF16, 256, 256, OpColsT<256>, OpColsT<256>)
SERIAL_KERNEL(mtk_gemm_bf16_tn_128x128_s, DT_BF16, 128, 128, OpColsT<128>, OpColsT<128>)

TILE_KERNEL(mtk_gemm_bf16_nt_256x256_v1, DT_BF16, 256, 256, 2, 2, A_MK, B_NK, 1, 1)
TILE_KERNEL(mtk_gemm_bf16_nt_128x128_v1, DT_BF16, 128, 128, 2, 2, A_MK, B_NK, 1, 1)
TILE_KERNEL(mtk_gemm_bf16_nn_256x256_v1, DT_BF16, 256, 256, 2, 2, A_MK, B_KN, 1, 1)
TILE_KERNEL(mtk_gemm_bf16_nn_128x128_v1, DT_BF16, 128, 128, 2, 2, A_MK, B_KN, 1, 1)

extern "C" __global__ void __launch_bounds__(256) mtk_splitk_reduce_bf16(const mtk_reduce_args a) {
  splitk_reduce<DT_BF16>(a);
}
