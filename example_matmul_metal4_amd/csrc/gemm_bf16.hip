// bf16 GEMM kernels (mtk_gemm_bf16_*) and the bf16 split-K second pass.
#define MTK_GEMM_DT mtk::DT_BF16
#define MTK_GEMM_NAME(x) mtk_gemm_bf16_##x
#define MTK_REDUCE_NAME mtk_splitk_reduce_bf16
#include "gemm_kernels.hpp"
