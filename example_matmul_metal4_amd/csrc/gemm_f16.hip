// fp16 GEMM kernels (mtk_gemm_f16_*) and the fp16 split-K second pass.
#define MTK_GEMM_DT mtk::DT_F16
#define MTK_GEMM_NAME(x) mtk_gemm_f16_##x
#define MTK_REDUCE_NAME mtk_splitk_reduce_f16
#include "gemm_kernels.hpp"
