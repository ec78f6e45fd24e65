// Flash-attention forward for head dimensions other than 128 (attention.hpp): padded head
// dimension 64 (D <= 64) and 256 (128 < D <= 256), plus the element-staged kernels for head
// dimensions that are not a multiple of 8 (padded to 64, 128 or 256). D = 128 and 64 < D <= 128
// with D % 8 == 0 use the padded-128 kernels of attention.hip.
#include "attention.hpp"

using namespace mtk;

// DP 64: two wavefronts per SIMD (the 128-query kernel's registers fit twice); DP 256: the output
// accumulators alone take 128 registers per lane, one wavefront per SIMD.
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d64_f16, DT_F16, false, 64, false, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d64_bf16, DT_BF16, false, 64, false, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d64_f16_causal, DT_F16, true, 64, false, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d64_bf16_causal, DT_BF16, true, 64, false, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d256_f16, DT_F16, false, 256, false, 1)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d256_bf16, DT_BF16, false, 256, false, 1)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d256_f16_causal, DT_F16, true, 256, false, 1)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_d256_bf16_causal, DT_BF16, true, 256, false, 1)

// element-staged (any D), padded to 64 / 128 / 256
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g64_f16, DT_F16, false, 64, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g64_bf16, DT_BF16, false, 64, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g64_f16_causal, DT_F16, true, 64, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g64_bf16_causal, DT_BF16, true, 64, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g128_f16, DT_F16, false, 128, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g128_bf16, DT_BF16, false, 128, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g128_f16_causal, DT_F16, true, 128, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g128_bf16_causal, DT_BF16, true, 128, true, 2)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g256_f16, DT_F16, false, 256, true, 1)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g256_bf16, DT_BF16, false, 256, true, 1)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g256_f16_causal, DT_F16, true, 256, true, 1)
MTK_ATTN_FWD_KERNEL(mtk_attn_fwd_g256_bf16_causal, DT_BF16, true, 256, true, 1)
