// kls_q8_0.hip — LDS-streamed GEMV kernels of rt_gemv_ls.h (q8_0).
#include "rt_gemv_ls.h"

RT_GEMV_LS(k_gemv_q8_0_f32_f32, FmtQ8_0, EPI_F32, float)
RT_GEMV_LS(k_gemv_q8_0_f32_f32add, FmtQ8_0, EPI_F32_ADD, float)
RT_GEMV_LS(k_gemv_q8_0_f32_f16, FmtQ8_0, EPI_F16, float)
RT_GEMV_LS(k_qkv_bias_q8_0, FmtQ8_0, EPI_QKV_BIAS, float)
RT_GEMV_LS(k_ffn_q8_0, FmtQ8_0, EPI_FFN, float)

// Workgroup-local K split kernels (the residual / plain forms of the down
// projections and the FFNs of long-K models)
RT_GEMV_LSK(k_gemv_q8_0_f32_f32, FmtQ8_0, EPI_F32, float, 1024)
RT_GEMV_LSK(k_gemv_q8_0_f32_f32add, FmtQ8_0, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_ffn_q8_0, FmtQ8_0, EPI_FFN, float, 1024)

// Small-launch kernels (the 0.5B model's norm-fused Q/K/V, O with the
// attention merge, norm-fused gate+up; plain and residual forms)
RT_GEMV_SM(k_gemv_q8_0_f32_f32, FmtQ8_0, EPI_F32, float)
RT_GEMV_SM(k_gemv_q8_0_f32_f32add, FmtQ8_0, EPI_F32_ADD, float)
RT_GEMV_SM(k_qkv_bias_q8_0, FmtQ8_0, EPI_QKV_BIAS, float)
RT_GEMV_SM(k_ffn_q8_0, FmtQ8_0, EPI_FFN, float)
RT_GEMV_SM(k_gemv_q8_0_attn_f32add, FmtQ8_0, EPI_F32_ADD, AttnX)
