// kls_q4.hip — LDS-streamed GEMV kernels of rt_gemv_ls.h (q4).
#include "rt_gemv_ls.h"

RT_GEMV_LS(k_gemv_q4_0_f32_f32, FmtQ4_0, EPI_F32, float)
RT_GEMV_LS(k_gemv_q4_0_f32_f32add, FmtQ4_0, EPI_F32_ADD, float)
RT_GEMV_LS(k_qkv_bias_q4_0, FmtQ4_0, EPI_QKV_BIAS, float)
RT_GEMV_LS(k_ffn_q4_0, FmtQ4_0, EPI_FFN, float)
RT_GEMV_LS(k_gemv_q4k_f32_f32, FmtQ4K, EPI_F32, float)
RT_GEMV_LS(k_gemv_q4k_f32_f32add, FmtQ4K, EPI_F32_ADD, float)
RT_GEMV_LS(k_ffn_q4k, FmtQ4K, EPI_FFN, float)
RT_GEMV_LSK(k_gemv_q4_0_f32_f32, FmtQ4_0, EPI_F32, float, 1024)
RT_GEMV_LSK(k_gemv_q4_0_f32_f32add, FmtQ4_0, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_ffn_q4_0, FmtQ4_0, EPI_FFN, float, 1024)
RT_GEMV_LSK(k_gemv_q4k_f32_f32, FmtQ4K, EPI_F32, float, 1024)
RT_GEMV_LSK(k_gemv_q4k_f32_f32add, FmtQ4K, EPI_F32_ADD, float, 1024)
RT_GEMV_LSBV(k_ffn_q4k, FmtQ4K, EPI_FFN, float, 1024)
