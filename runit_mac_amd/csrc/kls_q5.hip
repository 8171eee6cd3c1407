// kls_q5.hip — LDS-streamed GEMV kernels of rt_gemv_ls.h (q5).
#include "rt_gemv_ls.h"

RT_GEMV_LS(k_gemv_q5_0_f32_f32, FmtQ5_0, EPI_F32, float)
RT_GEMV_LS(k_gemv_q5_0_f32_f32add, FmtQ5_0, EPI_F32_ADD, float)
RT_GEMV_LS(k_ffn_q5_0, FmtQ5_0, EPI_FFN, float)
RT_GEMV_LS(k_gemv_q5k_f32_f32, FmtQ5K, EPI_F32, float)
RT_GEMV_LS(k_gemv_q5k_f32_f32add, FmtQ5K, EPI_F32_ADD, float)
RT_GEMV_LS(k_ffn_q5k, FmtQ5K, EPI_FFN, float)
RT_GEMV_LSK(k_gemv_q5k_f32_f32, FmtQ5K, EPI_F32, float, 1024)
RT_GEMV_LSK(k_gemv_q5k_f32_f32add, FmtQ5K, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_gemv_q5_0_f32_f32add, FmtQ5_0, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_ffn_q5k, FmtQ5K, EPI_FFN, float, 1024)
RT_GEMV_LSK(k_ffn_q5_0, FmtQ5_0, EPI_FFN, float, 1024)
RT_GEMV_LSK(k_gemv_q5_0_f32_f32, FmtQ5_0, EPI_F32, float, 1024)
