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
RT_GEMV_LSK(k_ffn_q4k, FmtQ4K, EPI_FFN, float, 1024)
RT_GEMV_LSBV(k_ffn_q4k, FmtQ4K, EPI_FFN, float, 1024)

// Small-launch kernels for Q4_K rows of ≤ 2 KB (the 7B-shape Q and K
// projections: 6.0 -> 5.6 and 5.65 -> 5.3 µs; the Q4_0 Q/K/V launch ran
// slower in this body, 6.7 against 9.1 µs, and keeps the matrix-core one)
RT_GEMV_SM(k_gemv_q4k_f32_f32, FmtQ4K, EPI_F32, float)
RT_GEMV_SM(k_gemv_q4k_f32_f32add, FmtQ4K, EPI_F32_ADD, float)
