// kg_q6k.hip — GEMV-family kernels of rt_gemv.h for Q6_K (reference layout).
#include "rt_gemv.h"

// Q6_K (new: the reference runs Q6_K through f16-dequantised weights)
// (matrix-core path: one super-block per lane; chunked path: 64-element units)
RT_GEMV_KERNEL2W(k_gemv_q6k_f32_f32, FmtQ6KB, FmtQ6K, EPI_F32, float, 1, RT_Q6K_WPE)
RT_GEMV_KERNEL2W(k_gemv_q6k_f32_f32add, FmtQ6KB, FmtQ6K, EPI_F32_ADD, float, 1, RT_Q6K_WPE)
RT_GEMV_KERNEL2W(k_gemv_q6k_f32_f16, FmtQ6KB, FmtQ6K, EPI_F16, float, 1, RT_Q6K_WPE)

RT_GEMV_PAIR(k_qkv2_bias_q4k_q6k, FmtQ4K, FmtQ6K, EPI_QKV_BIAS)
RT_GEMV_PAIR(k_qkv2_q4k_q6k, FmtQ4K, FmtQ6K, EPI_QKV)
