// kg_q5.hip — GEMV-family kernels of rt_gemv.h for Q5_0 and Q5_K.
#include "rt_gemv.h"

// Q5_0 / Q5_K (new: the reference dequantises both on the CPU,
// forward.rs:900-920 and 979-1012)
RT_GEMV_KERNEL(k_gemv_q5_0_f32_f32, FmtQ5_0, EPI_F32, float, 2)
RT_GEMV_KERNEL(k_gemv_q5_0_f32_f32add, FmtQ5_0, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL(k_gemv_q5_0_f32_f16, FmtQ5_0, EPI_F16, float, 2)
RT_GEMV_KERNEL(k_qkv_bias_q5_0, FmtQ5_0, EPI_QKV_BIAS, float, 2)
RT_GEMV_KERNEL(k_ffn_q5_0, FmtQ5_0, EPI_FFN, float, 2)
RT_GEMV_KERNEL_S(k_gemv_q5_0_f32_f32, FmtQ5_0S, EPI_F32, float, 4)
RT_GEMV_KERNEL_S(k_gemv_q5_0_f32_f32add, FmtQ5_0S, EPI_F32_ADD, float, 4)
RT_GEMV_KERNEL_S(k_gemv_q5_0_f32_f16, FmtQ5_0S, EPI_F16, float, 4)
RT_GEMV_KERNEL_S(k_qkv_bias_q5_0, FmtQ5_0S, EPI_QKV_BIAS, float, 4)
RT_GEMV_KERNEL_S(k_ffn_q5_0, FmtQ5_0S, EPI_FFN, float, 4)
RT_GEMV_KERNEL(k_gemv_q5k_f32_f32, FmtQ5K, EPI_F32, float, 1)
RT_GEMV_KERNEL(k_gemv_q5k_f32_f32add, FmtQ5K, EPI_F32_ADD, float, 1)
RT_GEMV_KERNEL(k_gemv_q5k_f32_f16, FmtQ5K, EPI_F16, float, 1)
RT_GEMV_KERNEL(k_qkv_bias_q5k, FmtQ5K, EPI_QKV_BIAS, float, 1)
RT_GEMV_KERNEL(k_ffn_q5k, FmtQ5K, EPI_FFN, float, 1)
