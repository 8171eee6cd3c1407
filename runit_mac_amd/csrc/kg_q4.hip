// kg_q4.hip — GEMV-family kernels of rt_gemv.h for Q4_0 and Q4_K (reference layouts).
#include "rt_gemv.h"

// Q4_0 (gemv_q4_0.metal)
RT_GEMV_KERNEL(k_gemv_q4_0_f32_f32, FmtQ4_0, EPI_F32, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f32_f32add, FmtQ4_0, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f32_f16, FmtQ4_0, EPI_F16, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f16_f16, FmtQ4_0, EPI_F16, uint16_t, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f16_f16add, FmtQ4_0, EPI_F16_ADD, uint16_t, 2)
RT_GEMV_KERNEL(k_qkv_bias_q4_0, FmtQ4_0, EPI_QKV_BIAS, float, 2)
RT_GEMV_KERNEL(k_ffn_q4_0, FmtQ4_0, EPI_FFN, float, 2)
RT_GEMV_KERNEL_S(k_gemv_q4_0_f32_f32, FmtQ4_0S, EPI_F32, float, 4)
RT_GEMV_KERNEL_S(k_gemv_q4_0_f32_f32add, FmtQ4_0S, EPI_F32_ADD, float, 4)
RT_GEMV_KERNEL_S(k_gemv_q4_0_f32_f16, FmtQ4_0S, EPI_F16, float, 4)
RT_GEMV_KERNEL_S(k_gemv_q4_0_f16_f16, FmtQ4_0S, EPI_F16, uint16_t, 4)
RT_GEMV_KERNEL_S(k_gemv_q4_0_f16_f16add, FmtQ4_0S, EPI_F16_ADD, uint16_t, 4)
RT_GEMV_KERNEL_S(k_qkv_bias_q4_0, FmtQ4_0S, EPI_QKV_BIAS, float, 4)
RT_GEMV_KERNEL_S(k_ffn_q4_0, FmtQ4_0S, EPI_FFN, float, 4)
// Q4_K (gemv_q4k.metal)
RT_GEMV_KERNEL(k_gemv_q4k_f32_f32, FmtQ4K, EPI_F32, float, 1)
RT_GEMV_KERNEL(k_gemv_q4k_f32_f32add, FmtQ4K, EPI_F32_ADD, float, 1)
RT_GEMV_KERNEL(k_gemv_q4k_f16_f16, FmtQ4K, EPI_F16, uint16_t, 1)
RT_GEMV_KERNEL(k_gemv_q4k_f16_f16add, FmtQ4K, EPI_F16_ADD, uint16_t, 1)
RT_GEMV_KERNEL(k_gemv_q4k_f16_f32add, FmtQ4K, EPI_F32_ADD, uint16_t, 1)
RT_GEMV_KERNEL(k_ffn_q4k, FmtQ4K, EPI_FFN, float, 1)
// all-Q4_K projections (the other layers of Q4_K_M files)
RT_GEMV_KERNEL(k_qkv_bias_q4k, FmtQ4K, EPI_QKV_BIAS, float, 1)
RT_GEMV_KERNEL(k_qkv_q4k, FmtQ4K, EPI_QKV, float, 1)

// Attention output projection with the split merge folded into the staging
// (the Q4_K form of k_gemv_q8_0_attn_f32add: decode_attention's merge, then
// the projection + residual, forward.rs:1588-1619); whole K in one slice
// round of up to 1024 threads (q_dim ≤ 4096).
extern "C" __global__ void __launch_bounds__(1024) k_gemv_q4k_attn_f32add_r1(GemvArgs a) {
    gemv_mq_body<FmtQ4K, EPI_F32_ADD, AttnX, 1, GEMV_PF1>(a);
}
