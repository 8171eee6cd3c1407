// kg_ggml.hip — GEMV-family kernels of rt_gemv.h for ggml layouts (upstream GGUF files).
#include "rt_gemv.h"

// ggml layouts of Q4_0, Q4_K, Q5_K and Q6_K (upstream GGUF files; the
// reference's own layouts differ, see the formats)
RT_GEMV_KERNEL(k_gemv_q4_0g_f32_f32, FmtQ4_0G, EPI_F32, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0g_f32_f32add, FmtQ4_0G, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0g_f32_f16, FmtQ4_0G, EPI_F16, float, 2)
RT_GEMV_KERNEL(k_ffn_q4_0g, FmtQ4_0G, EPI_FFN, float, 2)
RT_GEMV_KERNEL_S(k_gemv_q4_0g_f32_f32, FmtQ4_0GS, EPI_F32, float, 4)
RT_GEMV_KERNEL_S(k_gemv_q4_0g_f32_f32add, FmtQ4_0GS, EPI_F32_ADD, float, 4)
RT_GEMV_KERNEL_S(k_gemv_q4_0g_f32_f16, FmtQ4_0GS, EPI_F16, float, 4)
RT_GEMV_KERNEL_S(k_ffn_q4_0g, FmtQ4_0GS, EPI_FFN, float, 4)
RT_GEMV_KERNEL(k_gemv_q4kg_f32_f32, FmtQ4KG, EPI_F32, float, 1)
RT_GEMV_KERNEL(k_gemv_q4kg_f32_f32add, FmtQ4KG, EPI_F32_ADD, float, 1)
RT_GEMV_KERNEL(k_gemv_q4kg_f32_f16, FmtQ4KG, EPI_F16, float, 1)
RT_GEMV_KERNEL(k_ffn_q4kg, FmtQ4KG, EPI_FFN, float, 1)
RT_GEMV_KERNEL(k_gemv_q5kg_f32_f32, FmtQ5KG, EPI_F32, float, 1)
RT_GEMV_KERNEL(k_gemv_q5kg_f32_f32add, FmtQ5KG, EPI_F32_ADD, float, 1)
RT_GEMV_KERNEL(k_gemv_q5kg_f32_f16, FmtQ5KG, EPI_F16, float, 1)
RT_GEMV_KERNEL(k_ffn_q5kg, FmtQ5KG, EPI_FFN, float, 1)
RT_GEMV_KERNEL2W(k_gemv_q6kg_f32_f32, FmtQ6KGB, FmtQ6KG, EPI_F32, float, 1, RT_Q6K_WPE)
RT_GEMV_KERNEL2W(k_gemv_q6kg_f32_f32add, FmtQ6KGB, FmtQ6KG, EPI_F32_ADD, float, 1, RT_Q6K_WPE)
RT_GEMV_KERNEL2W(k_gemv_q6kg_f32_f16, FmtQ6KGB, FmtQ6KG, EPI_F16, float, 1, RT_Q6K_WPE)
RT_GEMV_PAIR(k_qkv2_bias_q4kg_q6kg, FmtQ4KG, FmtQ6KG, EPI_QKV_BIAS)
RT_GEMV_PAIR(k_qkv2_q4kg_q6kg, FmtQ4KG, FmtQ6KG, EPI_QKV)
RT_GEMV_KERNEL(k_qkv_bias_q4kg, FmtQ4KG, EPI_QKV_BIAS, float, 1)
RT_GEMV_KERNEL(k_qkv_q4kg, FmtQ4KG, EPI_QKV, float, 1)

// ggml-layout Q4_K form of k_gemv_q4k_attn_f32add (split merge in the staging)
extern "C" __global__ void __launch_bounds__(1024) k_gemv_q4kg_attn_f32add_r1(GemvArgs a) {
    gemv_mq_body<FmtQ4KG, EPI_F32_ADD, AttnX, 1, GEMV_PF1>(a);
}
