// kg_q8_0.hip — GEMV-family kernels of rt_gemv.h for Q8_0.
#include "rt_gemv.h"

RT_GEMV_KERNEL512(k_gemv_q8_0_f32_f32, FmtQ8_0, EPI_F32, float, 1)
RT_GEMV_KERNEL512(k_gemv_q8_0_f32_f32add, FmtQ8_0, EPI_F32_ADD, float, 1)
RT_GEMV_KERNEL512(k_gemv_q8_0_f32_f16, FmtQ8_0, EPI_F16, float, 1)
RT_GEMV_KERNEL512(k_gemv_q8_0_f16_f16, FmtQ8_0, EPI_F16, uint16_t, 1)
RT_GEMV_KERNEL512(k_gemv_q8_0_f16_f16add, FmtQ8_0, EPI_F16_ADD, uint16_t, 1)
RT_GEMV_KERNEL512(k_gemv_q8_0_f16_f32add, FmtQ8_0, EPI_F32_ADD, uint16_t, 1)
RT_GEMV_KERNEL512(k_qkv_q8_0, FmtQ8_0, EPI_QKV, float, 1)
RT_GEMV_KERNEL512(k_qkv_bias_q8_0, FmtQ8_0, EPI_QKV_BIAS, float, 1)
RT_GEMV_KERNEL512(k_ffn_q8_0, FmtQ8_0, EPI_FFN, float, 1)
RT_GEMV_KERNEL_S(k_gemv_q8_0_f32_f32, FmtQ8_0S, EPI_F32, float, 2)
RT_GEMV_KERNEL_S(k_gemv_q8_0_f32_f32add, FmtQ8_0S, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL_S(k_gemv_q8_0_f32_f16, FmtQ8_0S, EPI_F16, float, 2)
RT_GEMV_KERNEL_S(k_gemv_q8_0_f16_f16, FmtQ8_0S, EPI_F16, uint16_t, 2)
RT_GEMV_KERNEL_S(k_gemv_q8_0_f16_f16add, FmtQ8_0S, EPI_F16_ADD, uint16_t, 2)
RT_GEMV_KERNEL_S(k_gemv_q8_0_f16_f32add, FmtQ8_0S, EPI_F32_ADD, uint16_t, 2)
RT_GEMV_KERNEL_S(k_qkv_q8_0, FmtQ8_0S, EPI_QKV, float, 2)
RT_GEMV_KERNEL_S(k_qkv_bias_q8_0, FmtQ8_0S, EPI_QKV_BIAS, float, 2)
RT_GEMV_KERNEL_S(k_ffn_q8_0, FmtQ8_0S, EPI_FFN, float, 2)

// Attention output projection with the split merge folded into the staging
// (decode_attention's merge, then gemv_q8_0_add_f32_f32in: forward.rs:1588-
// 1619); one workgroup form only (matrix-core body, whole K, one slice round).
extern "C" __global__ void __launch_bounds__(512) k_gemv_q8_0_attn_f32add_r1(GemvArgs a) {
    gemv_mq_body<FmtQ8_0, EPI_F32_ADD, AttnX, 1, fmt_pf<FmtQ8_0>()>(a);
}

extern "C" __global__ void __launch_bounds__(256)
k_act_limbs_f32(const float* x, XRec* out, uint32_t nxb) { act_limbs_body<float, false>(x, out, nxb); }
extern "C" __global__ void __launch_bounds__(256)
k_act_limbs_f32_q40(const float* x, XRec* out, uint32_t nxb) { act_limbs_body<float, true>(x, out, nxb); }
extern "C" __global__ void __launch_bounds__(256)
k_act_limbs_f16(const uint16_t* x, XRec* out, uint32_t nxb) { act_limbs_body<uint16_t, false>(x, out, nxb); }
extern "C" __global__ void __launch_bounds__(256)
k_act_limbs_f16_q40(const uint16_t* x, XRec* out, uint32_t nxb) { act_limbs_body<uint16_t, true>(x, out, nxb); }
extern "C" __global__ void __launch_bounds__(256)
k_act_limbs_rows_f32(const float* x, const float* gamma, float eps, uint32_t K, XRec* out) {
    act_limbs_rows_body<false>(x, gamma, eps, K, out);
}
extern "C" __global__ void __launch_bounds__(256)
k_act_limbs_rows_f32_q40(const float* x, const float* gamma, float eps, uint32_t K, XRec* out) {
    act_limbs_rows_body<true>(x, gamma, eps, K, out);
}
