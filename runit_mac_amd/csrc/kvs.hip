// kvs.hip — VALU small-launch Q8_0 GEMV kernels of rt_gemv_vs.h: <name>_vs
// (activations as given) and <name>_vsn (RMSNorm(x)·γ computed in the body).
#include "rt_gemv_vs.h"

RT_GEMV_VS(k_gemv_q8_0_f32_f32, EPI_F32, false)
RT_GEMV_VS(k_gemv_q8_0_f32_f32add, EPI_F32_ADD, false)
RT_GEMV_VS(k_qkv_bias_q8_0, EPI_QKV_BIAS, false)
RT_GEMV_VS(k_ffn_q8_0, EPI_FFN, false)
#define RT_GEMV_VSN(NAME, EPI) \
    extern "C" __global__ void __launch_bounds__(1024) NAME##_vsn(GemvArgs a) { gemv_vs_body<EPI, true>(a); }
RT_GEMV_VSN(k_gemv_q8_0_f32_f32, EPI_F32)
RT_GEMV_VSN(k_qkv_bias_q8_0, EPI_QKV_BIAS)
RT_GEMV_VSN(k_ffn_q8_0, EPI_FFN)
