// kls_ggml.hip — LDS-streamed GEMV kernels of rt_gemv_ls.h (ggml).
#include "rt_gemv_ls.h"

RT_GEMV_LS(k_gemv_q4_0g_f32_f32, FmtQ4_0G, EPI_F32, float)
RT_GEMV_LS(k_gemv_q4_0g_f32_f32add, FmtQ4_0G, EPI_F32_ADD, float)
RT_GEMV_LS(k_ffn_q4_0g, FmtQ4_0G, EPI_FFN, float)
RT_GEMV_LS(k_gemv_q4kg_f32_f32, FmtQ4KG, EPI_F32, float)
RT_GEMV_LS(k_gemv_q4kg_f32_f32add, FmtQ4KG, EPI_F32_ADD, float)
RT_GEMV_LS(k_ffn_q4kg, FmtQ4KG, EPI_FFN, float)
RT_GEMV_LS(k_gemv_q5kg_f32_f32, FmtQ5KG, EPI_F32, float)
RT_GEMV_LS(k_gemv_q5kg_f32_f32add, FmtQ5KG, EPI_F32_ADD, float)
RT_GEMV_LS(k_ffn_q5kg, FmtQ5KG, EPI_FFN, float)
RT_GEMV_LSB(k_gemv_q6kg_f32_f32, FmtQ6KGB, EPI_F32, float, 256)
RT_GEMV_LSB(k_gemv_q6kg_f32_f32add, FmtQ6KGB, EPI_F32_ADD, float, 256)
RT_GEMV_LSK(k_gemv_q4kg_f32_f32add, FmtQ4KG, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_gemv_q5kg_f32_f32add, FmtQ5KG, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_gemv_q4_0g_f32_f32add, FmtQ4_0G, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_gemv_q6kg_f32_f32add, FmtQ6KG, EPI_F32_ADD, float, 1024)
RT_GEMV_LSK(k_ffn_q4kg, FmtQ4KG, EPI_FFN, float, 1024)
RT_GEMV_LSK(k_ffn_q4_0g, FmtQ4_0G, EPI_FFN, float, 1024)
RT_GEMV_LSK(k_ffn_q5kg, FmtQ5KG, EPI_FFN, float, 1024)
RT_GEMV_LSK(k_gemv_q4kg_f32_f32, FmtQ4KG, EPI_F32, float, 1024)
RT_GEMV_LSK(k_gemv_q4_0g_f32_f32, FmtQ4_0G, EPI_F32, float, 1024)
RT_GEMV_LSK(k_gemv_q5kg_f32_f32, FmtQ5KG, EPI_F32, float, 1024)

// Q/K (Q4_K) on the small-launch body and V (Q6_K) on the matrix-core body,
// ggml layouts, in one launch
#define RT_QKV_SMR(NAME, FA, FB, EPI)                                                        \
    extern "C" __global__ void __launch_bounds__(512) NAME##_smr(GemvArgs a, GemvArgs b) {  \
        if (blockIdx.x < b.blk0)                                                             \
            gemv_sm_body<FA, EPI, float, 2>(a);                                              \
        else                                                                                 \
            gemv_mq_body<FB, EPI, float, 1, (fmt_pf<FB>() ? fmt_pf<FB>() : GEMV_PF1)>(b);    \
    }
RT_QKV_SMR(k_qkv2_bias_q4kg_q6kg, FmtQ4KG, FmtQ6KG, EPI_QKV_BIAS)
RT_QKV_SMR(k_qkv2_q4kg_q6kg, FmtQ4KG, FmtQ6KG, EPI_QKV)
