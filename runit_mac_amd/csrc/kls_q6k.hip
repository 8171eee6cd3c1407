// kls_q6k.hip — LDS-streamed GEMV kernels of rt_gemv_ls.h (q6k).
#include "rt_gemv_ls.h"

RT_GEMV_LSB(k_gemv_q6k_f32_f32, FmtQ6KB, EPI_F32, float, 256)
RT_GEMV_LSB(k_gemv_q6k_f32_f32add, FmtQ6KB, EPI_F32_ADD, float, 256)

// Workgroup-local K split of the Q6_K down projections (64-element units:
// ~120 registers, so 16 waves share one copy of the activation records)
RT_GEMV_LSK(k_gemv_q6k_f32_f32add, FmtQ6K, EPI_F32_ADD, float, 1024)

// VALU-dot twin of the LM-head kernels (dot-form A/B)
RT_GEMV_LSBV(k_gemv_q6k_f32_f32, FmtQ6KB, EPI_F32, float, 256)

// Q/K (Q4_K, 2 KB rows) on the small-launch body and V (Q6_K) on the
// matrix-core body, in one 512-thread launch: workgroups [0, b.blk0) run
// part a, the rest part b
#define RT_QKV_SMR(NAME, FA, FB, EPI)                                                        \
    extern "C" __global__ void __launch_bounds__(512) NAME##_smr(GemvArgs a, GemvArgs b) {  \
        if (blockIdx.x < b.blk0)                                                             \
            gemv_sm_body<FA, EPI, float, 2>(a);                                              \
        else                                                                                 \
            gemv_mq_body<FB, EPI, float, 1, (fmt_pf<FB>() ? fmt_pf<FB>() : GEMV_PF1)>(b);    \
    }
RT_QKV_SMR(k_qkv2_bias_q4k_q6k, FmtQ4K, FmtQ6K, EPI_QKV_BIAS)
RT_QKV_SMR(k_qkv2_q4k_q6k, FmtQ4K, FmtQ6K, EPI_QKV)
