// kgx_rows.hip — multi-row (up to 8 activation rows) matrix-core GEMV
// kernels of rt_gemv.h for the batched verify / prefill step: plain, + residual,
// Q/K/V (+ bias; one to three matrices) and gate+up+SiLU, per format.
#include "rt_gemv.h"

#define RT_ROWS_SET(FN, FMT, LB)                                        \
    RT_GEMV_ROWS(k_gemv_##FN##_f32_f32, FMT, EPI_F32, LB)               \
    RT_GEMV_ROWS(k_gemv_##FN##_f32_f32add, FMT, EPI_F32_ADD, LB)        \
    RT_GEMV_ROWS(k_qkv_bias_##FN, FMT, EPI_QKV_BIAS, LB)                \
    RT_GEMV_ROWS(k_ffn_##FN, FMT, EPI_FFN, LB)

RT_ROWS_SET(q8_0, FmtQ8_0, 512)
RT_ROWS_SET(q4_0, FmtQ4_0, 512)
RT_ROWS_SET(q4k, FmtQ4K, 512)
RT_ROWS_SET(q6k, FmtQ6K, 512)
RT_ROWS_SET(q5_0, FmtQ5_0, 512)
RT_ROWS_SET(q5k, FmtQ5K, 512)
RT_ROWS_SET(q4_0g, FmtQ4_0G, 512)
RT_ROWS_SET(q4kg, FmtQ4KG, 512)
RT_ROWS_SET(q5kg, FmtQ5KG, 512)
RT_ROWS_SET(q6kg, FmtQ6KG, 512)
