// kls_q6k.hip — LDS-streamed GEMV kernels of rt_gemv_ls.h (q6k).
#include "rt_gemv_ls.h"

RT_GEMV_LSB(k_gemv_q6k_f32_f32, FmtQ6KB, EPI_F32, float, 256)
RT_GEMV_LSB(k_gemv_q6k_f32_f32add, FmtQ6KB, EPI_F32_ADD, float, 256)

// Workgroup-local K split of the Q6_K down projections (64-element units:
// ~120 registers, so 16 waves share one copy of the activation records)
RT_GEMV_LSK(k_gemv_q6k_f32_f32add, FmtQ6K, EPI_F32_ADD, float, 1024)

// VALU-dot twin of the LM-head kernels (dot-form A/B)
RT_GEMV_LSBV(k_gemv_q6k_f32_f32, FmtQ6KB, EPI_F32, float, 256)
