// k_gemv.hip — M=1 quantized GEMV, fused QKV(+bias) and fused gate+up+SiLU
// kernels for gfx950.
//
// One kernel template serves every format and epilogue:
//   1. the workgroup turns the activation vector into limb records in LDS
//      (once per workgroup when all of K fits, else per K-chunk);
//   2. a wave is split into 64/lpr row groups of `lpr` lanes; each group owns
//      RPL consecutive (virtual) rows, lane j walks units j, j+lpr, ... of
//      those rows, reusing one unit of activations for all RPL rows;
//   3. group sums via DPP / ds_swizzle, lane 0 of the group runs the epilogue.
// Virtual rows let one launch cover several matrices: fused QKV maps row r to
// (Q|K|V, local row); fused FFN interleaves gate and up rows so both dots of
// an output land in the same lane.
#include "rt_formats.h"

struct GemvArgs {
    const uint8_t* w[3];
    void* out[3];
    const void* aux[3];  // residual (f32/f16) or f16 bias, per matrix
    const void* x;
    uint32_t n[3];       // rows per matrix
    uint32_t nvrows;     // virtual rows covered by the launch
    uint32_t K;
    uint32_t lpr;        // lanes per row group (1..64, power of two)
    uint32_t xb_chunk;   // activation records staged per LDS pass (multiple of 8)
    uint64_t row_bytes;
};

enum Epi : int {
    EPI_F32 = 0,      // y = v                     (f32 out)
    EPI_F32_ADD = 1,  // y = v + res               (f32 out, f32 residual)
    EPI_F16 = 2,      // y = half(v)
    EPI_F16_ADD = 3,  // y = half(v + float(res16))
    EPI_QKV = 4,      // 3 matrices, no bias
    EPI_QKV_BIAS = 5, // 3 matrices, + float(bias16)
    EPI_FFN = 6,      // act = silu(gate)·up, rows interleaved
};

template <int EPI>
RT_DEV void vrow_map(const GemvArgs& a, uint32_t vr, uint32_t& mat, uint32_t& r) {
    if (EPI == EPI_FFN) {
        mat = vr & 1;
        r = vr >> 1;
    } else if (EPI == EPI_QKV || EPI == EPI_QKV_BIAS) {
        if (vr < a.n[0]) {
            mat = 0; r = vr;
        } else if (vr < a.n[0] + a.n[1]) {
            mat = 1; r = vr - a.n[0];
        } else {
            mat = 2; r = vr - a.n[0] - a.n[1];
        }
    } else {
        mat = 0;
        r = vr;
    }
}

RT_DEV float silu_ref(float g) {
    // x / (1 + exp(-x))  (fused_ffn.metal:24-26; dispatch.rs:1684-1686)
    return g / (1.0f + expf(-g));
}

template <int EPI>
RT_DEV void store_row(const GemvArgs& a, uint32_t vr, float v) {
    uint32_t mat, r;
    vrow_map<EPI>(a, vr, mat, r);
    if (EPI == EPI_F32) {
        ((float*)a.out[0])[r] = v;
    } else if (EPI == EPI_F32_ADD) {
        // read residual[r] then write y[r] in the same lane: y may alias res
        const float res = ((const float*)a.aux[0])[r];
        ((float*)a.out[0])[r] = v + res;
    } else if (EPI == EPI_F16) {
        ((uint16_t*)a.out[0])[r] = f2h(v);
    } else if (EPI == EPI_F16_ADD) {
        const float res = h2f(((const uint16_t*)a.aux[0])[r]);
        ((uint16_t*)a.out[0])[r] = f2h(v + res);
    } else if (EPI == EPI_QKV) {
        ((float*)a.out[mat])[r] = v;
    } else if (EPI == EPI_QKV_BIAS) {
        ((float*)a.out[mat])[r] = v + h2f(((const uint16_t*)a.aux[mat])[r]);
    }
}

template <class F, int EPI, typename XT, int RPL>
RT_DEV void gemv_body(const GemvArgs& a) {
    extern __shared__ XRec xs[];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t lpr = a.lpr;
    const uint32_t g = lane / lpr, j = lane % lpr;
    const uint32_t groups = 64 / lpr;
    const uint32_t vrows_per_wave = groups * RPL;
    const uint32_t vrows_per_wg = nwaves * vrows_per_wave;
    const uint32_t nxb = a.K / 32;
    const uint32_t ntiles = (a.nvrows + vrows_per_wg - 1) / vrows_per_wg;
    const XT* x = (const XT*)a.x;
    const bool one_chunk = a.xb_chunk >= nxb;

    if (one_chunk) {
        stage_x_limbs<XT, F::Q40PERM>(x, 0, nxb, xs);
        __syncthreads();
    }

    for (uint32_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const uint32_t vr0 = tile * vrows_per_wg + wave * vrows_per_wave + g * RPL;
        const uint8_t* rowp[RPL];
#pragma unroll
        for (int i = 0; i < RPL; ++i) {
            uint32_t vr = vr0 + i;
            if (vr >= a.nvrows) vr = a.nvrows - 1;  // clamp loads; store is skipped
            uint32_t mat, r;
            vrow_map<EPI>(a, vr, mat, r);
            rowp[i] = a.w[mat] + (size_t)r * a.row_bytes;
        }
        float acc[RPL];
#pragma unroll
        for (int i = 0; i < RPL; ++i) acc[i] = 0.0f;

        for (uint32_t xc = 0; xc < nxb; xc += a.xb_chunk) {
            const uint32_t nx = min(a.xb_chunk, nxb - xc);
            if (!one_chunk) {
                __syncthreads();
                stage_x_limbs<XT, F::Q40PERM>(x, xc, nx, xs);
                __syncthreads();
            }
            const uint32_t units = nx * 32 / F::UNIT_EL;
            const uint32_t u0 = xc * 32 / F::UNIT_EL;
            for (uint32_t uu = j; uu < units; uu += lpr) {
                typename F::Raw raw[RPL];
#pragma unroll
                for (int i = 0; i < RPL; ++i) F::load(rowp[i], u0 + uu, raw[i]);
                typename F::XU xu;
                F::load_x(xs, uu, xu);
#pragma unroll
                for (int i = 0; i < RPL; ++i) acc[i] += F::dot(raw[i], xu);
            }
        }
#pragma unroll
        for (int i = 0; i < RPL; ++i) acc[i] = group_sum(acc[i], (int)lpr);

        if (j == 0) {
            if (EPI == EPI_FFN) {
#pragma unroll
                for (int i = 0; i + 1 < RPL; i += 2) {
                    const uint32_t vr = vr0 + i;
                    if (vr + 1 < a.nvrows) {
                        // act[r] = silu(gate)·up  (fused_ffn.metal:90-92)
                        ((float*)a.out[0])[vr >> 1] = silu_ref(acc[i]) * acc[i + 1];
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < RPL; ++i) {
                    if (vr0 + i < a.nvrows) store_row<EPI>(a, vr0 + i, acc[i]);
                }
            }
        }
    }
}

#define RT_GEMV_KERNEL(NAME, FMT, EPI, XT, RPL)                                   \
    extern "C" __global__ void __launch_bounds__(256) NAME(GemvArgs a) {         \
        gemv_body<FMT, EPI, XT, RPL>(a);                                          \
    }

// Q8_0 (gemv_q8_0.metal, gemv_multirow.metal, fused_qkv.metal, fused_ffn.metal)
RT_GEMV_KERNEL(k_gemv_q8_0_f32_f32, FmtQ8_0, EPI_F32, float, 2)
RT_GEMV_KERNEL(k_gemv_q8_0_f32_f32add, FmtQ8_0, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL(k_gemv_q8_0_f32_f16, FmtQ8_0, EPI_F16, float, 2)
RT_GEMV_KERNEL(k_gemv_q8_0_f16_f16, FmtQ8_0, EPI_F16, uint16_t, 2)
RT_GEMV_KERNEL(k_gemv_q8_0_f16_f16add, FmtQ8_0, EPI_F16_ADD, uint16_t, 2)
RT_GEMV_KERNEL(k_gemv_q8_0_f16_f32add, FmtQ8_0, EPI_F32_ADD, uint16_t, 2)
RT_GEMV_KERNEL(k_qkv_q8_0, FmtQ8_0, EPI_QKV, float, 2)
RT_GEMV_KERNEL(k_qkv_bias_q8_0, FmtQ8_0, EPI_QKV_BIAS, float, 2)
RT_GEMV_KERNEL(k_ffn_q8_0, FmtQ8_0, EPI_FFN, float, 2)
// Q4_0 (gemv_q4_0.metal)
RT_GEMV_KERNEL(k_gemv_q4_0_f32_f32, FmtQ4_0, EPI_F32, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f32_f32add, FmtQ4_0, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f32_f16, FmtQ4_0, EPI_F16, float, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f16_f16, FmtQ4_0, EPI_F16, uint16_t, 2)
RT_GEMV_KERNEL(k_gemv_q4_0_f16_f16add, FmtQ4_0, EPI_F16_ADD, uint16_t, 2)
RT_GEMV_KERNEL(k_qkv_bias_q4_0, FmtQ4_0, EPI_QKV_BIAS, float, 2)
RT_GEMV_KERNEL(k_ffn_q4_0, FmtQ4_0, EPI_FFN, float, 2)
// Q4_K (gemv_q4k.metal)
RT_GEMV_KERNEL(k_gemv_q4k_f32_f32, FmtQ4K, EPI_F32, float, 2)
RT_GEMV_KERNEL(k_gemv_q4k_f32_f32add, FmtQ4K, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL(k_gemv_q4k_f16_f16, FmtQ4K, EPI_F16, uint16_t, 2)
RT_GEMV_KERNEL(k_gemv_q4k_f16_f16add, FmtQ4K, EPI_F16_ADD, uint16_t, 2)
RT_GEMV_KERNEL(k_gemv_q4k_f16_f32add, FmtQ4K, EPI_F32_ADD, uint16_t, 2)
RT_GEMV_KERNEL(k_ffn_q4k, FmtQ4K, EPI_FFN, float, 2)
// Q6_K (new: the reference runs Q6_K through f16-dequantised weights)
RT_GEMV_KERNEL(k_gemv_q6k_f32_f32, FmtQ6K, EPI_F32, float, 2)
RT_GEMV_KERNEL(k_gemv_q6k_f32_f32add, FmtQ6K, EPI_F32_ADD, float, 2)
RT_GEMV_KERNEL(k_gemv_q6k_f32_f16, FmtQ6K, EPI_F16, float, 2)
