// k_decode.hip — the non-GEMV kernels of one decode step: RMSNorm, RoPE,
// KV-cache scatter, decode attention (plain and fused with RoPE + cache
// write) and the Q8_0 embedding lookup.
#include "rt_attn.h"

// rms_norm_f32_f32_f32g (norm.metal:126-154): one workgroup per row,
// y = x · rsqrt(mean(x²) + eps) · γ.  y may alias x.
// Rows of up to 8 float4 per thread (8192 elements at 256 threads) whose
// start is 16-byte aligned are read in one round trip: every x and γ load is
// issued before the first is used, and x stays in registers for the second
// pass.  Other rows take the element loop.
extern "C" __global__ void __launch_bounds__(256)
k_rms_norm_f32g(const float* x, float* y, const float* gamma, float eps, uint32_t hidden) {
    __shared__ float red[16];
    constexpr uint32_t MAXV = 8;
    const float* xr = x + (size_t)blockIdx.x * hidden;
    float* yr = y + (size_t)blockIdx.x * hidden;
    const uint32_t tid = threadIdx.x, nt = wg_threads();
    const uint32_t n4 = hidden / 4;
    const bool vec = hidden % 4 == 0 && n4 <= MAXV * nt &&
                     (((uintptr_t)xr | (uintptr_t)yr | (uintptr_t)gamma) & 15) == 0;
    if (vec) {
        const f32x4* x4 = (const f32x4*)xr;
        const f32x4* g4 = (const f32x4*)gamma;
        f32x4 xv[MAXV], gv[MAXV];
#pragma unroll
        for (uint32_t j = 0; j < MAXV; ++j) {
            const uint32_t i = tid + j * nt;
            xv[j] = i < n4 ? x4[i] : f32x4{0, 0, 0, 0};
            gv[j] = i < n4 ? g4[i] : f32x4{0, 0, 0, 0};
        }
        float ss = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < MAXV; ++j)
            ss += xv[j].x * xv[j].x + xv[j].y * xv[j].y + xv[j].z * xv[j].z + xv[j].w * xv[j].w;
        ss = block_sum(ss, red);
        const float rms = rsqrtf(ss / (float)hidden + eps);
        f32x4* y4 = (f32x4*)yr;
#pragma unroll
        for (uint32_t j = 0; j < MAXV; ++j) {
            const uint32_t i = tid + j * nt;
            if (i < n4)
                y4[i] = f32x4{xv[j].x * rms * gv[j].x, xv[j].y * rms * gv[j].y,
                              xv[j].z * rms * gv[j].z, xv[j].w * rms * gv[j].w};
        }
        return;
    }
    float ss = 0.0f;
    for (uint32_t i = tid; i < hidden; i += nt) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    const float rms = rsqrtf(ss / (float)hidden + eps);
    for (uint32_t i = tid; i < hidden; i += nt) yr[i] = xr[i] * rms * gamma[i];
}

// fused_rope_qk_f32 (fused_rope.metal:17-56): non-interleaved pairs (d, d+hd/2).
extern "C" __global__ void __launch_bounds__(256)
k_rope_qk_f32(float* Q, float* K, uint32_t head_dim, uint32_t q_heads, uint32_t kv_heads,
              uint32_t pos, float theta) {
    const uint32_t half = head_dim / 2;
    const uint32_t d = blockIdx.x * wg_threads() + threadIdx.x;
    const uint32_t h = blockIdx.y;
    if (d >= half) return;
    float c, s;
    rope_cs(d, head_dim, pos, theta, c, s);
    if (h < q_heads) {
        float* q = Q + (size_t)h * head_dim;
        const float r = q[d], i = q[d + half];
        q[d] = r * c - i * s;
        q[d + half] = r * s + i * c;
    }
    if (h < kv_heads) {
        float* k = K + (size_t)h * head_dim;
        const float r = k[d], i = k[d + half];
        k[d] = r * c - i * s;
        k[d + half] = r * s + i * c;
    }
}

// kv_copy_to_cache_f32 (activation.metal:30-45): dst[(h·max_seq + pos)·hd + d].
extern "C" __global__ void __launch_bounds__(256)
k_kv_copy_f32(const float* src, float* dst, uint32_t pos, uint32_t max_seq, uint32_t head_dim,
              uint32_t n) {
    const uint32_t t = blockIdx.x * wg_threads() + threadIdx.x;
    if (t >= n) return;
    const uint32_t h = t / head_dim, d = t % head_dim;
    dst[((size_t)h * max_seq + pos) * head_dim + d] = src[t];
}

#define RT_ATTN_KERNELS(HD)                                                                \
    extern "C" __global__ void __launch_bounds__(256 * attn_hg<HD>())                     \
        k_decode_attention_f32_hd##HD(AttnArgs a) {                                        \
        attn_split<HD, false, attn_hg<HD>(), attn_gm<HD>()>(a, blockIdx.x, gridDim.x,      \
                                                           blockIdx.y, blockIdx.z);        \
    }                                                                                      \
    extern "C" __global__ void __launch_bounds__(256 * attn_hg<HD>())                     \
        k_attn_rope_f32_hd##HD(AttnArgs a) {                                               \
        attn_split<HD, true, attn_hg<HD>(), attn_gm<HD>()>(a, blockIdx.x, gridDim.x,       \
                                                          blockIdx.y, blockIdx.z);         \
    }
RT_ATTN_KERNELS(64)
RT_ATTN_KERNELS(128)
RT_ATTN_KERNELS(256)

// add_f16_into_f32 (dispatch.rs:316-330): acc[i] += f32(src[i]), the bias add
// of the reference's separate-dispatch Q/K/V fallback (forward.rs:1561-1568).
extern "C" __global__ void __launch_bounds__(256)
k_add_f16_into_f32(const uint16_t* __restrict__ src, float* __restrict__ acc, uint32_t n) {
    for (uint32_t i = threadIdx.x + blockIdx.x * wg_threads(); i < n; i += wg_threads() * gridDim.x)
        acc[i] += h2f(src[i]);
}
