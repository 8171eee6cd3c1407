// k_aux.hip — bit-exact dequantisation, argmax and seeded synthetic data.
#include "rt_device.h"

// ───────────────────────────── dequantisation ─────────────────────────────
// One thread per element.  Every product/difference is written with the
// _rn intrinsics so no FMA contraction changes the rounding: the results are
// bit-identical to the reference's f32 CPU decoders.

// Element e of one block, per format.
RT_DEV float q8_0_value(const uint8_t* blk, uint32_t e) {
    const float d = h2f(*(const uint16_t*)blk);
    return __fmul_rn(d, (float)(int8_t)blk[2 + e]);  // forward.rs:951-963: d * qs[i] as i8 as f32
}

RT_DEV float q4_0_value(const uint8_t* blk, uint32_t e) {
    const float d = h2f(*(const uint16_t*)blk);
    const uint8_t byte = blk[2 + e / 2];
    const int nib = (e & 1) ? (byte >> 4) : (byte & 15);
    return __fmul_rn(d, (float)(nib - 8));  // forward.rs:964-978
}

RT_DEV void q4k_scale_min(uint32_t j, const uint8_t* s, uint32_t& sc, uint32_t& m) {
    // get_scale_min_k4 (forward.rs:359-369)
    if (j < 4) {
        sc = s[j] & 63u;
        m = s[j + 4] & 63u;
    } else {
        sc = (s[j + 4] & 15u) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

RT_DEV float q4k_value(const uint8_t* blk, uint32_t e) {
    const float d = h2f(*(const uint16_t*)blk);
    const float dmin = h2f(*(const uint16_t*)(blk + 2));
    const uint32_t j = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    uint32_t sc, m;
    q4k_scale_min(j + 4 * hi, blk + 4, sc, m);
    const uint8_t byte = blk[16 + 32 * j + l];
    const uint32_t q = hi ? (byte >> 4) : (byte & 15u);
    const float dsc = __fmul_rn(d, (float)sc);
    const float mm = __fmul_rn(dmin, (float)m);
    return __fsub_rn(__fmul_rn(dsc, (float)q), mm);  // forward.rs:1043-1053
}

// Q6_K element h + 32t + l; the reference reads scale slot h/16 + 2t
// (forward.rs:935-946), ggml slot h/16 + l/16 + 2t (dequantize_row_q6_K).
template <bool GGML>
RT_DEV float q6k_value(const uint8_t* blk, uint32_t e) {
    const uint32_t h = e & 128u, t = (e >> 5) & 3, l = e & 31;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = h2f(*(const uint16_t*)(blk + 208));
    const uint32_t qlb = ql[h / 2 + l + ((t & 1) ? 32 : 0)];
    const uint32_t lo4 = (t < 2) ? (qlb & 15u) : (qlb >> 4);
    const uint32_t hi2 = (qh[h / 4 + l] >> (2 * t)) & 3u;
    const int q = (int)(lo4 | (hi2 << 4)) - 32;
    const float s = (float)sc[h / 16 + (GGML ? l / 16 : 0) + 2 * t];
    return __fmul_rn(__fmul_rn(d, s), (float)q);
}
RT_DEV float q6k_ref_value(const uint8_t* blk, uint32_t e) { return q6k_value<false>(blk, e); }
RT_DEV float q6kg_value(const uint8_t* blk, uint32_t e) { return q6k_value<true>(blk, e); }

// Q5_0: d f16 @0, qh u32 @2, qs[16] @6; element j < 16 is the low nibble of
// qs[j] with qh bit j on top, element 16 + j the high nibble with bit 16 + j;
// value d·(q − 16) (forward.rs:900-920).
RT_DEV float q5_0_value(const uint8_t* blk, uint32_t e) {
    const float d = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const uint32_t j = e & 15;
    const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                        ((uint32_t)blk[5] << 24);
    const uint32_t byte = blk[6 + j];
    const uint32_t nib = (e < 16) ? (byte & 15u) : (byte >> 4);
    const int q = (int)(nib | (((qh >> e) & 1u) << 4));
    return __fmul_rn(d, (float)(q - 16));
}

// Q5_K: d, dmin f16 @0, scales[12] @4, qh[32] @16, qs[128] @48; element
// 64j + l (+32) takes the low (high) nibble of qs[32j + l], bit (e % 8) of
// qh[e / 8] on top, and (sc, m) of sub-block j (j + 4) (forward.rs:979-1012).
RT_DEV float q5k_value(const uint8_t* blk, uint32_t e) {
    const uint32_t j = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    const float d = h2f(*(const uint16_t*)blk);
    const float dmin = h2f(*(const uint16_t*)(blk + 2));
    uint32_t sc, m;
    q4k_scale_min(j + 4 * hi, blk + 4, sc, m);
    const uint32_t byte = blk[48 + 32 * j + l];
    const uint32_t q = (hi ? (byte >> 4) : (byte & 15u)) | (((blk[16 + e / 8] >> (e % 8)) & 1u) << 4);
    const float dsc = __fmul_rn(d, (float)sc);
    const float mm = __fmul_rn(dmin, (float)m);
    return __fsub_rn(__fmul_rn(dsc, (float)q), mm);
}

// ggml layouts (upstream GGUF files), same rounding as the decoders above.
// Q4_0: element j < 16 low nibble of qs[j], 16 + j its high nibble
// (dequantize_row_q4_0).
RT_DEV float q4_0g_value(const uint8_t* blk, uint32_t e) {
    const float d = h2f(*(const uint16_t*)blk);
    const uint8_t byte = blk[2 + (e & 15)];
    const int nib = (e < 16) ? (byte & 15) : (byte >> 4);
    return __fmul_rn(d, (float)(nib - 8));
}

// Q4_K: chunk j of 64 elements uses sub-blocks 2j (low nibbles) and 2j + 1
// (high nibbles) (dequantize_row_q4_K); Q5_K: as Q4_K (qs at 48) with the
// fifth bit = bit 2j(+1) of qh[l] (dequantize_row_q5_K).
RT_DEV float q4kg_value(const uint8_t* blk, uint32_t e, uint32_t qs_off, bool five,
                        const uint8_t* qh) {
    const float d = h2f(*(const uint16_t*)blk);
    const float dmin = h2f(*(const uint16_t*)(blk + 2));
    const uint32_t j = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    uint32_t sc, m;
    q4k_scale_min(2 * j + hi, blk + 4, sc, m);
    const uint8_t byte = blk[qs_off + 32 * j + l];
    uint32_t q = hi ? (byte >> 4) : (byte & 15u);
    if (five) q |= ((qh[l] >> (2 * j + hi)) & 1u) << 4;
    const float dsc = __fmul_rn(d, (float)sc);
    const float mm = __fmul_rn(dmin, (float)m);
    return __fsub_rn(__fmul_rn(dsc, (float)q), mm);
}
RT_DEV float q4kg_value(const uint8_t* blk, uint32_t e) { return q4kg_value(blk, e, 16, false, nullptr); }
RT_DEV float q5kg_value(const uint8_t* blk, uint32_t e) { return q4kg_value(blk, e, 48, true, blk + 16); }

// Plain f16 / f32 rows (one-element "blocks").
RT_DEV float f16_value(const uint8_t* blk, uint32_t) { return h2f(*(const uint16_t*)blk); }
RT_DEV float f32_value(const uint8_t* blk, uint32_t) { return *(const float*)blk; }

// Per format: k_dequant_<fmt>_f32 — one thread per element of a block
// stream — and k_embed_<fmt>_f32 — the table row of the token id read from
// device memory (the reference copies a dequantised token_embd row into the
// residual stream on the CPU, forward.rs:1494-1505; reading the id on the
// device lets a captured decode step consume the previous step's argmax
// without a host round trip).
#define RT_DEQ_KERNELS(NAME, EL, BY, VALUE)                                                       \
    extern "C" __global__ void __launch_bounds__(256)                                            \
        k_dequant_##NAME##_f32(const uint8_t* __restrict__ in, float* __restrict__ out,          \
                               uint64_t n_el) {                                                  \
        const uint64_t i = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x;                    \
        if (i >= n_el) return;                                                                   \
        out[i] = VALUE(in + (i / (EL)) * (BY), (uint32_t)(i % (EL)));                            \
    }                                                                                            \
    extern "C" __global__ void __launch_bounds__(256)                                            \
        k_embed_##NAME##_f32(const uint8_t* __restrict__ table, const uint32_t* token,           \
                             float* __restrict__ out, uint32_t k) {                              \
        /* grid row y embeds token[y] into out[y·k ..] */                                        \
        const uint8_t* row = table + (size_t)token[blockIdx.y] * (k / (EL)) * (BY);              \
        float* o = out + (size_t)blockIdx.y * k;                                                 \
        for (uint32_t i = threadIdx.x + blockIdx.x * wg_threads(); i < k;                        \
             i += wg_threads() * gridDim.x)                                                      \
            o[i] = VALUE(row + (i / (EL)) * (BY), i % (EL));                                     \
    }
RT_DEQ_KERNELS(q8_0, 32, 34, q8_0_value)
RT_DEQ_KERNELS(q4_0, 32, 18, q4_0_value)
RT_DEQ_KERNELS(q4k, 256, 144, q4k_value)
RT_DEQ_KERNELS(q6k, 256, 210, q6k_ref_value)
RT_DEQ_KERNELS(q5_0, 32, 22, q5_0_value)
RT_DEQ_KERNELS(q5k, 256, 176, q5k_value)
RT_DEQ_KERNELS(q4_0g, 32, 18, q4_0g_value)
RT_DEQ_KERNELS(q4kg, 256, 144, q4kg_value)
RT_DEQ_KERNELS(q5kg, 256, 176, q5kg_value)
RT_DEQ_KERNELS(q6kg, 256, 210, q6kg_value)
RT_DEQ_KERNELS(f16, 1, 2, f16_value)
RT_DEQ_KERNELS(f32, 1, 4, f32_value)

// dequant.metal:53-98 — Q4_K to f16 (value rounded to nearest-even half).
extern "C" __global__ void __launch_bounds__(256)
k_dequant_q4k_f16(const uint8_t* __restrict__ in, uint16_t* __restrict__ out, uint64_t n_el) {
    const uint64_t i = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x;
    if (i >= n_el) return;
    float v = q4k_value(in + (i >> 8) * 144, (uint32_t)(i & 255));
    // Materialise the f32 value before the f16 conversion: the reference
    // rounds to f32 first, then to half (double rounding); without the
    // barrier the compiler fuses d·q − m with the conversion (one rounding).
    asm volatile("" : "+v"(v));
    out[i] = f2h(v);
}

// ───────────────────────────── argmax ─────────────────────────────
// greedy_argmax_f32 (sampler.rs:111-116) folds with Rust's max_by: the
// running best m is replaced by x unless m > x (partial_cmp None → Equal).
// Unrolled, that fold returns:
//   * the index of the last NaN, if the last element is NaN;
//   * otherwise the LAST index of the maximum of the elements after the last
//     NaN (of all elements when there is no NaN).
// Both parts are order-independent reductions, so each workgroup reduces its
// contiguous range with coalesced loads to a state (last NaN index, best
// (value, index) after it), and the last workgroup to finish (arrival
// counter, reset by that workgroup) reduces the states and writes the result.
struct AmState {
    int32_t nan_idx;  // last NaN index in the range, -1 if none
    int32_t idx;      // index of the best element after nan_idx, -1 if none
    float v;
};
constexpr uint32_t AM_T = 256;

RT_DEV bool am_better(float v, int32_t i, float bv, int32_t bi) {
    // later wins ties; the best so far is replaced unless it is strictly greater
    return bi < 0 || v > bv || (v == bv && i > bi);
}

template <typename T>
RT_DEV float am_load(const T* p, uint32_t i);
template <>
RT_DEV float am_load<float>(const float* p, uint32_t i) { return p[i]; }
template <>
RT_DEV float am_load<uint16_t>(const uint16_t* p, uint32_t i) { return h2f(p[i]); }

constexpr int AM_PER = 4;  // elements per thread per workgroup range

// The states reduce in any order: with P the largest NaN index over all of
// them, the result is the later-wins maximum over the states whose best
// index exceeds P (ranges before P hold only indices below it, and the range
// holding P reports its best after P).
template <typename T>
RT_DEV void argmax_body(const T* __restrict__ in, uint32_t* __restrict__ result, uint32_t n,
                        AmState* __restrict__ states, uint32_t* __restrict__ counter) {
    __shared__ int32_t sn[AM_T / 64];
    __shared__ AmState sb[AM_T / 64];
    __shared__ bool last;
    const uint32_t per = (n + gridDim.x - 1) / gridDim.x;
    const uint32_t b0 = blockIdx.x * per, b1 = min(n, b0 + per);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Ranges up to AM_PER·AM_T elements take one pass with all loads issued
    // up front and the values kept for the second reduction; longer ranges
    // loop over such chunks, reading the range twice.
    constexpr uint32_t CH = AM_PER * AM_T;
    const bool one = b1 - b0 <= CH;  // workgroup-uniform
    float xv[AM_PER];
    int32_t nl = -1;
    for (uint32_t c0 = b0; c0 < b1; c0 += CH) {
#pragma unroll
        for (int u = 0; u < AM_PER; ++u) {
            const uint32_t i = c0 + tid + u * AM_T;
            xv[u] = i < b1 ? am_load<T>(in, i) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < AM_PER; ++u) {
            const uint32_t i = c0 + tid + u * AM_T;
            if (i < b1 && xv[u] != xv[u]) nl = (int32_t)i;
        }
    }
    for (int o = 32; o > 0; o >>= 1) nl = max(nl, __shfl_xor(nl, o, 64));
    if (lane == 0) sn[wave] = nl;
    __syncthreads();
    int32_t P = -1;
    for (uint32_t w = 0; w < AM_T / 64; ++w) P = max(P, sn[w]);
    // best element after P (later index wins ties)
    float bv = 0.0f;
    int32_t bi = -1;
    for (uint32_t c0 = b0; c0 < b1; c0 += CH) {
        if (!one) {
#pragma unroll
            for (int u = 0; u < AM_PER; ++u) {
                const uint32_t i = c0 + tid + u * AM_T;
                xv[u] = i < b1 ? am_load<T>(in, i) : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < AM_PER; ++u) {
            const int32_t i = (int32_t)(c0 + tid + u * AM_T);
            if ((uint32_t)i < b1 && i > P && am_better(xv[u], i, bv, bi)) { bv = xv[u]; bi = i; }
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int32_t oi = __shfl_xor(bi, o, 64);
        if (oi >= 0 && am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) sb[wave] = AmState{P, bi, bv};
    __syncthreads();
    if (tid == 0) {
        AmState st{P, -1, 0.0f};
        for (uint32_t w = 0; w < AM_T / 64; ++w)
            if (sb[w].idx >= 0 && am_better(sb[w].v, sb[w].idx, st.v, st.idx)) {
                st.v = sb[w].v;
                st.idx = sb[w].idx;
            }
        AmState* dst = &states[blockIdx.x];
        dev_store(&dst->nan_idx, st.nan_idx);
        dev_store(&dst->idx, st.idx);
        dev_store(&dst->v, st.v);
        dev_stores_done();
        last = arrive(counter) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last || wave != 0) return;
    // the last workgroup's first wave: up to AM_T states, AM_T / 64 per lane
    const uint32_t G = gridDim.x;
    AmState s[AM_T / 64];
    int32_t gp = -1;
#pragma unroll
    for (uint32_t r = 0; r < AM_T / 64; ++r) {
        const uint32_t g = lane + 64 * r;
        s[r] = AmState{-1, -1, 0.0f};
        if (g < G) {
            const AmState* vs = &states[g];
            s[r] = AmState{dev_load(&vs->nan_idx), dev_load(&vs->idx), dev_load(&vs->v)};
        }
        gp = max(gp, s[r].nan_idx);
    }
    for (int o = 32; o > 0; o >>= 1) gp = max(gp, __shfl_xor(gp, o, 64));
    bv = 0.0f;
    bi = -1;
#pragma unroll
    for (uint32_t r = 0; r < AM_T / 64; ++r)
        if (s[r].idx > gp && am_better(s[r].v, s[r].idx, bv, bi)) { bv = s[r].v; bi = s[r].idx; }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int32_t oi = __shfl_xor(bi, o, 64);
        if (oi >= 0 && am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) {
        uint32_t res = 0;
        if (n > 0) {
            if (gp == (int32_t)n - 1 || bi < 0)
                res = gp >= 0 ? (uint32_t)gp : 0u;
            else
                res = (uint32_t)bi;
        }
        result[0] = res;
        dev_store(counter, 0u);  // ready for the next call (also under graph replay)
    }
}

extern "C" __global__ void __launch_bounds__(256)
k_argmax_f32(const float* in, uint32_t* result, uint32_t n, AmState* states, uint32_t* counter) {
    argmax_body<float>(in, result, n, states, counter);
}
extern "C" __global__ void __launch_bounds__(256)
k_argmax_f16(const uint16_t* in, uint32_t* result, uint32_t n, AmState* states, uint32_t* counter) {
    argmax_body<uint16_t>(in, result, n, states, counter);
}

// ───────────────────────────── synthetic data ─────────────────────────────
// Counter-based: element `idx` of stream `seed` is one splitmix64 hash turned
// into a standard normal by Box–Muller (cos branch), so any slice can be
// generated independently and in parallel.

RT_DEV uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// ln(u), u in (0, 1], and cos(2π·v), v in [0, 1), from correctly rounded f32
// operations only (+, −, ×, /, fma; contraction off), so that every machine
// that evaluates the same sequence gets the same bits.  ln: u = m·2^e with m
// in [√½, √2), ln m = 2·atanh(s), s = (m−1)/(m+1), odd series to s^11
// (|s| ≤ 0.172).  cos: quadrant n = rint(4v), r = v − n/4 in [−1/8, 1/8]
// (exact), θ = 2π·r, Taylor series of sin / cos to degree 11 / 10.
RT_DEV float synth_ln(float u) {
#pragma clang fp contract(off)
    int e = 0;
    float m = frexpf(u, &e);  // u = m·2^e, m in [0.5, 1)
    if (m < 0.70710678f) { m = m * 2.0f; e -= 1; }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float z = s * s;
    float p = __builtin_fmaf(z, 1.0f / 11.0f, 1.0f / 9.0f);
    p = __builtin_fmaf(z, p, 1.0f / 7.0f);
    p = __builtin_fmaf(z, p, 1.0f / 5.0f);
    p = __builtin_fmaf(z, p, 1.0f / 3.0f);
    const float lnm = __builtin_fmaf(2.0f * s, z * p, 2.0f * s);
    return __builtin_fmaf((float)e, 0.693147182f, lnm);
}
RT_DEV float synth_cos2pi(float v) {
#pragma clang fp contract(off)
    const float n = rintf(4.0f * v);
    const float r = v - 0.25f * n;
    const float t = r * 6.28318548f;
    const float z = t * t;
    float c = __builtin_fmaf(z, -2.75573192e-7f, 2.48015873e-5f);
    c = __builtin_fmaf(z, c, -1.38888889e-3f);
    c = __builtin_fmaf(z, c, 4.16666667e-2f);
    c = __builtin_fmaf(z, c, -0.5f);
    c = __builtin_fmaf(z, c, 1.0f);
    float sn = __builtin_fmaf(z, -2.50521084e-8f, 2.75573192e-6f);
    sn = __builtin_fmaf(z, sn, -1.98412698e-4f);
    sn = __builtin_fmaf(z, sn, 8.33333333e-3f);
    sn = __builtin_fmaf(z, sn, -1.66666667e-1f);
    sn = __builtin_fmaf(t * z, sn, t);
    const int q = ((int)n) & 3;
    return q == 0 ? c : q == 1 ? -sn : q == 2 ? -c : sn;
}
RT_DEV float synth_normal(uint64_t seed, uint64_t idx) {
#pragma clang fp contract(off)
    const uint64_t h = splitmix64(seed ^ splitmix64(idx));
    const float u1 = (float)((h >> 40) + 1) * 5.9604644775390625e-8f;  // (0, 1]
    const float u2 = (float)(h & 0xFFFFFFull) * 5.9604644775390625e-8f;  // [0, 1)
    return sqrtf(-2.0f * synth_ln(u1)) * synth_cos2pi(u2);  // sqrtf: correctly rounded
}

extern "C" __global__ void __launch_bounds__(256)
k_synth_normal_f32(float* out, uint64_t n, uint64_t seed, float mean, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t i = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * wg_threads())
        out[i] = mean + stdv * synth_normal(seed, i);
}
extern "C" __global__ void __launch_bounds__(256)
k_synth_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, float mean, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t i = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * wg_threads())
        out[i] = f2h(mean + stdv * synth_normal(seed, i));
}

// Q8_0: d = max|w|/127 stored as f16; q = clamp(round(w/d), −127, 127) with
// the unrounded d (round half away from zero).
extern "C" __global__ void __launch_bounds__(256)
k_synth_q8_0(uint8_t* out, uint64_t nblk, uint64_t seed, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t b = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * wg_threads()) {
        float w[32];
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            w[i] = stdv * synth_normal(seed, b * 32 + i);
            amax = fmaxf(amax, fabsf(w[i]));
        }
        const float d = amax / 127.0f;
        uint8_t* p = out + b * 34;
        const uint16_t dh = f2h(d);
        p[0] = dh & 255; p[1] = dh >> 8;
        for (int i = 0; i < 32; ++i) {
            int q = d > 0.0f ? (int)roundf(w[i] / d) : 0;
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            p[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

// Q4_0: d = m/−8 where m is the signed value of largest magnitude;
// nib = clamp(int(w/d + 8.5), 0, 15); reference nibble order (2i low, 2i+1 high).
extern "C" __global__ void __launch_bounds__(256)
k_synth_q4_0(uint8_t* out, uint64_t nblk, uint64_t seed, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t b = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * wg_threads()) {
        float w[32];
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i) {
            w[i] = stdv * synth_normal(seed, b * 32 + i);
            if (fabsf(w[i]) > amax) { amax = fabsf(w[i]); mx = w[i]; }
        }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t* p = out + b * 18;
        const uint16_t dh = f2h(d);
        p[0] = dh & 255; p[1] = dh >> 8;
        for (int i = 0; i < 16; ++i) {
            int n0 = (int)(w[2 * i] * id + 8.5f), n1 = (int)(w[2 * i + 1] * id + 8.5f);
            n0 = n0 < 0 ? 0 : (n0 > 15 ? 15 : n0);
            n1 = n1 < 0 ? 0 : (n1 > 15 ? 15 : n1);
            p[2 + i] = (uint8_t)(n0 | (n1 << 4));
        }
    }
}

// Q4_K: scale index s ∈ 0..7 covers elements 64(s%4) + 32(s/4) + [0,32) —
// the reference's (j, j+4) pairing.  Per s: min_s = max(0, −min w),
// scale_s = (max w + min_s)/15; d = max scale/63, dmin = max min/63 (f16);
// sc_s = round(scale_s/d), m_s = round(min_s/dmin) (6-bit);
// q = clamp(round((w + dmin·m_s)/(d·sc_s)), 0, 15).
extern "C" __global__ void __launch_bounds__(256)
k_synth_q4k(uint8_t* out, uint64_t nblk, uint64_t seed, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t b = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * wg_threads()) {
        float w[256];
        for (int i = 0; i < 256; ++i) w[i] = stdv * synth_normal(seed, b * 256 + i);
        float scl[8], mns[8], maxs = 0.0f, maxm = 0.0f;
        for (int s = 0; s < 8; ++s) {
            const int base = 64 * (s & 3) + 32 * (s >> 2);
            float mn = 0.0f, mx = -3.0e38f;
            for (int l = 0; l < 32; ++l) { mn = fminf(mn, w[base + l]); mx = fmaxf(mx, w[base + l]); }
            mns[s] = -mn;
            scl[s] = (mx - mn) / 15.0f;
            maxs = fmaxf(maxs, scl[s]);
            maxm = fmaxf(maxm, mns[s]);
        }
        const float d = maxs / 63.0f, dmin = maxm / 63.0f;
        const uint16_t dh = f2h(d), dmh = f2h(dmin);
        const float dq = h2f(dh), dmq = h2f(dmh);
        uint32_t sc[8], m[8];
        for (int s = 0; s < 8; ++s) {
            int a = d > 0.0f ? (int)roundf(scl[s] / d) : 0;
            int c = dmin > 0.0f ? (int)roundf(mns[s] / dmin) : 0;
            sc[s] = a < 0 ? 0 : (a > 63 ? 63 : a);
            m[s] = c < 0 ? 0 : (c > 63 ? 63 : c);
        }
        uint8_t* p = out + b * 144;
        p[0] = dh & 255; p[1] = dh >> 8; p[2] = dmh & 255; p[3] = dmh >> 8;
        uint8_t* S = p + 4;
        for (int j = 0; j < 4; ++j) {
            S[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            S[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            S[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t* qs = p + 16;
        for (int j = 0; j < 4; ++j) {
            for (int l = 0; l < 32; ++l) {
                uint32_t qq[2];
                for (int hi = 0; hi < 2; ++hi) {
                    const int s = j + 4 * hi;
                    const float ds = dq * (float)sc[s], ms = dmq * (float)m[s];
                    int q = ds > 0.0f ? (int)roundf((w[64 * j + 32 * hi + l] + ms) / ds) : 0;
                    qq[hi] = q < 0 ? 0 : (q > 15 ? 15 : q);
                }
                qs[32 * j + l] = (uint8_t)(qq[0] | (qq[1] << 4));
            }
        }
    }
}

// Q5_0: d = m/−16 (m: signed value of largest magnitude), q = clamp(int(w/d
// + 16.5), 0, 31); element j < 16 in the low nibble of qs[j] and qh bit j,
// element 16 + j in the high nibble and qh bit 16 + j.
extern "C" __global__ void __launch_bounds__(256)
k_synth_q5_0(uint8_t* out, uint64_t nblk, uint64_t seed, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t b = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * wg_threads()) {
        float w[32];
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i) {
            w[i] = stdv * synth_normal(seed, b * 32 + i);
            if (fabsf(w[i]) > amax) { amax = fabsf(w[i]); mx = w[i]; }
        }
        const float d = mx / -16.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t* p = out + b * 22;
        const uint16_t dh = f2h(d);
        p[0] = dh & 255; p[1] = dh >> 8;
        uint32_t qh = 0;
        for (int j = 0; j < 16; ++j) {
            int q0 = (int)(w[j] * id + 16.5f), q1 = (int)(w[j + 16] * id + 16.5f);
            q0 = q0 < 0 ? 0 : (q0 > 31 ? 31 : q0);
            q1 = q1 < 0 ? 0 : (q1 > 31 ? 31 : q1);
            p[6 + j] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
            qh |= (uint32_t)(q0 >> 4) << j;
            qh |= (uint32_t)(q1 >> 4) << (j + 16);
        }
        for (int i = 0; i < 4; ++i) p[2 + i] = (uint8_t)(qh >> (8 * i));
    }
}

// Q5_K: the Q4_K construction with 31 levels; the high bit of element e goes
// to bit e%8 of qh[e/8].
extern "C" __global__ void __launch_bounds__(256)
k_synth_q5k(uint8_t* out, uint64_t nblk, uint64_t seed, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t b = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * wg_threads()) {
        float w[256];
        for (int i = 0; i < 256; ++i) w[i] = stdv * synth_normal(seed, b * 256 + i);
        float scl[8], mns[8], maxs = 0.0f, maxm = 0.0f;
        for (int s = 0; s < 8; ++s) {
            const int base = 64 * (s & 3) + 32 * (s >> 2);
            float mn = 0.0f, mx = -3.0e38f;
            for (int l = 0; l < 32; ++l) { mn = fminf(mn, w[base + l]); mx = fmaxf(mx, w[base + l]); }
            mns[s] = -mn;
            scl[s] = (mx - mn) / 31.0f;
            maxs = fmaxf(maxs, scl[s]);
            maxm = fmaxf(maxm, mns[s]);
        }
        const float d = maxs / 63.0f, dmin = maxm / 63.0f;
        const uint16_t dh = f2h(d), dmh = f2h(dmin);
        const float dq = h2f(dh), dmq = h2f(dmh);
        uint32_t sc[8], m[8];
        for (int s = 0; s < 8; ++s) {
            int a = d > 0.0f ? (int)roundf(scl[s] / d) : 0;
            int c = dmin > 0.0f ? (int)roundf(mns[s] / dmin) : 0;
            sc[s] = a < 0 ? 0 : (a > 63 ? 63 : a);
            m[s] = c < 0 ? 0 : (c > 63 ? 63 : c);
        }
        uint8_t* p = out + b * 176;
        p[0] = dh & 255; p[1] = dh >> 8; p[2] = dmh & 255; p[3] = dmh >> 8;
        uint8_t* S = p + 4;
        for (int j = 0; j < 4; ++j) {
            S[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            S[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            S[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t qh[32];
        for (int i = 0; i < 32; ++i) qh[i] = 0;
        uint8_t* qs = p + 48;
        for (int j = 0; j < 4; ++j) {
            for (int l = 0; l < 32; ++l) {
                uint32_t qq[2];
                for (int hi = 0; hi < 2; ++hi) {
                    const int s = j + 4 * hi, e = 64 * j + 32 * hi + l;
                    const float ds = dq * (float)sc[s], ms = dmq * (float)m[s];
                    int q = ds > 0.0f ? (int)roundf((w[e] + ms) / ds) : 0;
                    qq[hi] = q < 0 ? 0 : (q > 31 ? 31 : q);
                    qh[e / 8] |= (uint8_t)((qq[hi] >> 4) << (e % 8));
                }
                qs[32 * j + l] = (uint8_t)((qq[0] & 15) | ((qq[1] & 15) << 4));
            }
        }
        for (int i = 0; i < 32; ++i) p[16 + i] = qh[i];
    }
}

// Q6_K: group g = 4·(h/128) + t covers elements h + 32t + [0,32) and uses
// scale slot h/16 + 2t (the only slots the reference decoder reads).
// scale_g = m_g/−32 (m_g: signed value of largest magnitude), d = max|scale|/127,
// sc_g = round(scale_g/d), q = clamp(round(w/(d·sc_g)) + 32, 0, 63).
// The odd scale slots, which the reference ignores, hold 0x5A.
extern "C" __global__ void __launch_bounds__(256)
k_synth_q6k(uint8_t* out, uint64_t nblk, uint64_t seed, float stdv) {
#pragma clang fp contract(off)
    for (uint64_t b = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * wg_threads()) {
        float w[256];
        for (int i = 0; i < 256; ++i) w[i] = stdv * synth_normal(seed, b * 256 + i);
        float scl[8], dmax = 0.0f;
        for (int g = 0; g < 8; ++g) {
            const int base = 128 * (g >> 2) + 32 * (g & 3);
            float amax = 0.0f, mx = 0.0f;
            for (int l = 0; l < 32; ++l)
                if (fabsf(w[base + l]) > amax) { amax = fabsf(w[base + l]); mx = w[base + l]; }
            scl[g] = mx / -32.0f;
            dmax = fmaxf(dmax, fabsf(scl[g]));
        }
        const float d = dmax / 127.0f;
        const uint16_t dh = f2h(d);
        const float dq = h2f(dh);
        int sc[8];
        for (int g = 0; g < 8; ++g) {
            int a = d > 0.0f ? (int)roundf(scl[g] / d) : 0;
            sc[g] = a < -127 ? -127 : (a > 127 ? 127 : a);
        }
        int q[256];
        for (int g = 0; g < 8; ++g) {
            const int base = 128 * (g >> 2) + 32 * (g & 3);
            const float ds = dq * (float)sc[g];
            for (int l = 0; l < 32; ++l) {
                int v = ds != 0.0f ? (int)roundf(w[base + l] / ds) + 32 : 32;
                q[base + l] = v < 0 ? 0 : (v > 63 ? 63 : v);
            }
        }
        uint8_t* p = out + b * 210;
        uint8_t* ql = p;
        uint8_t* qh = p + 128;
        int8_t* S = (int8_t*)(p + 192);
        for (int h = 0; h < 256; h += 128) {
            for (int l = 0; l < 32; ++l) {
                const int q1 = q[h + l], q2 = q[h + l + 32], q3 = q[h + l + 64], q4 = q[h + l + 96];
                ql[h / 2 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
                ql[h / 2 + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
                qh[h / 4 + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        }
        for (int g = 0; g < 8; ++g) {
            const int slot = 8 * (g >> 2) + 2 * (g & 3);
            S[slot] = (int8_t)sc[g];
            S[slot + 1] = (int8_t)0x5A;
        }
        p[208] = dh & 255; p[209] = dh >> 8;
    }
}

// ───────────────────────────── calibration ─────────────────────────────
// Plain HBM streams of known size: the achievable-bandwidth reference for the
// GEMV kernels and the scale for rocprof's FETCH_SIZE / WRITE_SIZE counters.

// Reads n16 16-byte vectors (grid-stride, 4 in flight per thread) and writes
// one xor-folded dword per workgroup so the loads cannot be elided.
extern "C" __global__ void __launch_bounds__(256)
k_stream_read(const u32x4* __restrict__ src, uint64_t n16, uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    const uint64_t stride = (uint64_t)gridDim.x * wg_threads();
    uint64_t i = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u32x4 a = __builtin_nontemporal_load(src + i);
        u32x4 b = __builtin_nontemporal_load(src + i + stride);
        u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
        u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^
               d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        u32x4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o, 64);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (wg_threads() / 64) + (threadIdx.x >> 6)] = acc;
}

extern "C" __global__ void __launch_bounds__(256)
k_stream_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst, uint64_t n16) {
    const uint64_t stride = (uint64_t)gridDim.x * wg_threads();
    for (uint64_t i = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}
