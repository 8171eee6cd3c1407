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

// ───────────────────── batched verify / prefill glue ─────────────────────
// The M-row kernels between the GEMMs of verify_draft (forward.rs:2186-2271),
// on f32 activations [rows][dim].

// add_bias_broadcast_f16 (activation.metal:211-227, called at forward.rs:2199-2207):
// x[s][i] += f32(bias[i]).
extern "C" __global__ void __launch_bounds__(256)
k_add_bias_broadcast_f32(float* __restrict__ x, const uint16_t* __restrict__ bias, uint32_t seq,
                         uint32_t dim) {
    const uint64_t n = (uint64_t)seq * dim;
    for (uint64_t t = blockIdx.x * (uint64_t)wg_threads() + threadIdx.x; t < n;
         t += (uint64_t)gridDim.x * wg_threads())
        x[t] += h2f(bias[t % dim]);
}

// rope_batch_inplace_f16 (rope.metal:92-121): row s of [seq][heads][hd] at
// position start_pos + s, pairs (d, d + hd/2), angle = pos / θ^(2d/hd) (a
// division, where the single-token fused_rope multiplies by the inverse).
// Grid (⌈hd/2 / 64⌉, heads, seq).
extern "C" __global__ void __launch_bounds__(64)
k_rope_batch_f32(float* x, uint32_t head_dim, uint32_t heads, uint32_t start_pos, float theta) {
    const uint32_t half = head_dim / 2;
    const uint32_t d = blockIdx.x * wg_threads() + threadIdx.x;
    if (d >= half) return;
    const float angle = (float)(start_pos + blockIdx.z) / powf(theta, (float)(2 * d) / (float)head_dim);
    float c, s;
    sincosf(angle, &s, &c);
    float* v = x + ((size_t)blockIdx.z * heads + blockIdx.y) * head_dim;
    const float r = v[d], i = v[d + half];
    v[d] = r * c - i * s;
    v[d + half] = i * c + r * s;
}

// rope_batch_inplace_f16 of q and k (rope.metal:92-121) and KvCache::write_at
// of the rotated k and of v (forward.rs:2209-2231) in one launch: grid
// (⌈hd/2 / 64⌉, max(heads, kv_heads), seq); q rotated in place, k and v
// written to cache[h][start_pos + s].
extern "C" __global__ void __launch_bounds__(64)
k_rope_kv_write_batch_f32(float* q, const float* k, const float* v, float* kc, float* vc,
                          uint32_t head_dim, uint32_t heads, uint32_t kv_heads, uint32_t start_pos,
                          float theta, uint32_t max_seq) {
    const uint32_t half = head_dim / 2;
    const uint32_t d = blockIdx.x * wg_threads() + threadIdx.x;
    if (d >= half) return;
    const uint32_t h = blockIdx.y, s = blockIdx.z, pos = start_pos + s;
    const float angle = (float)pos / powf(theta, (float)(2 * d) / (float)head_dim);
    float c, sn;
    sincosf(angle, &sn, &c);
    if (h < heads) {
        float* x = q + ((size_t)s * heads + h) * head_dim;
        const float r = x[d], i = x[d + half];
        x[d] = r * c - i * sn;
        x[d + half] = i * c + r * sn;
    }
    if (h < kv_heads) {
        const size_t src = ((size_t)s * kv_heads + h) * head_dim;
        const size_t dst = ((size_t)h * max_seq + pos) * head_dim;
        const float r = k[src + d], i = k[src + d + half];
        kc[dst + d] = r * c - i * sn;
        kc[dst + d + half] = i * c + r * sn;
        vc[dst + d] = v[src + d];
        vc[dst + d + half] = v[src + d + half];
    }
}

// KvCache::write_at (kv_cache.rs:132-150) for rows start_pos .. start_pos+seq-1
// (the loop of forward.rs:2216-2231):
// k / v [seq][kv_heads][hd] → cache[h][start_pos + s][d], both caches in one launch.
extern "C" __global__ void __launch_bounds__(256)
k_kv_write_batch_f32(const float* __restrict__ k, const float* __restrict__ v, float* kc,
                     float* vc, uint32_t start_pos, uint32_t max_seq, uint32_t head_dim,
                     uint32_t kv_heads, uint32_t n) {
    const uint32_t t = blockIdx.x * wg_threads() + threadIdx.x;
    if (t >= n) return;
    const uint32_t row = kv_heads * head_dim;
    const uint32_t s = t / row, h = (t % row) / head_dim, d = t % head_dim;
    const size_t o = ((size_t)h * max_seq + start_pos + s) * head_dim + d;
    kc[o] = k[t];
    vc[o] = v[t];
}

// add_f16 (activation.metal:175-185, forward.rs:2247) on f32: out = a + b
// (out may alias a or b).
extern "C" __global__ void __launch_bounds__(256)
k_add_f32(const float* a, const float* b, float* out, uint32_t n) {
    for (uint32_t i = blockIdx.x * wg_threads() + threadIdx.x; i < n; i += gridDim.x * wg_threads())
        out[i] = a[i] + b[i];
}

// silu_mul_f32 (activation.metal:156-173; f16 form at forward.rs:2256):
// out = silu(gate) · up, silu(g) = g / (1 + e^−g).
extern "C" __global__ void __launch_bounds__(256)
k_silu_mul_f32(const float* gate, const float* up, float* out, uint32_t n) {
    for (uint32_t i = blockIdx.x * wg_threads() + threadIdx.x; i < n; i += gridDim.x * wg_threads()) {
        const float g = gate[i];
        out[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

// The per-row argmax of verify_draft (forward.rs:2283-2293): the FIRST index
// whose value is strictly greater than every earlier one, starting from −∞
// (NaN never wins; a row of −∞ / NaN gives 0).  Grid (G, rows): workgroup g
// scans range g of row y and leaves (value, index) in `states`; the last
// workgroup of the row to arrive (counter, reset by it) merges the G ranges
// in order.
extern "C" __global__ void __launch_bounds__(256)
k_argmax_rows_first_f32(const float* __restrict__ in, uint32_t* __restrict__ out, uint32_t n,
                        float2* __restrict__ states, uint32_t* __restrict__ counters) {
    __shared__ float bv_s[4];
    __shared__ uint32_t bi_s[4];
    __shared__ bool last;
    const uint32_t G = gridDim.x, g = blockIdx.x, row = blockIdx.y;
    const uint32_t per = (n + G - 1) / G, b0 = g * per, b1 = min(n, b0 + per);
    const float* r = in + (size_t)row * n;
    float bv = -__builtin_huge_valf();
    uint32_t bi = 0xFFFFFFFFu;  // none yet
    for (uint32_t i = b0 + threadIdx.x; i < b1; i += wg_threads()) {
        const float v = r[i];
        if (v > bv) { bv = v; bi = i; }
    }
    // larger value wins; equal values: the smaller index (none = UINT_MAX)
    auto better = [](float v, uint32_t i, float w, uint32_t j) { return w > v || (w == v && j < i); };
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(bv, o, 64);
        const uint32_t j = __shfl_xor(bi, o, 64);
        if (better(bv, bi, w, j)) { bv = w; bi = j; }
    }
    const uint32_t wv = threadIdx.x >> 6, nw = wg_threads() >> 6;
    if ((threadIdx.x & 63) == 0) { bv_s[wv] = bv; bi_s[wv] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t k = 1; k < nw; ++k)
            if (better(bv, bi, bv_s[k], bi_s[k])) { bv = bv_s[k]; bi = bi_s[k]; }
        dev_store(&states[(size_t)row * G + g].x, bv);
        dev_store(&states[(size_t)row * G + g].y, __uint_as_float(bi));
        dev_stores_done();
        last = arrive(&counters[row]) == G - 1;
        if (last) {
            // ranges in order: a later range wins only with a strictly greater value
            float best = -__builtin_huge_valf();
            uint32_t bidx = 0xFFFFFFFFu;
            for (uint32_t k = 0; k < G; ++k) {
                const float v = dev_load(&states[(size_t)row * G + k].x);
                const uint32_t j = __float_as_uint(dev_load(&states[(size_t)row * G + k].y));
                if (j != 0xFFFFFFFFu && v > best) { best = v; bidx = j; }
            }
            out[row] = bidx == 0xFFFFFFFFu ? 0u : bidx;
            dev_store(&counters[row], 0u);  // ready for the next call (also under graph replay)
        }
    }
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
// wave form of the RoPE attention (attn_split_w): one query head per
// workgroup, parts-only or single-split launches
#define RT_ATTN_W_KERNEL(HD)                                                                \
    extern "C" __global__ void __launch_bounds__(256) k_attn_rope_w_f32_hd##HD(AttnArgs a) { \
        attn_split_w<HD>(a, blockIdx.x, gridDim.x, blockIdx.y, blockIdx.z);                  \
    }
RT_ATTN_W_KERNEL(64)
RT_ATTN_W_KERNEL(128)

// add_f16_into_f32 (dispatch.rs:316-330): acc[i] += f32(src[i]), the bias add
// of the reference's separate-dispatch Q/K/V fallback (forward.rs:1561-1568).
extern "C" __global__ void __launch_bounds__(256)
k_add_f16_into_f32(const uint16_t* __restrict__ src, float* __restrict__ acc, uint32_t n) {
    for (uint32_t i = threadIdx.x + blockIdx.x * wg_threads(); i < n; i += wg_threads() * gridDim.x)
        acc[i] += h2f(src[i]);
}

// Σ y² over rows 4i..4i+3 of y (m rows), one thread per row quad: the
// partial sums a norm-fused launch reads instead of reducing y itself, for
// a producing launch whose body does not write them.
extern "C" __global__ void __launch_bounds__(256)
k_ssq_quads(const float* __restrict__ y, uint32_t m, float* __restrict__ out) {
    const uint32_t qd = blockIdx.x * 256 + threadIdx.x;
    if (qd * 4 >= m) return;
    float s = 0.0f;
    for (uint32_t r = 0; r < 4; ++r) {
        const uint32_t i = qd * 4 + r;
        const float v = i < m ? y[i] : 0.0f;
        s += v * v;
    }
    out[qd] = s;
}

// Causal multi-query attention on the matrix cores (f32 MFMA 16x16x4): one
// workgroup takes 16 query columns — consecutive (row, head) pairs of one KV
// head's query-head group, flattened row-major — and one of nsp ranges of
// a.chunk key tiles (16 positions each) of the positions the columns see;
// its W waves split the range's tiles (wave w: tiles w, w + W, ...).  Per
// tile a wave computes Sᵀ = K·Qᵀ (16 positions × 16 columns), the online
// softmax per column, and Oᵀ += Vᵀ·Pᵀ, the next tile's K and V already in
// flight; the waves' partial (O, max, sum) meet in LDS.  With one range the
// workgroup writes the normalised rows; with several it writes its partial
// and the last of the column group's workgroups to arrive merges them in
// range order.  The sums over d and over positions are taken in orders of
// the layout's choosing:
//   Sᵀ k-step s, lane group g (lane / 16) supplies d = (HD/4)·g + s, so a lane
//   reads one contiguous quarter row of K and of its query (four
//   accumulators, one per s mod 4, summed at the end);
//   Oᵀ k-step i, lane group g supplies position 4g + i of the tile (the
//   lane's own i-th score), block b, lane row n supplies d = (HD/16)·n + b.
// Positions past a column's causal limit score -inf; rows past the last
// position any column sees are never read (indices clamp to it).
template <int HD>
RT_DEV void attn_mq(const AttnArgs& a) {
    constexpr uint32_t QC = HD / 4, NB = HD / 16;
    extern __shared__ f32x4 mq_lds[];
    __shared__ uint32_t last_flag;
    float* lds = (float*)mq_lds;
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6, W = wg_threads() >> 6;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t G = a.H / a.KVH, kvh = blockIdx.y, bt = blockIdx.z;
    const uint32_t R = a.q_len * G, cgs = (R + 15) / 16, nsp = gridDim.x / cgs;
    const uint32_t cg = blockIdx.x / nsp, sp = blockIdx.x % nsp, c0 = cg * 16;
    const uint32_t qi = c0 + n;
    const bool valid = qi < R;
    const uint32_t r = valid ? qi / G : 0, h = kvh * G + (valid ? qi % G : 0);
    const uint32_t lim = valid ? min(a.kv_len, a.q_start + r + 1) : 0;
    const uint32_t Lmax = min(a.kv_len, a.q_start + (min(R, c0 + 16) - 1) / G + 1);
    const size_t qrow = (size_t)(bt * a.q_len + r) * a.H + h;
    float qv[QC];
    {
        const f32x4* q4 = (const f32x4*)(a.q + qrow * HD + QC * g);
#pragma unroll
        for (uint32_t j = 0; j < QC / 4; ++j) {
            const f32x4 t = q4[j];
            qv[4 * j] = t.x; qv[4 * j + 1] = t.y; qv[4 * j + 2] = t.z; qv[4 * j + 3] = t.w;
        }
    }
    const size_t cb = ((size_t)bt * a.KVH + kvh) * a.stride * HD;
    const float* kb = a.kc + cb;
    const float* vb = a.vc + cb;
    f32x4 acc[NB];
#pragma unroll
    for (uint32_t j = 0; j < NB; ++j) acc[j] = f32x4{0, 0, 0, 0};
    const float NEG = -__builtin_huge_valf();
    float m = NEG, l = 0.0f;
    const uint32_t T = min((Lmax + 15) / 16, (sp + 1) * a.chunk);
    f32x4 kk[QC / 4], vv[4][NB / 4];
    auto load = [&](uint32_t t, f32x4 (&kd)[QC / 4], f32x4 (&vd)[4][NB / 4]) {
        const uint32_t p0 = t * 16;
        const f32x4* kr = (const f32x4*)(kb + (size_t)min(p0 + n, Lmax - 1) * HD + QC * g);
#pragma unroll
        for (uint32_t j = 0; j < QC / 4; ++j) kd[j] = kr[j];
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const f32x4* vr = (const f32x4*)(vb + (size_t)min(p0 + 4 * g + i, Lmax - 1) * HD + NB * n);
#pragma unroll
            for (uint32_t j = 0; j < NB / 4; ++j) vd[i][j] = vr[j];
        }
    };
    auto tile = [&](uint32_t t, const f32x4 (&kd)[QC / 4], const f32x4 (&vd)[4][NB / 4]) {
        const uint32_t p0 = t * 16;
        f32x4 s4[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (uint32_t j = 0; j < QC / 4; ++j) {
            s4[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(kd[j].x, qv[4 * j], s4[0], 0, 0, 0);
            s4[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kd[j].y, qv[4 * j + 1], s4[1], 0, 0, 0);
            s4[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(kd[j].z, qv[4 * j + 2], s4[2], 0, 0, 0);
            s4[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(kd[j].w, qv[4 * j + 3], s4[3], 0, 0, 0);
        }
        const f32x4 s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        float sv[4], tmax = NEG;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            sv[i] = p0 + 4 * g + i < lim ? s[i] * a.scale : NEG;
            tmax = fmaxf(tmax, sv[i]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m, tmax);
        const float alpha = m == NEG ? 0.0f : expf(m - m_new);
        float p[4], ps = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            p[i] = sv[i] == NEG ? 0.0f : expf(sv[i] - m_new);
            ps += p[i];
        }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l = l * alpha + ps;
        m = m_new;
#pragma unroll
        for (uint32_t j = 0; j < NB; ++j) acc[j] *= alpha;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i)
#pragma unroll
            for (uint32_t j = 0; j < NB / 4; ++j) {
                acc[4 * j] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[i][j].x, p[i], acc[4 * j], 0, 0, 0);
                acc[4 * j + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[i][j].y, p[i], acc[4 * j + 1], 0, 0, 0);
                acc[4 * j + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[i][j].z, p[i], acc[4 * j + 2], 0, 0, 0);
                acc[4 * j + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vd[i][j].w, p[i], acc[4 * j + 3], 0, 0, 0);
            }
    };
    // two register sets in turn: the next tile's loads (unconditional, the
    // last tile again at the end) issue ahead of this tile's matrix work.
    // Head size 256 has the registers for one set only.
    uint32_t t = sp * a.chunk + w;
    if constexpr (HD > 128) {
        for (; t < T; t += W) {
            load(t, kk, vv);
            tile(t, kk, vv);
        }
    }
    f32x4 k2[QC / 4], v2[4][NB / 4];
    if (t < T) load(t, kk, vv);
    for (; t < T; t += 2 * W) {
        load(min(t + W, T - 1), k2, v2);
        __builtin_amdgcn_sched_barrier(0);
        tile(t, kk, vv);
        if (t + W >= T) break;
        load(min(t + 2 * W, T - 1), kk, vv);
        __builtin_amdgcn_sched_barrier(0);
        tile(t + W, k2, v2);
    }
    // the wave's partial: O[column][d] unnormalised, then max and sum per column
    constexpr uint32_t WS = 16 * HD + 32;
    float* wo = lds + w * WS;
#pragma unroll
    for (uint32_t rr = 0; rr < 4; ++rr)
#pragma unroll
        for (uint32_t j = 0; j < NB / 4; ++j)
            *(f32x4*)(wo + n * HD + NB * (4 * g + rr) + 4 * j) =
                f32x4{acc[4 * j][rr], acc[4 * j + 1][rr], acc[4 * j + 2][rr], acc[4 * j + 3][rr]};
    if (g == 0) {
        wo[16 * HD + n] = m;
        wo[16 * HD + 16 + n] = l;
    }
    __syncthreads();
    // partials of a multi-range column group: [pair][range][16][HD] and
    // [pair][range][16][max, sum], pair = (batch · KVH + kvh) · cgs + cg
    const size_t pair = ((size_t)bt * a.KVH + kvh) * cgs + cg;
    for (uint32_t e = threadIdx.x; e < 16 * (HD / 4); e += wg_threads()) {
        const uint32_t col = e / (HD / 4), d4 = e % (HD / 4);
        const uint32_t qc = c0 + col;
        if (qc >= R) continue;
        float M = NEG;
        for (uint32_t v = 0; v < W; ++v) M = fmaxf(M, lds[v * WS + 16 * HD + col]);
        f32x4 o = {0, 0, 0, 0};
        float den = 0.0f;
        for (uint32_t v = 0; v < W; ++v) {
            const float mv = lds[v * WS + 16 * HD + col];
            const float f = mv == NEG ? 0.0f : expf(mv - M);
            den += f * lds[v * WS + 16 * HD + 16 + col];
            o += f * *(const f32x4*)(lds + v * WS + col * HD + 4 * d4);
        }
        if (nsp == 1) {
            const uint32_t orow = qc / G, oh = kvh * G + qc % G;
            *(f32x4*)(a.out + ((size_t)(bt * a.q_len + orow) * a.H + oh) * HD + 4 * d4) = o / den;
        } else {
            float* pp = a.part + ((pair * nsp + sp) * 16 + col) * HD + 4 * d4;
            dev_store(pp + 0, o.x);
            dev_store(pp + 1, o.y);
            dev_store(pp + 2, o.z);
            dev_store(pp + 3, o.w);
            if (d4 == 0) {
                float* mlp = a.ml + ((pair * nsp + sp) * 16 + col) * 2;
                dev_store(mlp + 0, M);
                dev_store(mlp + 1, den);
            }
        }
    }
    // parts only: the consumer merges (k_gemm_xh_prep1a_mg*)
    if (nsp == 1 || a.parts_only) return;
    dev_stores_done();
    __syncthreads();
    uint32_t* counter = a.counters + pair;
    if (threadIdx.x == 0) last_flag = arrive(counter) == nsp - 1;
    __syncthreads();
    if (!last_flag) return;
    // o = Σ o_s·e^(m_s−M) / Σ l_s·e^(m_s−M) over the ranges, in range order;
    // every range's loads are issued before the first is used (indices past
    // nsp repeat the last range, weighted 0), so the merge waits once
    for (uint32_t e = threadIdx.x; e < 16 * (HD / 4); e += wg_threads()) {
        const uint32_t col = e / (HD / 4), d4 = e % (HD / 4);
        const uint32_t qc = c0 + col;
        if (qc >= R) continue;
        const float* mlv = a.ml + (pair * nsp * 16 + col) * 2;
        float mj[RT_ATTN_MQ_NSP_MAX], lj[RT_ATTN_MQ_NSP_MAX];
        f32x4 oj[RT_ATTN_MQ_NSP_MAX];
#pragma unroll
        for (uint32_t j = 0; j < RT_ATTN_MQ_NSP_MAX; ++j) {
            const uint32_t jj = min(j, nsp - 1);
            mj[j] = dev_load(mlv + 32 * jj);
            lj[j] = dev_load(mlv + 32 * jj + 1);
            const float* pj = a.part + ((pair * nsp + jj) * 16 + col) * HD + 4 * d4;
            oj[j] = f32x4{dev_load(pj), dev_load(pj + 1), dev_load(pj + 2), dev_load(pj + 3)};
        }
        float M = NEG;
#pragma unroll
        for (uint32_t j = 0; j < RT_ATTN_MQ_NSP_MAX; ++j) M = fmaxf(M, mj[j]);
        float L = 0.0f;
        f32x4 o = {0, 0, 0, 0};
#pragma unroll
        for (uint32_t j = 0; j < RT_ATTN_MQ_NSP_MAX; ++j) {
            const float f = (j >= nsp || mj[j] == NEG) ? 0.0f : expf(mj[j] - M);
            L += f * lj[j];
            o += f * oj[j];
        }
        const uint32_t orow = qc / G, oh = kvh * G + qc % G;
        *(f32x4*)(a.out + ((size_t)(bt * a.q_len + orow) * a.H + oh) * HD + 4 * d4) = o / L;
    }
    if (threadIdx.x == 0) dev_store(counter, 0u);  // ready for the next call (also under graph replay)
}
// at most 8 / 8 / 4 waves at head size 64 / 128 / 256 (the registers of two
// tiles' K and V, the query and the output slices)
#define RT_ATTN_MQ_KERNEL(HD)                                                                  \
    extern "C" __global__ void __launch_bounds__(64 * rt_attn_mq_wmax(HD))                    \
        k_attn_mq_f32_hd##HD(AttnArgs a) {                                                     \
        attn_mq<HD>(a);                                                                          \
    }
RT_ATTN_MQ_KERNEL(64)
RT_ATTN_MQ_KERNEL(128)
RT_ATTN_MQ_KERNEL(256)
