// k_decode.hip — the non-GEMV kernels of one decode step: RMSNorm, RoPE,
// KV-cache scatter, decode attention (plain and fused with RoPE + cache
// write) and the Q8_0 embedding lookup.
#include "rt_device.h"

// Sum over a workgroup (any multiple of 64 threads ≤ 1024); `red` holds ≥ 16
// floats of LDS.  Every thread receives the total.
RT_DEV float block_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const uint32_t w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();  // previous users of `red` are done
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (uint32_t i = 0; i < nw; ++i) t += red[i];
    return t;
}
RT_DEV float block_max(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const uint32_t w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = -__builtin_huge_valf();
    for (uint32_t i = 0; i < nw; ++i) t = fmaxf(t, red[i]);
    return t;
}

// rms_norm_f32_f32_f32g (norm.metal:126-154): one workgroup per row,
// y = x · rsqrt(mean(x²) + eps) · γ.  y may alias x.
extern "C" __global__ void __launch_bounds__(256)
k_rms_norm_f32g(const float* x, float* y, const float* gamma, float eps, uint32_t hidden) {
    __shared__ float red[16];
    const float* xr = x + (size_t)blockIdx.x * hidden;
    float* yr = y + (size_t)blockIdx.x * hidden;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < hidden; i += blockDim.x) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    const float rms = rsqrtf(ss / (float)hidden + eps);
    for (uint32_t i = threadIdx.x; i < hidden; i += blockDim.x) yr[i] = xr[i] * rms * gamma[i];
}

// RoPE angle for pair d (fused_rope.metal:34-38): freq = 1/θ^(2d/hd).
RT_DEV void rope_cs(uint32_t d, uint32_t head_dim, uint32_t pos, float theta, float& c, float& s) {
    const float freq = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
    const float angle = (float)pos * freq;
    sincosf(angle, &s, &c);
}

// fused_rope_qk_f32 (fused_rope.metal:17-56): non-interleaved pairs (d, d+hd/2).
extern "C" __global__ void __launch_bounds__(256)
k_rope_qk_f32(float* Q, float* K, uint32_t head_dim, uint32_t q_heads, uint32_t kv_heads,
              uint32_t pos, float theta) {
    const uint32_t half = head_dim / 2;
    const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
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
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const uint32_t h = t / head_dim, d = t % head_dim;
    dst[((size_t)h * max_seq + pos) * head_dim + d] = src[t];
}

// ───────────────────────────── attention ─────────────────────────────
// One workgroup (256 threads) per (query head, batch row); decode attention
// is latency-bound (a few hundred KB per layer), so each phase issues all of
// its loads at once:
//   scores : thread t takes positions t, t+256, ...; a key row is HD/4
//            float4 loads, issued together;
//   softmax: block max / block sum (chunks of ATT_CHUNK positions merged with
//            the usual running max / sum / output rescaling, any kv_len);
//   output : thread t owns float4 column (t % (HD/4)) for positions
//            ≡ t / (HD/4) (mod 256/(HD/4)), loads unrolled by 8; the partial
//            outputs are summed in LDS in a fixed order.
// Same math as the online softmax of attention.metal:248-308 up to f32
// rounding order.
constexpr uint32_t ATT_CHUNK = 4096;
constexpr uint32_t ATT_T = 256;

struct AttnIO {
    const float* q;       // this head's query (already rotated), hd floats
    const float* kc;      // cache base of the kv head: [pos][hd]
    const float* vc;
    const float* k_last;  // if non-null: the key/value of position kv_len-1
    const float* v_last;  //   come from these (not yet visible in the cache)
};

template <int HD>
RT_DEV void attend(const AttnIO& io, float* o, uint32_t kv_len, float scale, float* qs, float* sc,
                   float* red, f32x4* part) {
    constexpr int C4 = HD / 4;            // float4 columns of a row
    constexpr int G = ATT_T / C4;         // position groups in the output pass
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < HD; i += ATT_T) qs[i] = io.q[i];
    __syncthreads();
    f32x4 qv[C4];
#pragma unroll
    for (int c = 0; c < C4; ++c) qv[c] = ((const f32x4*)qs)[c];
    float m_run = -__builtin_huge_valf(), l_run = 0.0f;
    const uint32_t col = tid % C4, g = tid / C4;
    f32x4 o_run = {0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int PF = 16;  // value rows per thread fetched before the softmax
    auto vrow = [&](uint32_t p) -> const float* {
        return (io.v_last && p == kv_len - 1) ? io.v_last : io.vc + (size_t)p * HD;
    };
    for (uint32_t c0 = 0; c0 < kv_len; c0 += ATT_CHUNK) {
        const uint32_t cn = min(ATT_CHUNK, kv_len - c0);
        // value loads of this thread's first PF positions of the chunk go out
        // with the key loads (one memory round trip for both)
        f32x4 vpre[PF];
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const uint32_t j = g + u * G;
            vpre[u] = ((const f32x4*)vrow(c0 + (j < cn ? j : 0)))[col];
        }
        float mloc = -__builtin_huge_valf();
        for (uint32_t j = tid; j < cn; j += ATT_T) {
            const uint32_t p = c0 + j;
            const float* kr = (io.k_last && p == kv_len - 1) ? io.k_last : io.kc + (size_t)p * HD;
            f32x4 kv[C4];
#pragma unroll
            for (int c = 0; c < C4; ++c) kv[c] = ((const f32x4*)kr)[c];
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < C4; ++c)
                dot += qv[c].x * kv[c].x + qv[c].y * kv[c].y + qv[c].z * kv[c].z + qv[c].w * kv[c].w;
            const float s = dot * scale;
            sc[j] = s;
            mloc = fmaxf(mloc, s);
        }
        const float m_new = fmaxf(m_run, block_max(mloc, red));
        float lloc = 0.0f;
        for (uint32_t j = tid; j < cn; j += ATT_T) {
            const float pexp = expf(sc[j] - m_new);
            sc[j] = pexp;
            lloc += pexp;
        }
        const float lsum = block_sum(lloc, red);  // also orders sc[] writes before reads
        const float resc = (m_run == -__builtin_huge_valf()) ? 0.0f : expf(m_run - m_new);
        l_run = l_run * resc + lsum;
        o_run = o_run * resc;
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const uint32_t j = g + u * G;
            if (j < cn) o_run += sc[j] * vpre[u];
        }
        for (uint32_t j0 = g + PF * G; j0 < cn; j0 += PF * G) {
            f32x4 vv[PF];
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                const uint32_t j = j0 + u * G;
                vv[u] = ((const f32x4*)vrow(c0 + (j < cn ? j : j0)))[col];
            }
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                const uint32_t j = j0 + u * G;
                if (j < cn) o_run += sc[j] * vv[u];
            }
        }
        m_run = m_new;
        __syncthreads();  // sc[] reused by the next chunk
    }
    part[g * C4 + col] = o_run;
    __syncthreads();
    const float inv_l = (l_run > 0.0f) ? (1.0f / l_run) : 0.0f;
    if (tid < C4) {
        f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int gg = 0; gg < G; ++gg) t += part[gg * C4 + tid];
        ((f32x4*)o)[tid] = t * inv_l;
    }
}

template <int HD>
RT_DEV void attention_head(const float* Q, const float* K, const float* V, float* O,
                           uint32_t kv_len, uint32_t num_heads, uint32_t num_kv_heads, float scale,
                           uint32_t kv_head_stride) {
    __shared__ float qs[HD], sc[ATT_CHUNK], red[16];
    __shared__ f32x4 part[ATT_T];
    const uint32_t h = blockIdx.x, b = blockIdx.y;
    const uint32_t kvh = h / (num_heads / num_kv_heads);
    const size_t kv_base = ((size_t)b * num_kv_heads + kvh) * kv_head_stride * HD;
    AttnIO io{Q + ((size_t)b * num_heads + h) * HD, K + kv_base, V + kv_base, nullptr, nullptr};
    attend<HD>(io, O + ((size_t)b * num_heads + h) * HD, kv_len, scale, qs, sc, red, part);
}

// decode_attention_f32 (attention.metal:248-308; dispatch.rs:1575-1612).
// K/V cache: [batch][num_kv_heads][kv_head_stride][head_dim].  Instantiated
// for head_dim 64, 128 and 256 (the host checks).
#define RT_ATTN_KERNEL(HD)                                                                        \
    extern "C" __global__ void __launch_bounds__(256) k_decode_attention_f32_hd##HD(               \
        const float* Q, const float* K, const float* V, float* O, uint32_t kv_len,                 \
        uint32_t num_heads, uint32_t num_kv_heads, float scale, uint32_t kv_head_stride) {         \
        attention_head<HD>(Q, K, V, O, kv_len, num_heads, num_kv_heads, scale, kv_head_stride);    \
    }
RT_ATTN_KERNEL(64)
RT_ATTN_KERNEL(128)
RT_ATTN_KERNEL(256)

// Fused decode attention for one new token at position `pos` (new, for the
// graph-captured decode step).  Equivalent to fused_rope_qk_f32 on (q, k),
// kv_copy_to_cache_f32 of k and v at `pos`, then decode_attention_f32 with
// kv_len = pos + 1.  The first query head of each group writes the rotated key
// and the value into the cache; every workgroup takes position `pos` from its
// own LDS copy, so no workgroup waits for another's cache write.
template <int HD>
RT_DEV void attn_rope_head(const float* q_raw, const float* k_raw, const float* v_raw,
                           float* k_cache, float* v_cache, float* O, uint32_t pos,
                           uint32_t max_seq, uint32_t num_heads, uint32_t num_kv_heads,
                           float theta, float scale) {
    __shared__ float qs[HD], ks[HD], vs[HD], qr[HD], sc[ATT_CHUNK], red[16];
    __shared__ f32x4 part[ATT_T];
    const uint32_t h = blockIdx.x, group = num_heads / num_kv_heads, kvh = h / group;
    constexpr uint32_t half = HD / 2;
    const float* q = q_raw + (size_t)h * HD;
    const float* k = k_raw + (size_t)kvh * HD;
    const float* v = v_raw + (size_t)kvh * HD;
    for (uint32_t d = threadIdx.x; d < half; d += blockDim.x) {
        float c, s;
        rope_cs(d, HD, pos, theta, c, s);
        const float q0 = q[d], q1 = q[d + half], k0 = k[d], k1 = k[d + half];
        qr[d] = q0 * c - q1 * s;
        qr[d + half] = q0 * s + q1 * c;
        ks[d] = k0 * c - k1 * s;
        ks[d + half] = k0 * s + k1 * c;
    }
    for (uint32_t d = threadIdx.x; d < HD; d += blockDim.x) vs[d] = v[d];
    __syncthreads();
    float* kc = k_cache + (size_t)kvh * max_seq * HD;
    float* vc = v_cache + (size_t)kvh * max_seq * HD;
    if (h % group == 0) {
        for (uint32_t d = threadIdx.x; d < HD; d += blockDim.x) {
            kc[(size_t)pos * HD + d] = ks[d];
            vc[(size_t)pos * HD + d] = vs[d];
        }
    }
    AttnIO io{qr, kc, vc, ks, vs};
    attend<HD>(io, O + (size_t)h * HD, pos + 1, scale, qs, sc, red, part);
}
#define RT_ATTN_ROPE_KERNEL(HD)                                                                   \
    extern "C" __global__ void __launch_bounds__(256) k_attn_rope_f32_hd##HD(                      \
        const float* q_raw, const float* k_raw, const float* v_raw, float* k_cache,                \
        float* v_cache, float* O, uint32_t pos, uint32_t max_seq, uint32_t num_heads,              \
        uint32_t num_kv_heads, float theta, float scale) {                                         \
        attn_rope_head<HD>(q_raw, k_raw, v_raw, k_cache, v_cache, O, pos, max_seq, num_heads,      \
                           num_kv_heads, theta, scale);                                            \
    }
RT_ATTN_ROPE_KERNEL(64)
RT_ATTN_ROPE_KERNEL(128)
RT_ATTN_ROPE_KERNEL(256)

// Q8_0 embedding row (the reference copies a dequantised token_embd row into
// the residual stream on the CPU, forward.rs:1494-1505).  The token id is
// read from device memory so a captured decode step can consume the previous
// step's argmax without a host round trip.
extern "C" __global__ void __launch_bounds__(256)
k_embed_q8_0_f32(const uint8_t* table, const uint32_t* token, float* out, uint32_t k) {
    const size_t row = (size_t)token[0] * (k / 32) * 34;
    for (uint32_t i = threadIdx.x + blockIdx.x * blockDim.x; i < k; i += blockDim.x * gridDim.x) {
        const uint8_t* blk = table + row + (i / 32) * 34;
        out[i] = __fmul_rn(h2f(*(const uint16_t*)blk), (float)(int8_t)blk[2 + (i & 31)]);
    }
}
