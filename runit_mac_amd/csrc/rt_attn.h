// rt_attn.h — device bodies shared by the decode kernels (k_decode.hip) and
// the persistent decode step (k_step.hip): workgroup reductions, the RoPE
// angle and split-KV decode attention.
#pragma once
#include "rt_device.h"
#include "rt_shared.h"

// Sum over a workgroup (any multiple of 64 threads ≤ 1024); `red` holds ≥ 16
// floats of LDS.  Every thread receives the total.
RT_DEV float block_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const uint32_t w = threadIdx.x >> 6, nw = wg_threads() >> 6;
    __syncthreads();  // previous users of `red` are done
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (uint32_t i = 0; i < nw; ++i) t += red[i];
    return t;
}
RT_DEV float block_max(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const uint32_t w = threadIdx.x >> 6, nw = wg_threads() >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = -__builtin_huge_valf();
    for (uint32_t i = 0; i < nw; ++i) t = fmaxf(t, red[i]);
    return t;
}

// RoPE angle for pair d (fused_rope.metal:34-38): freq = 1/θ^(2d/hd).
RT_DEV void rope_cs(uint32_t d, uint32_t head_dim, uint32_t pos, float theta, float& c, float& s) {
    const float freq = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
    const float angle = (float)pos * freq;
    sincosf(angle, &s, &c);
}

// ───────────────────────────── attention ─────────────────────────────
//
// Split-KV decode attention.  Decode attention reads a few hundred KB per
// layer, so it is bound by memory latency, not bandwidth: the design keeps the
// number of dependent memory round trips per workgroup at one per 64
// positions and spreads the positions over many workgroups.
//
// Grid (nsplit, num_kv_heads · head_blocks, batch), 256 threads.  Workgroup
// (s, kvh·HB + hb, b) takes positions [s·chunk, min(kv_len, (s+1)·chunk)) of
// kv head kvh for the (up to rt_attn_gm(HD)) query heads of head block hb of that kv
// head's group, so each K/V row is fetched once for all of them.  Per 64
// positions:
//   loads  : thread t holds a quarter of key row t/4 and HD/16 float4 of the
//            value rows ≡ t/(HD/4) (mod 1024/HD), column t % (HD/4) — all
//            issued together;
//   scores : quarter dots reduced over 4 lanes, written to LDS;
//   softmax: one wave per query head (64 lanes = 64 positions), running
//            max / sum with rescaling (the online softmax of
//            attention.metal:248-308);
//   output : each thread accumulates its value rows weighted by the
//            probabilities.
// With nsplit > 1 each workgroup writes (m, l, o) for its heads; the last
// workgroup of a (b, kvh, hb) group to arrive (arrival counter, reset by that
// workgroup) merges the splits in split order.
constexpr uint32_t ATT_SUB = 64;  // positions per inner step

struct AttnArgs {
    const float* q;       // [batch][H][HD]; with rope: the raw query of the token
    float* kc;            // cache [batch][KVH][stride][HD]
    float* vc;
    float* out;           // [batch][H][HD]
    const float* k_new;   // rope: raw key / value of the token, [KVH][HD]
    const float* v_new;
    float* part;          // nsplit > 1: [batch][H][nsplit][HD] unnormalised outputs
    float* ml;            //             [batch][H][nsplit][2] running max, sum
    uint32_t* counters;   //             [batch][KVH][HB] arrival counters
    uint32_t kv_len, stride, H, KVH, chunk, pos;
    float scale, theta;
    uint32_t parts_only;  // write (o, m, l) of every split, merge nothing (the
                          // consumer merges: k_gemv_q8_0_attn_f32add)
    uint32_t q_len;       // > 0: causal multi-query rows (no rope): grid row b is
                          // query r = b % q_len of sequence b / q_len, at
                          // position q_start + r; it attends to the first
                          // min(kv_len, q_start + r + 1) positions of its
                          // sequence's cache
    uint32_t q_start;
};

// (s, nsp, y, b): the split, the number of splits, the (kv head, head
// block) index and the batch row — the grid position of a stand-alone launch,
// or a persistent kernel's virtual one.  COH: q / k / v come from other
// workgroups of the same launch (device-scope loads); Hook: see NoHook.
template <int HD, bool ROPE, int HG, int GMT, bool COH = false, class Hook = NoHook>
RT_DEV void attn_split(const AttnArgs& a, uint32_t s, uint32_t nsp, uint32_t y, uint32_t b,
                       const Hook& hook = Hook()) {
    // HG groups of 256 threads share the block's query heads: group g takes
    // heads g, g + HG, ... (shorter per-thread chains; every group reads the
    // same K / V rows)
    constexpr uint32_t GM = GMT, SUB = ATT_SUB, NT = 256 * HG, HPT = GM / HG;
    constexpr uint32_t NQ = HD / 16;   // float4 per thread: K quarter row, V rows
    constexpr uint32_t C4 = HD / 4;    // float4 columns of a row
    constexpr uint32_t PG = 256 / C4;  // value position groups
    static_assert(SUB == 64 && NQ * PG == SUB && GM % HG == 0, "layout");
    __shared__ f32x4 qs4[GM][C4];
    __shared__ f32x4 ks4[C4], vs4[C4];
    __shared__ float sc[GM][SUB];
    __shared__ float m_run[GM], l_run[GM], resc[GM];
    __shared__ f32x4 ored[4][GM][C4];
    __shared__ uint32_t last_flag;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t hg = tid >> 8, lt = tid & 255, lw = w & 3;  // group, thread / wave in group
    const uint32_t G = a.H / a.KVH, HB = (G + GM - 1) / GM;
    const uint32_t kvh = y / HB, hb = y % HB;
    const uint32_t gh = min(GM, G - hb * GM);
    const uint32_t h0 = kvh * G + hb * GM;  // first query head of the block
    // causal rows share their sequence's cache and see a prefix of it
    const uint32_t seq = a.q_len ? b / a.q_len : b;
    const uint32_t kv_len = a.q_len ? min(a.kv_len, a.q_start + b % a.q_len + 1) : a.kv_len;
    const size_t kvb = ((size_t)seq * a.KVH + kvh) * a.stride * HD;
    float* kc = a.kc + kvb;
    float* vc = a.vc + kvb;
    // (a split past a causal row's prefix is empty: it contributes m = −∞, l = 0)
    const uint32_t p_begin = s * a.chunk, p_end = min(kv_len, p_begin + a.chunk);
    float* qsf = (float*)qs4;
    const uint32_t kp = lt >> 2, kq = lt & 3;      // key layout
    const uint32_t vcol = lt % C4, vg = lt / C4;  // value layout
    // K / V rows of a step (rows past the range load row p_begin: in bounds,
    // their scores are masked); the first step's loads are issued before the
    // query staging, each later step's while the previous one computes
    auto load_kv = [&](uint32_t p0, f32x4 (&kr)[NQ], f32x4 (&vr)[NQ]) {
        const uint32_t pk = p0 + kp;
        const f32x4* krow = (const f32x4*)(kc + (size_t)(pk < p_end ? pk : p_begin) * HD) + kq * NQ;
#pragma unroll
        for (uint32_t i = 0; i < NQ; ++i) kr[i] = krow[i];
#pragma unroll
        for (uint32_t i = 0; i < NQ; ++i) {
            const uint32_t pv = p0 + vg + i * PG;
            vr[i] = ((const f32x4*)(vc + (size_t)(pv < p_end ? pv : p_begin) * HD))[vcol];
        }
    };
    // The token's raw query / key / value (or the queries) go to registers
    // first: a stand-alone launch issues them ahead of the K / V rows, which
    // would otherwise queue in front of them (the RoPE and the scores wait for
    // the query); a persistent phase issues the K / V rows before its hook,
    // since only the token's vectors depend on the previous phase.
    auto act = [&](const float* p) { if constexpr (COH) return dev_load(p); else return *p; };
    constexpr uint32_t half = HD / 2;
    constexpr uint32_t PPT = ((GM + 1) * half + NT - 1) / NT;  // (q heads + key) pairs per thread
    constexpr uint32_t VPT = (HD + NT - 1) / NT;               // value elements per thread
    constexpr uint32_t QPT = (GM * HD + NT - 1) / NT;          // query elements per thread (no rope)
    const uint32_t npair = (gh + 1) * half;
    float rre[ROPE ? PPT : 1], rim[ROPE ? PPT : 1], rv[ROPE ? VPT : 1], rq[ROPE ? 1 : QPT];
    auto load_token = [&]() {
        if constexpr (ROPE) {
#pragma unroll
            for (uint32_t j = 0; j < PPT; ++j) {
                const uint32_t i = tid + j * NT, ii = i < npair ? i : 0;
                const uint32_t hh = ii / half, d = ii % half;
                const float* src = hh < gh ? a.q + (size_t)(h0 + hh) * HD : a.k_new + (size_t)kvh * HD;
                rre[j] = act(src + d);
                rim[j] = act(src + d + half);
            }
#pragma unroll
            for (uint32_t j = 0; j < VPT; ++j) {
                const uint32_t dd = tid + j * NT;
                rv[j] = act(a.v_new + (size_t)kvh * HD + (dd < HD ? dd : 0));
            }
        } else {
            const float* q = a.q + ((size_t)b * a.H + h0) * HD;
#pragma unroll
            for (uint32_t j = 0; j < QPT; ++j) {
                const uint32_t i = tid + j * NT;
                rq[j] = act(q + (i < gh * HD ? i : 0));
            }
        }
    };
    f32x4 kr[NQ], vr[NQ];
    if constexpr (is_hook<Hook>()) {
        if (p_begin < p_end) load_kv(p_begin, kr, vr);
        hook();
        load_token();
    } else {
        load_token();
        if (p_begin < p_end) load_kv(p_begin, kr, vr);
    }
    if constexpr (ROPE) {
        // fused_rope_qk_f32 (fused_rope.metal:28-55) on the block's query
        // heads and on the kv head's key
#pragma unroll
        for (uint32_t j = 0; j < PPT; ++j) {
            const uint32_t i = tid + j * NT;
            if (i < npair) {
                const uint32_t hh = i / half, d = i % half;
                float c, sn;
                rope_cs(d, HD, a.pos, a.theta, c, sn);
                float* dst = hh < gh ? qsf + hh * HD : (float*)ks4;
                dst[d] = rre[j] * c - rim[j] * sn;
                dst[d + half] = rre[j] * sn + rim[j] * c;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < VPT; ++j) {
            const uint32_t dd = tid + j * NT;
            if (dd < HD) ((float*)vs4)[dd] = rv[j];
        }
    } else {
#pragma unroll
        for (uint32_t j = 0; j < QPT; ++j) {
            const uint32_t i = tid + j * NT;
            if (i < gh * HD) qsf[i] = rq[j];
        }
    }
    if (tid < GM) {
        m_run[tid] = -__builtin_huge_valf();
        l_run[tid] = 0.0f;
    }
    lds_barrier();
    if constexpr (ROPE) {
        // kv_copy_to_cache_f32 (activation.metal:30-45) of the rotated key and
        // the value, by the one workgroup whose range holds `pos`
        if (hb == 0 && a.pos >= p_begin && a.pos < p_end)
            for (uint32_t d = tid; d < HD; d += NT) {
                kc[(size_t)a.pos * HD + d] = ((const float*)ks4)[d];
                vc[(size_t)a.pos * HD + d] = ((const float*)vs4)[d];
            }
    }
    f32x4 oacc[HPT];  // heads hg + HG·j
#pragma unroll
    for (uint32_t j = 0; j < HPT; ++j) oacc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t p0 = p_begin; p0 < p_end; p0 += SUB) {
        const uint32_t pk = p0 + kp;
        const bool kvalid = pk < p_end;
        f32x4 kn[NQ], vn[NQ];
        if (p0 + SUB < p_end) load_kv(p0 + SUB, kn, vn);  // next step (workgroup-uniform)
        if constexpr (ROPE) {
            // position `pos` comes from LDS (the cache write above may not be
            // visible to this workgroup's loads, and other workgroups never
            // read it)
            if (pk == a.pos)
#pragma unroll
                for (uint32_t i = 0; i < NQ; ++i) kr[i] = ks4[kq * NQ + i];
#pragma unroll
            for (uint32_t i = 0; i < NQ; ++i)
                if (p0 + vg + i * PG == a.pos) vr[i] = vs4[vcol];
        }
#pragma unroll
        for (uint32_t j = 0; j < HPT; ++j) {
            const uint32_t h = hg + HG * j;
            if (h < gh) {
                float dot = 0.0f;
#pragma unroll
                for (uint32_t i = 0; i < NQ; ++i) {
                    const f32x4 qv = qs4[h][kq * NQ + i];
                    dot += qv.x * kr[i].x + qv.y * kr[i].y + qv.z * kr[i].z + qv.w * kr[i].w;
                }
                dot = group_sum(dot, 4);
                if (kq == 0) sc[h][kp] = kvalid ? dot * a.scale : -__builtin_huge_valf();
            }
        }
        lds_barrier();
        // softmax: wave w takes query heads w, w + 4·HG (one or two per wave)
#pragma unroll
        for (uint32_t u = 0; u < (GM + 4 * HG - 1) / (4 * HG); ++u) {
            const uint32_t h = w + 4 * HG * u;
            if (h < GM) {  // wave-uniform
                const float sv = h < gh ? sc[h][lane] : -__builtin_huge_valf();
                const float mx = group_max(sv, 64);
                const float m_old = h < gh ? m_run[h] : 0.0f, m_new = fmaxf(m_old, mx);
                const float e = (sv == -__builtin_huge_valf()) ? 0.0f : expf(sv - m_new);
                const float sum = group_sum(e, 64);
                if (h < gh) {
                    sc[h][lane] = e;
                    if (lane == 0) {
                        const float r =
                            (m_old == -__builtin_huge_valf()) ? 0.0f : expf(m_old - m_new);
                        resc[h] = r;
                        l_run[h] = l_run[h] * r + sum;
                        m_run[h] = m_new;
                    }
                }
            }
        }
        lds_barrier();
#pragma unroll
        for (uint32_t j = 0; j < HPT; ++j) {
            const uint32_t h = hg + HG * j;
            if (h < gh) {
                f32x4 acc = oacc[j] * resc[h];
#pragma unroll
                for (uint32_t i = 0; i < NQ; ++i) acc += sc[h][vg + i * PG] * vr[i];
                oacc[j] = acc;
            }
        }
        lds_barrier();  // sc / resc reused by the next step
        if (p0 + SUB < p_end) {
#pragma unroll
            for (uint32_t i = 0; i < NQ; ++i) {
                kr[i] = kn[i];
                vr[i] = vn[i];
            }
        }
    }
    // sum the value position groups: within the wave, then over the group's
    // 4 waves
#pragma unroll
    for (uint32_t j = 0; j < HPT; ++j) {
        const uint32_t h = hg + HG * j;
        if (h < gh) {
            f32x4 v = oacc[j];
            if constexpr (C4 == 16) {
                v.x += swz_xor_f<16>(v.x);
                v.y += swz_xor_f<16>(v.y);
                v.z += swz_xor_f<16>(v.z);
                v.w += swz_xor_f<16>(v.w);
            }
            if constexpr (C4 <= 32) {
                v.x += __shfl_xor(v.x, 32, 64);
                v.y += __shfl_xor(v.y, 32, 64);
                v.z += __shfl_xor(v.z, 32, 64);
                v.w += __shfl_xor(v.w, 32, 64);
            }
            if (lane < C4) ored[lw][h][lane] = v;
        }
    }
    lds_barrier();
    const bool direct = nsp == 1 && !a.parts_only;
    for (uint32_t i = tid; i < gh * C4; i += NT) {
        const uint32_t h = i / C4, c = i % C4;
        const f32x4 t = ored[0][h][c] + ored[1][h][c] + ored[2][h][c] + ored[3][h][c];
        if (direct) {
            const float l = l_run[h];
            ((f32x4*)(a.out + ((size_t)b * a.H + h0 + h) * HD))[c] = t * (l > 0.0f ? 1.0f / l : 0.0f);
        } else {
            float* pp = a.part + (((size_t)b * a.H + h0 + h) * nsp + s) * HD + 4 * c;
            dev_store(pp + 0, t.x);
            dev_store(pp + 1, t.y);
            dev_store(pp + 2, t.z);
            dev_store(pp + 3, t.w);
        }
    }
    if (direct) return;
    if (tid < gh) {
        float* mlp = a.ml + (((size_t)b * a.H + h0 + tid) * nsp + s) * 2;
        dev_store(mlp + 0, m_run[tid]);
        dev_store(mlp + 1, l_run[tid]);
    }
    if (a.parts_only) return;
    dev_stores_done();
    __syncthreads();
    uint32_t* counter = a.counters + ((size_t)b * a.KVH + kvh) * HB + hb;
    if (tid == 0) last_flag = arrive(counter) == nsp - 1;
    __syncthreads();
    if (!last_flag) return;
    // merge the splits in split order: o = Σ o_s·e^(m_s−M) / Σ l_s·e^(m_s−M)
    for (uint32_t i = tid; i < gh * C4; i += NT) {
        const uint32_t h = i / C4, c = i % C4;
        const size_t row = ((size_t)b * a.H + h0 + h) * nsp;
        const float* mlv = a.ml + row * 2;
        float M = -__builtin_huge_valf();
#pragma unroll 8
        for (uint32_t j = 0; j < nsp; ++j) M = fmaxf(M, dev_load(mlv + 2 * j));
        float L = 0.0f;
        f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
        for (uint32_t j = 0; j < nsp; ++j) {
            const float f = expf(dev_load(mlv + 2 * j) - M);
            L += dev_load(mlv + 2 * j + 1) * f;
            const float* pj = a.part + (row + j) * HD + 4 * c;
            o += f32x4{dev_load(pj), dev_load(pj + 1), dev_load(pj + 2), dev_load(pj + 3)} * f;
        }
        ((f32x4*)(a.out + ((size_t)b * a.H + h0 + h) * HD))[c] = o * (L > 0.0f ? 1.0f / L : 0.0f);
    }
    if (tid == 0) dev_store(counter, 0u);  // ready for the next call (also under graph replay)
}

// Head groups and query heads per workgroup: rt_attn_hg / rt_attn_gm
// (rt_shared.h, shared with the host's grid sizing).
template <int HD> constexpr int attn_hg() { return (int)rt_attn_hg(HD); }
template <int HD> constexpr int attn_gm() { return (int)rt_attn_gm(HD); }


// ───────────── decode attention, wave form (one query head, RoPE) ─────────────
//
// The token's attention for one query head over one split of the KV range,
// with the split's positions spread over the 4 waves of a 256-thread
// workgroup: lane l of wave w holds dims [16·(l mod LPP), +16) of position
// p0 + PPW·w + l / LPP (LPP = HD/16 lanes per position, PPW = 64/LPP
// positions per wave), with the next step's K / V rows in flight.  Scores,
// the running max, the exponentials and the probability-weighted values are
// reduced inside the wave (cross-lane adds), each wave keeps its own running
// (m, l, o), and the 4 waves' states meet in LDS once, at the end — one
// barrier after the query staging and one for that merge, where attn_split
// takes three per 64 positions.  Output as attn_split's: the normalised o
// (one split) or the split's (o, m, l) for the consumer to merge.
template <int HD>
RT_DEV void attn_split_w(const AttnArgs& a, uint32_t s, uint32_t nsp, uint32_t y, uint32_t b) {
    constexpr uint32_t LPP = HD / 16, PPW = 64 / LPP, PPS = 4 * PPW, C4 = HD / 4, half = HD / 2;
    static_assert(HD == 64 || HD == 128, "head size");
    __shared__ f32x4 qs4[C4], ks4[C4], vs4[C4];
    __shared__ f32x4 wo[4][C4];
    __shared__ float wm[4], wl[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t G = a.H / a.KVH;
    const uint32_t kvh = y / G, hb = y % G;  // one query head per workgroup
    const uint32_t h = kvh * G + hb;
    const size_t kvb = ((size_t)b * a.KVH + kvh) * a.stride * HD;
    float* kc = a.kc + kvb;
    float* vc = a.vc + kvb;
    const uint32_t p_begin = s * a.chunk, p_end = min(a.kv_len, p_begin + a.chunk);
    const uint32_t kq = lane % LPP, pl = lane / LPP;
    auto load_kv = [&](uint32_t p0, f32x4 (&kr)[4], f32x4 (&vr)[4]) {
        const uint32_t p = p0 + PPW * w + pl;
        const size_t pc = p < p_end ? p : p_begin;
        const f32x4* kp = (const f32x4*)(kc + pc * HD) + 4 * kq;
        const f32x4* vp = (const f32x4*)(vc + pc * HD) + 4 * kq;
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[i] = kp[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) vr[i] = vp[i];
    };
    // the token's raw q / k (one RoPE pair per thread: threads [0, half) the
    // query, [half, HD) the key) and v (threads [HD, 2·HD)), loaded ahead of
    // the K / V rows
    const bool pair = tid < HD, isv = tid >= HD && tid < 2 * HD;
    const uint32_t d = tid % half;
    const float* src = tid < half ? a.q + (size_t)(b * a.H + h) * HD : a.k_new + (size_t)kvh * HD;
    float re = 0.0f, im = 0.0f, vv = 0.0f;
    if (pair) {
        re = src[d];
        im = src[d + half];
    }
    if (isv) vv = a.v_new[(size_t)kvh * HD + (tid - HD)];
    f32x4 kr[4], vr[4];
    if (p_begin < p_end) load_kv(p_begin, kr, vr);
    if (pair) {
        // fused_rope_qk_f32 (fused_rope.metal:28-55)
        float c, sn;
        rope_cs(d, HD, a.pos, a.theta, c, sn);
        float* dst = tid < half ? (float*)qs4 : (float*)ks4;
        dst[d] = re * c - im * sn;
        dst[d + half] = re * sn + im * c;
    }
    if (isv) ((float*)vs4)[tid - HD] = vv;
    lds_barrier();
    // kv_copy_to_cache_f32 (activation.metal:30-45) of the rotated key and the
    // value, by the first head's workgroup whose range holds `pos`
    if (hb == 0 && a.pos >= p_begin && a.pos < p_end && tid < C4) {
        ((f32x4*)(kc + (size_t)a.pos * HD))[tid] = ks4[tid];
        ((f32x4*)(vc + (size_t)a.pos * HD))[tid] = vs4[tid];
    }
    f32x4 qv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = qs4[4 * kq + i];
    float m = -__builtin_huge_valf(), l = 0.0f;
    f32x4 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // sum / max over the wave's positions (lanes ≡ kq mod LPP)
    auto pos_sum = [&](float v) {
#pragma unroll
        for (uint32_t x = LPP; x < 32; x <<= 1) v += __shfl_xor(v, x, 64);
        return v + __shfl_xor(v, 32, 64);
    };
    auto pos_max = [&](float v) {
#pragma unroll
        for (uint32_t x = LPP; x < 32; x <<= 1) v = fmaxf(v, __shfl_xor(v, x, 64));
        return fmaxf(v, __shfl_xor(v, 32, 64));
    };
    for (uint32_t p0 = p_begin; p0 < p_end; p0 += PPS) {
        f32x4 kn[4], vn[4];
        if (p0 + PPS < p_end) load_kv(p0 + PPS, kn, vn);  // next step (workgroup-uniform)
        const uint32_t p = p0 + PPW * w + pl;
        const bool valid = p < p_end;
        if (p == a.pos) {  // the token's own row (the cache write may not be visible yet)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kr[i] = ks4[4 * kq + i];
                vr[i] = vs4[4 * kq + i];
            }
        }
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            dot += qv[i].x * kr[i].x + qv[i].y * kr[i].y + qv[i].z * kr[i].z + qv[i].w * kr[i].w;
        dot = group_sum(dot, LPP);
        const float sc = valid ? dot * a.scale : -__builtin_huge_valf();
        const float m_new = fmaxf(m, pos_max(sc));
        // (a wave whose positions are all past the range keeps m = −∞)
        const float e = valid ? expf(sc - m_new) : 0.0f;
        const float r = (m == -__builtin_huge_valf()) ? 0.0f : expf(m - m_new);
        l = l * r + pos_sum(e);  // (e is the same in the LPP lanes of a position)
        m = m_new;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = o[i] * r + e * vr[i];
        if (p0 + PPS < p_end) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kr[i] = kn[i];
                vr[i] = vn[i];
            }
        }
    }
    // the wave's o over its positions, then the 4 waves' states in LDS
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[i].x = pos_sum(o[i].x);
        o[i].y = pos_sum(o[i].y);
        o[i].z = pos_sum(o[i].z);
        o[i].w = pos_sum(o[i].w);
    }
    if (lane < LPP) {
#pragma unroll
        for (int i = 0; i < 4; ++i) wo[w][4 * kq + i] = o[i];
    }
    if (lane == 0) {
        wm[w] = m;
        wl[w] = l;
    }
    lds_barrier();
    if (tid < C4) {
        float M = -__builtin_huge_valf();
#pragma unroll
        for (int v = 0; v < 4; ++v) M = fmaxf(M, wm[v]);
        float L = 0.0f;
        f32x4 O = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float f = wm[v] == -__builtin_huge_valf() ? 0.0f : expf(wm[v] - M);
            L += wl[v] * f;
            O += wo[v][tid] * f;
        }
        if (nsp == 1 && !a.parts_only) {
            ((f32x4*)(a.out + ((size_t)b * a.H + h) * HD))[tid] = O * (L > 0.0f ? 1.0f / L : 0.0f);
        } else {
            const size_t row = ((size_t)b * a.H + h) * nsp + s;
            ((f32x4*)(a.part + row * HD))[tid] = O;
            if (tid == 0) {
                a.ml[row * 2] = M;
                a.ml[row * 2 + 1] = L;
            }
        }
    }
}
