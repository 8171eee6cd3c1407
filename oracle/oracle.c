/*
 * oracle.c — CPU restatement of RunIT's quantized-GEMV decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker and CPU baseline, never
 * part of the shipped path.  Build flags: -O2 -ffp-contract=off (no FMA
 * contraction, no fast-math) so f32 arithmetic rounds like the reference's
 * Rust code.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ───────────────────────── f16 (half 2.7.1) ───────────────────────── */

float ora_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: m·2^-24 */
            float v = (float)m * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t ora_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* Inf / NaN (quiet, payload kept) */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    const int e = (int)(ax >> 23) - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 14 - e;
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry to Inf: correct */
    return (uint16_t)(sign | q);
}

static float rd_h(const uint8_t* p) { return ora_h2f((uint16_t)(p[0] | (p[1] << 8))); }

size_t ora_block_elems(int fmt) {
    return (fmt == ORA_Q4K || fmt == ORA_Q6K || fmt == ORA_Q5K || fmt == ORA_Q4KG ||
            fmt == ORA_Q5KG || fmt == ORA_Q6KG) ? 256 : 32;
}
size_t ora_block_bytes(int fmt) {
    switch (fmt) {
        case ORA_Q8_0: return 34;
        case ORA_Q4_0: return 18;
        case ORA_Q4K: return 144;
        case ORA_Q6K: return 210;
        case ORA_Q5_0: return 22;
        case ORA_Q5K: return 176;
        case ORA_Q4_0G: return 18;
        case ORA_Q4KG: return 144;
        case ORA_Q5KG: return 176;
        case ORA_Q6KG: return 210;
    }
    return 0;
}

/* ───────────────────────── dequantisers ───────────────────────── */

/* forward.rs:951-963: f32_vec.push(d * qs[i] as i8 as f32) */
void ora_dequant_q8_0(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 34;
        const float d = rd_h(blk);
        for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* forward.rs:964-978: byte = qs[i/2]; nibble = i%2==0 ? lo : hi;
 * push(d * (nibble as i32 - 8) as f32) */
void ora_dequant_q4_0(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 18;
        const float d = rd_h(blk);
        for (int i = 0; i < 32; ++i) {
            const uint8_t byte = blk[2 + i / 2];
            const int nib = (i % 2 == 0) ? (byte & 0x0F) : ((byte >> 4) & 0x0F);
            out[b * 32 + i] = d * (float)(nib - 8);
        }
    }
}

/* get_scale_min_k4, forward.rs:359-369 */
static void scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 0x3F;
        *m = s[j + 4] & 0x3F;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* forward.rs:1026-1057 */
void ora_dequant_q4k(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 144;
        const float d = rd_h(blk), dmin = rd_h(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qs = blk + 16;
        float* vals = out + b * 256;
        for (int j = 0; j < 4; ++j) {
            uint8_t sc_lo, m_lo, sc_hi, m_hi;
            scale_min_k4(j, scales, &sc_lo, &m_lo);
            scale_min_k4(j + 4, scales, &sc_hi, &m_hi);
            const float d_lo = d * (float)sc_lo, m_lo2 = dmin * (float)m_lo;
            const float d_hi = d * (float)sc_hi, m_hi2 = dmin * (float)m_hi;
            for (int l = 0; l < 32; ++l) {
                const uint8_t bv = qs[j * 32 + l];
                vals[j * 64 + l] = d_lo * (float)(bv & 0x0F) - m_lo2;
                vals[j * 64 + l + 32] = d_hi * (float)(bv >> 4) - m_hi2;
            }
        }
    }
}

/* forward.rs:921-950 (f32 variant; is = n_half/16, scales is+0,2,4,6) */
void ora_dequant_q6k(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const uint8_t* scales = blk + 192;
        const float d = rd_h(blk + 208);
        float* vals = out + b * 256;
        for (int n_half = 0; n_half < 256; n_half += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = n_half / 16;
                const int i0 = n_half / 2 + l, i1 = n_half / 2 + l + 32, ih = n_half / 4 + l;
                const int q1 = ((ql[i0] & 0x0F) | (((qh[ih] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[i1] & 0x0F) | (((qh[ih] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[i0] >> 4) | (((qh[ih] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[i1] >> 4) | (((qh[ih] >> 6) & 3) << 4)) - 32;
                vals[n_half + l + 0] = d * (float)(int8_t)scales[is + 0] * (float)q1;
                vals[n_half + l + 32] = d * (float)(int8_t)scales[is + 2] * (float)q2;
                vals[n_half + l + 64] = d * (float)(int8_t)scales[is + 4] * (float)q3;
                vals[n_half + l + 96] = d * (float)(int8_t)scales[is + 6] * (float)q4;
            }
        }
    }
}

/* forward.rs:900-920: d f16, qh[4], qs[16]; for j in 0..16:
 * xh_0 = (qh[j/8] >> j%8) & 1, xh_1 = (qh[j/8+2] >> j%8) & 1,
 * vals[j] = d·((qs[j]&15 | xh_0<<4) − 16), vals[j+16] = d·((qs[j]>>4 | xh_1<<4) − 16) */
void ora_dequant_q5_0(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 22;
        const float d = rd_h(blk);
        const uint8_t* qh = blk + 2;
        const uint8_t* qs = blk + 6;
        for (int j = 0; j < 16; ++j) {
            const int xh0 = (qh[j / 8] >> (j % 8)) & 1;
            const int xh1 = (qh[j / 8 + 2] >> (j % 8)) & 1;
            const int x0 = (qs[j] & 0x0F) | (xh0 << 4);
            const int x1 = ((qs[j] >> 4) & 0x0F) | (xh1 << 4);
            out[b * 32 + j] = d * (float)(x0 - 16);
            out[b * 32 + j + 16] = d * (float)(x1 - 16);
        }
    }
}

/* forward.rs:979-1012: d, dmin f16, scales[12], qh[32], qs[128]; pair j
 * uses (sc, m) j and j+4 (get_scale_min_k4); element e = 64j+l (+32) takes
 * the low (high) nibble of qs[32j+l] and bit e%8 of qh[e/8] as bit 4. */
void ora_dequant_q5k(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 176;
        const float d = rd_h(blk), dmin = rd_h(blk + 2);
        const uint8_t* scales = blk + 4;
        const uint8_t* qh = blk + 16;
        const uint8_t* qs = blk + 48;
        float* vals = out + b * 256;
        for (int j = 0; j < 4; ++j) {
            uint8_t sc_lo, m_lo, sc_hi, m_hi;
            scale_min_k4(j, scales, &sc_lo, &m_lo);
            scale_min_k4(j + 4, scales, &sc_hi, &m_hi);
            const float d_lo = d * (float)sc_lo, m_lo2 = dmin * (float)m_lo;
            const float d_hi = d * (float)sc_hi, m_hi2 = dmin * (float)m_hi;
            for (int l = 0; l < 32; ++l) {
                const uint8_t bv = qs[j * 32 + l];
                const int elo = j * 64 + l, ehi = j * 64 + l + 32;
                const unsigned hlo = (qh[elo / 8] >> (elo % 8)) & 1;
                const unsigned hhi = (qh[ehi / 8] >> (ehi % 8)) & 1;
                vals[elo] = d_lo * (float)((bv & 0x0Fu) | (hlo << 4)) - m_lo2;
                vals[ehi] = d_hi * (float)((unsigned)(bv >> 4) | (hhi << 4)) - m_hi2;
            }
        }
    }
}

/* ggml dequantize_row_q4_0: x0 = (qs[j] & 0x0F) − 8, x1 = (qs[j] >> 4) − 8,
 * y[j] = x0·d, y[j + 16] = x1·d */
void ora_dequant_q4_0g(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 18;
        const float d = rd_h(blk);
        for (int j = 0; j < 16; ++j) {
            const int x0 = (blk[2 + j] & 0x0F) - 8, x1 = (blk[2 + j] >> 4) - 8;
            out[b * 32 + j] = (float)x0 * d;
            out[b * 32 + j + 16] = (float)x1 * d;
        }
    }
}

/* ggml dequantize_row_q4_K / _q5_K: for chunk j (64 elements, sub-blocks
 * is = 2j, 2j+1): d1 = d·sc, m1 = min·m; y[l] = d1·q_lo − m1, y[32+l] = d2·q_hi − m2;
 * Q5_K adds 16 when bit 2j (low) / 2j+1 (high) of qh[l] is set. */
static void dequant_k_ggml(const uint8_t* blk, const uint8_t* qh, const uint8_t* qs, float* y) {
    const float d = rd_h(blk), dmin = rd_h(blk + 2);
    const uint8_t* scales = blk + 4;
    for (int j = 0; j < 4; ++j) {
        uint8_t sc, m;
        scale_min_k4(2 * j, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        scale_min_k4(2 * j + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) {
            int q1 = qs[32 * j + l] & 0x0F, q2 = qs[32 * j + l] >> 4;
            if (qh) {
                q1 += (qh[l] >> (2 * j)) & 1 ? 16 : 0;
                q2 += (qh[l] >> (2 * j + 1)) & 1 ? 16 : 0;
            }
            y[64 * j + l] = d1 * (float)q1 - m1;
            y[64 * j + 32 + l] = d2 * (float)q2 - m2;
        }
    }
}
void ora_dequant_q4kg(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) dequant_k_ggml(in + b * 144, NULL, in + b * 144 + 16, out + b * 256);
}
void ora_dequant_q5kg(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b)
        dequant_k_ggml(in + b * 176, in + b * 176 + 16, in + b * 176 + 48, out + b * 256);
}

/* ggml dequantize_row_q6_K: is = l/16; y[l + 32t] = d·sc[is + 2t]·q_t, the
 * scale pointer advancing by 8 per 128-element half */
void ora_dequant_q6kg(const uint8_t* in, size_t nblk, float* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const uint8_t* blk = in + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        const float d = rd_h(blk + 208);
        float* y = out + b * 256;
        for (int n = 0; n < 2; ++n) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * (float)sc[is + 0] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

void ora_dequant(int fmt, const uint8_t* in, size_t nblk, float* out) {
    switch (fmt) {
        case ORA_Q8_0: ora_dequant_q8_0(in, nblk, out); break;
        case ORA_Q4_0: ora_dequant_q4_0(in, nblk, out); break;
        case ORA_Q4K: ora_dequant_q4k(in, nblk, out); break;
        case ORA_Q6K: ora_dequant_q6k(in, nblk, out); break;
        case ORA_Q5_0: ora_dequant_q5_0(in, nblk, out); break;
        case ORA_Q5K: ora_dequant_q5k(in, nblk, out); break;
        case ORA_Q4_0G: ora_dequant_q4_0g(in, nblk, out); break;
        case ORA_Q4KG: ora_dequant_q4kg(in, nblk, out); break;
        case ORA_Q5KG: ora_dequant_q5kg(in, nblk, out); break;
        case ORA_Q6KG: ora_dequant_q6kg(in, nblk, out); break;
    }
}

/* dequant.metal:53-98: half(actual_scale * q - actual_min) */
void ora_dequant_q4k_f16(const uint8_t* in, size_t nblk, uint16_t* out) {
    float tmp[256];
    for (size_t b = 0; b < nblk; ++b) {
        ora_dequant_q4k(in + b * 144, 1, tmp);
        for (int i = 0; i < 256; ++i) out[b * 256 + i] = ora_f2h(tmp[i]);
    }
}

/* ───────────────────────── GEMV ───────────────────────── */

void ora_gemv_packed(int fmt, const uint8_t* w, const float* x, size_t m_vec, size_t n,
                     size_t k, double* y, double* sabs) {
    const size_t be = ora_block_elems(fmt), bb = ora_block_bytes(fmt);
    const size_t nb = k / be, rb = nb * bb;
#pragma omp parallel
    {
        float* row = (float*)malloc(k * sizeof(float));
#pragma omp for schedule(static)
        for (long long r = 0; r < (long long)n; ++r) {
            ora_dequant(fmt, w + (size_t)r * rb, nb, row);
            for (size_t mv = 0; mv < m_vec; ++mv) {
                const float* xv = x + mv * k;
                double acc = 0.0, sa = 0.0;
                for (size_t c = 0; c < k; ++c) {
                    const double p = (double)row[c] * (double)xv[c];
                    acc += p;
                    sa += fabs(p);
                }
                y[mv * n + (size_t)r] = acc;
                sabs[mv * n + (size_t)r] = sa;
            }
        }
        free(row);
    }
}

/* cpu_gemv (dispatch.rs:1705-1709): (0..k).map(|c| a[r*k+c] * x[c]).sum() */
void ora_gemv_ref_f32(int fmt, const uint8_t* w, const float* x, size_t n, size_t k, float* y,
                      int threads) {
    const size_t be = ora_block_elems(fmt), bb = ora_block_bytes(fmt);
    const size_t nb = k / be, rb = nb * bb;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
#endif
    {
        float* row = (float*)malloc(k * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (long long r = 0; r < (long long)n; ++r) {
            ora_dequant(fmt, w + (size_t)r * rb, nb, row);
            float acc = 0.0f;
            for (size_t c = 0; c < k; ++c) acc += row[c] * x[c];
            y[r] = acc;
        }
        free(row);
    }
    (void)threads;
}

double ora_silu(double x) { return x / (1.0 + exp(-x)); }

/* sampler.rs:111-116: iter().enumerate().max_by(partial_cmp or Equal) —
 * the running best is replaced unless it compares Greater. */
uint32_t ora_argmax_f32(const float* v, size_t n) {
    if (n == 0) return 0;
    size_t best = 0;
    for (size_t i = 1; i < n; ++i) {
        const float m = v[best], c = v[i];
        const int greater = (m > c); /* partial_cmp == Some(Greater) */
        if (!greater) best = i;
    }
    return (uint32_t)best;
}

/* ───────────────────────── decode glue ───────────────────────── */

void ora_rms_norm(const float* x, const float* gamma, double eps, size_t hidden, size_t rows,
                  double* y) {
    for (size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * hidden;
        double ss = 0.0;
        for (size_t i = 0; i < hidden; ++i) ss += (double)xr[i] * (double)xr[i];
        const double inv = 1.0 / sqrt(ss / (double)hidden + eps);
        for (size_t i = 0; i < hidden; ++i) y[r * hidden + i] = (double)xr[i] * inv * (double)gamma[i];
    }
}

void ora_rope(double* v, size_t heads, size_t head_dim, uint32_t pos, float theta) {
    const size_t half = head_dim / 2;
    for (size_t d = 0; d < half; ++d) {
        const float freq = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
        const float angle = (float)pos * freq;
        const double c = cos((double)angle), s = sin((double)angle);
        for (size_t h = 0; h < heads; ++h) {
            double* x = v + h * head_dim;
            const double r = x[d], i = x[d + half];
            x[d] = r * c - i * s;
            x[d + half] = r * s + i * c;
        }
    }
}

void ora_rope_batch(double* v, size_t seq, size_t heads, size_t head_dim, uint32_t start_pos,
                    float theta) {
    const size_t half = head_dim / 2;
    for (size_t s = 0; s < seq; ++s)
        for (size_t d = 0; d < half; ++d) {
            const float angle =
                (float)(start_pos + (uint32_t)s) / powf(theta, (float)(2 * d) / (float)head_dim);
            const double c = cos((double)angle), sn = sin((double)angle);
            for (size_t h = 0; h < heads; ++h) {
                double* x = v + (s * heads + h) * head_dim;
                const double r = x[d], i = x[d + half];
                x[d] = r * c - i * sn;
                x[d + half] = i * c + r * sn;
            }
        }
}

void ora_argmax_rows_first_f32(const float* v, size_t rows, size_t n, uint32_t* out) {
    for (size_t r = 0; r < rows; ++r) {
        const float* row = v + r * n;
        uint32_t best = 0;
        float best_val = -INFINITY;
        for (size_t j = 0; j < n; ++j)
            if (row[j] > best_val) {
                best_val = row[j];
                best = (uint32_t)j;
            }
        out[r] = best;
    }
}

void ora_attention(const double* q, const float* k, const float* v, size_t num_heads,
                   size_t num_kv_heads, size_t head_dim, size_t kv_len, size_t kv_stride,
                   double scale, double* out) {
    const size_t group = num_heads / num_kv_heads;
    double* sc = (double*)malloc((kv_len ? kv_len : 1) * sizeof(double));
    for (size_t h = 0; h < num_heads; ++h) {
        const size_t kvh = h / group;
        const double* qh = q + h * head_dim;
        double m = -INFINITY;
        for (size_t j = 0; j < kv_len; ++j) {
            const float* kr = k + (kvh * kv_stride + j) * head_dim;
            double dot = 0.0;
            for (size_t d = 0; d < head_dim; ++d) dot += qh[d] * (double)kr[d];
            sc[j] = dot * scale;
            if (sc[j] > m) m = sc[j];
        }
        double l = 0.0;
        for (size_t j = 0; j < kv_len; ++j) {
            sc[j] = exp(sc[j] - m);
            l += sc[j];
        }
        for (size_t d = 0; d < head_dim; ++d) {
            double o = 0.0;
            for (size_t j = 0; j < kv_len; ++j) o += sc[j] * (double)v[(kvh * kv_stride + j) * head_dim + d];
            out[h * head_dim + d] = l > 0.0 ? o / l : 0.0;
        }
    }
    free(sc);
}

/* ───────────────────────── synthetic data ───────────────────────── */

static uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* ln(u) for u in (0, 1] and cos(2π·v) for v in [0, 1), built from correctly
 * rounded f32 operations only (+, −, ×, /, fmaf; no contraction), so that the
 * device generator, which evaluates the same sequence, yields the same bits.
 * ln: u = m·2^e with m in [√½, √2), ln m = 2·atanh(s), s = (m−1)/(m+1), odd
 * series to s^11 (|s| ≤ 0.172).  cos: quadrant n = rint(4v), r = v − n/4 in
 * [−1/8, 1/8] (exact), θ = 2π·r, Taylor series of sin / cos to degree 11 / 10. */
static float synth_ln(float u) {
    int e = 0;
    float m = frexpf(u, &e); /* u = m·2^e, m in [0.5, 1) */
    if (m < 0.70710678f) { m = m * 2.0f; e -= 1; }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float z = s * s;
    float p = fmaf(z, 1.0f / 11.0f, 1.0f / 9.0f);
    p = fmaf(z, p, 1.0f / 7.0f);
    p = fmaf(z, p, 1.0f / 5.0f);
    p = fmaf(z, p, 1.0f / 3.0f);
    const float lnm = fmaf(2.0f * s, z * p, 2.0f * s);
    return fmaf((float)e, 0.693147182f, lnm);
}
static float synth_cos2pi(float v) {
    const float n = rintf(4.0f * v);
    const float r = v - 0.25f * n;
    const float t = r * 6.28318548f;
    const float z = t * t;
    float c = fmaf(z, -2.75573192e-7f, 2.48015873e-5f);
    c = fmaf(z, c, -1.38888889e-3f);
    c = fmaf(z, c, 4.16666667e-2f);
    c = fmaf(z, c, -0.5f);
    c = fmaf(z, c, 1.0f);
    float sn = fmaf(z, -2.50521084e-8f, 2.75573192e-6f);
    sn = fmaf(z, sn, -1.98412698e-4f);
    sn = fmaf(z, sn, 8.33333333e-3f);
    sn = fmaf(z, sn, -1.66666667e-1f);
    sn = fmaf(t * z, sn, t);
    switch (((int)n) & 3) {
    case 0: return c;
    case 1: return -sn;
    case 2: return -c;
    default: return sn;
    }
}

float ora_synth_normal(uint64_t seed, uint64_t idx) {
    const uint64_t h = splitmix64(seed ^ splitmix64(idx));
    const float u1 = (float)((h >> 40) + 1) * 5.9604644775390625e-8f;  /* (0, 1] */
    const float u2 = (float)(h & 0xFFFFFFull) * 5.9604644775390625e-8f; /* [0, 1) */
    return sqrtf(-2.0f * synth_ln(u1)) * synth_cos2pi(u2);
}

void ora_synth_normal_f32(uint64_t seed, uint64_t n, float mean, float stdv, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) out[i] = mean + stdv * ora_synth_normal(seed, (uint64_t)i);
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
static void wr_h(uint8_t* p, uint16_t h) { p[0] = (uint8_t)(h & 255); p[1] = (uint8_t)(h >> 8); }

void ora_quantize_q8_0(const float* w, size_t nblk, uint8_t* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const float* x = w + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
        const float d = amax / 127.0f;
        uint8_t* p = out + b * 34;
        wr_h(p, ora_f2h(d));
        for (int i = 0; i < 32; ++i) {
            const int q = d > 0.0f ? (int)roundf(x[i] / d) : 0;
            p[2 + i] = (uint8_t)(int8_t)clampi(q, -127, 127);
        }
    }
}

void ora_quantize_q4_0(const float* w, size_t nblk, uint8_t* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const float* x = w + b * 32;
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i)
            if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); mx = x[i]; }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t* p = out + b * 18;
        wr_h(p, ora_f2h(d));
        for (int i = 0; i < 16; ++i) {
            const int n0 = clampi((int)(x[2 * i] * id + 8.5f), 0, 15);
            const int n1 = clampi((int)(x[2 * i + 1] * id + 8.5f), 0, 15);
            p[2 + i] = (uint8_t)(n0 | (n1 << 4));
        }
    }
}

void ora_quantize_q4k(const float* w, size_t nblk, uint8_t* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const float* x = w + b * 256;
        float scl[8], mns[8], maxs = 0.0f, maxm = 0.0f;
        for (int s = 0; s < 8; ++s) {
            const int base = 64 * (s & 3) + 32 * (s >> 2);
            float mn = 0.0f, mx = -3.0e38f;
            for (int l = 0; l < 32; ++l) { mn = fminf(mn, x[base + l]); mx = fmaxf(mx, x[base + l]); }
            mns[s] = -mn;
            scl[s] = (mx - mn) / 15.0f;
            maxs = fmaxf(maxs, scl[s]);
            maxm = fmaxf(maxm, mns[s]);
        }
        const float d = maxs / 63.0f, dmin = maxm / 63.0f;
        const uint16_t dh = ora_f2h(d), dmh = ora_f2h(dmin);
        const float dq = ora_h2f(dh), dmq = ora_h2f(dmh);
        int sc[8], m[8];
        for (int s = 0; s < 8; ++s) {
            sc[s] = clampi(d > 0.0f ? (int)roundf(scl[s] / d) : 0, 0, 63);
            m[s] = clampi(dmin > 0.0f ? (int)roundf(mns[s] / dmin) : 0, 0, 63);
        }
        uint8_t* p = out + b * 144;
        wr_h(p, dh);
        wr_h(p + 2, dmh);
        uint8_t* S = p + 4;
        for (int j = 0; j < 4; ++j) {
            S[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            S[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            S[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t* qs = p + 16;
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 32; ++l) {
                int qq[2];
                for (int hi = 0; hi < 2; ++hi) {
                    const int s = j + 4 * hi;
                    const float ds = dq * (float)sc[s], ms = dmq * (float)m[s];
                    const int q = ds > 0.0f ? (int)roundf((x[64 * j + 32 * hi + l] + ms) / ds) : 0;
                    qq[hi] = clampi(q, 0, 15);
                }
                qs[32 * j + l] = (uint8_t)(qq[0] | (qq[1] << 4));
            }
    }
}

void ora_quantize_q6k(const float* w, size_t nblk, uint8_t* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const float* x = w + b * 256;
        float scl[8], dmax = 0.0f;
        for (int g = 0; g < 8; ++g) {
            const int base = 128 * (g >> 2) + 32 * (g & 3);
            float amax = 0.0f, mx = 0.0f;
            for (int l = 0; l < 32; ++l)
                if (fabsf(x[base + l]) > amax) { amax = fabsf(x[base + l]); mx = x[base + l]; }
            scl[g] = mx / -32.0f;
            dmax = fmaxf(dmax, fabsf(scl[g]));
        }
        const float d = dmax / 127.0f;
        const uint16_t dh = ora_f2h(d);
        const float dq = ora_h2f(dh);
        int sc[8], q[256];
        for (int g = 0; g < 8; ++g) sc[g] = clampi(d > 0.0f ? (int)roundf(scl[g] / d) : 0, -127, 127);
        for (int g = 0; g < 8; ++g) {
            const int base = 128 * (g >> 2) + 32 * (g & 3);
            const float ds = dq * (float)sc[g];
            for (int l = 0; l < 32; ++l) {
                const int v = ds != 0.0f ? (int)roundf(x[base + l] / ds) + 32 : 32;
                q[base + l] = clampi(v, 0, 63);
            }
        }
        uint8_t* p = out + b * 210;
        uint8_t* ql = p;
        uint8_t* qh = p + 128;
        for (int h = 0; h < 256; h += 128)
            for (int l = 0; l < 32; ++l) {
                const int q1 = q[h + l], q2 = q[h + l + 32], q3 = q[h + l + 64], q4 = q[h + l + 96];
                ql[h / 2 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
                ql[h / 2 + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
                qh[h / 4 + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        for (int g = 0; g < 8; ++g) {
            const int slot = 8 * (g >> 2) + 2 * (g & 3);
            p[192 + slot] = (uint8_t)(int8_t)sc[g];
            p[192 + slot + 1] = 0x5A;
        }
        wr_h(p + 208, dh);
    }
}

/* Test-data quantisers for the 5-bit formats (not in the reference, which
 * only reads such files): Q5_0 d = x[amax]/−16, q = clamp(x/d + 16.5, 0, 31)
 * in the reference's layout; Q5_K as the Q4_K quantiser with 31 levels and
 * the reference's high-bit order (bit e%8 of qh[e/8]). */
void ora_quantize_q5_0(const float* w, size_t nblk, uint8_t* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const float* x = w + b * 32;
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i)
            if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); mx = x[i]; }
        const float d = mx / -16.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t* p = out + b * 22;
        wr_h(p, ora_f2h(d));
        uint32_t qh = 0;
        for (int j = 0; j < 16; ++j) {
            const int q0 = clampi((int)(x[j] * id + 16.5f), 0, 31);
            const int q1 = clampi((int)(x[j + 16] * id + 16.5f), 0, 31);
            p[6 + j] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
            qh |= (uint32_t)(q0 >> 4) << j;
            qh |= (uint32_t)(q1 >> 4) << (j + 16);
        }
        for (int i = 0; i < 4; ++i) p[2 + i] = (uint8_t)(qh >> (8 * i));
    }
}

void ora_quantize_q5k(const float* w, size_t nblk, uint8_t* out) {
    for (size_t b = 0; b < nblk; ++b) {
        const float* x = w + b * 256;
        float scl[8], mns[8], maxs = 0.0f, maxm = 0.0f;
        for (int s = 0; s < 8; ++s) {
            const int base = 64 * (s & 3) + 32 * (s >> 2);
            float mn = 0.0f, mx = -3.0e38f;
            for (int l = 0; l < 32; ++l) { mn = fminf(mn, x[base + l]); mx = fmaxf(mx, x[base + l]); }
            mns[s] = -mn;
            scl[s] = (mx - mn) / 31.0f;
            maxs = fmaxf(maxs, scl[s]);
            maxm = fmaxf(maxm, mns[s]);
        }
        const float d = maxs / 63.0f, dmin = maxm / 63.0f;
        const uint16_t dh = ora_f2h(d), dmh = ora_f2h(dmin);
        const float dq = ora_h2f(dh), dmq = ora_h2f(dmh);
        int sc[8], m[8];
        for (int s = 0; s < 8; ++s) {
            sc[s] = clampi(d > 0.0f ? (int)roundf(scl[s] / d) : 0, 0, 63);
            m[s] = clampi(dmin > 0.0f ? (int)roundf(mns[s] / dmin) : 0, 0, 63);
        }
        uint8_t* p = out + b * 176;
        memset(p, 0, 176);
        wr_h(p, dh);
        wr_h(p + 2, dmh);
        uint8_t* S = p + 4;
        for (int j = 0; j < 4; ++j) {
            S[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            S[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
            S[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
        }
        uint8_t* qh = p + 16;
        uint8_t* qs = p + 48;
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 32; ++l) {
                int qq[2];
                for (int hi = 0; hi < 2; ++hi) {
                    const int s = j + 4 * hi, e = 64 * j + 32 * hi + l;
                    const float ds = dq * (float)sc[s], ms = dmq * (float)m[s];
                    const int q = ds > 0.0f ? (int)roundf((x[e] + ms) / ds) : 0;
                    qq[hi] = clampi(q, 0, 31);
                    qh[e / 8] |= (uint8_t)((qq[hi] >> 4) << (e % 8));
                }
                qs[32 * j + l] = (uint8_t)((qq[0] & 15) | ((qq[1] & 15) << 4));
            }
    }
}

/* ───────────────── re-layout to ggml (test data) ───────────────── */

static void pack_scales_k4(const int sc[8], const int m[8], uint8_t* S) {
    for (int j = 0; j < 4; ++j) {
        S[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        S[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        S[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
}
/* reference sub-block j (chunk j low) = ggml 2j, reference j + 4 (chunk j
 * high) = ggml 2j + 1 */
static void relayout_k_scales(const uint8_t* S_ref, uint8_t* S_g) {
    int sc[8], m[8];
    for (int j = 0; j < 4; ++j) {
        uint8_t a, b;
        scale_min_k4(j, S_ref, &a, &b);
        sc[2 * j] = a; m[2 * j] = b;
        scale_min_k4(j + 4, S_ref, &a, &b);
        sc[2 * j + 1] = a; m[2 * j + 1] = b;
    }
    pack_scales_k4(sc, m, S_g);
}

void ora_relayout_to_ggml(int fmt, const uint8_t* in, size_t nblk, uint8_t* out) {
    for (size_t b = 0; b < nblk; ++b) {
        if (fmt == ORA_Q4_0) {
            const uint8_t* r = in + b * 18;
            uint8_t* g = out + b * 18;
            int c[32];
            for (int i = 0; i < 16; ++i) { c[2 * i] = r[2 + i] & 15; c[2 * i + 1] = r[2 + i] >> 4; }
            g[0] = r[0]; g[1] = r[1];
            for (int j = 0; j < 16; ++j) g[2 + j] = (uint8_t)(c[j] | (c[j + 16] << 4));
        } else if (fmt == ORA_Q4K) {
            const uint8_t* r = in + b * 144;
            uint8_t* g = out + b * 144;
            memcpy(g, r, 144);
            relayout_k_scales(r + 4, g + 4);
        } else if (fmt == ORA_Q5K) {
            const uint8_t* r = in + b * 176;
            uint8_t* g = out + b * 176;
            memcpy(g, r, 176);
            relayout_k_scales(r + 4, g + 4);
            uint8_t qh[32];
            memset(qh, 0, 32);
            for (int e = 0; e < 256; ++e) {
                const int bit = (r[16 + e / 8] >> (e % 8)) & 1;
                const int j = e / 64, hi = (e / 32) & 1, l = e % 32;
                qh[l] |= (uint8_t)(bit << (2 * j + hi));
            }
            memcpy(g + 16, qh, 32);
        }
    }
}

void ora_quantize_q4_0g(const float* w, size_t nblk, uint8_t* out) {
    ora_quantize_q4_0(w, nblk, out);
    uint8_t tmp[18];
    for (size_t b = 0; b < nblk; ++b) {
        ora_relayout_to_ggml(ORA_Q4_0, out + b * 18, 1, tmp);
        memcpy(out + b * 18, tmp, 18);
    }
}
void ora_quantize_q4kg(const float* w, size_t nblk, uint8_t* out) {
    ora_quantize_q4k(w, nblk, out);
    uint8_t tmp[144];
    for (size_t b = 0; b < nblk; ++b) {
        ora_relayout_to_ggml(ORA_Q4K, out + b * 144, 1, tmp);
        memcpy(out + b * 144, tmp, 144);
    }
}
void ora_quantize_q5kg(const float* w, size_t nblk, uint8_t* out) {
    ora_quantize_q5k(w, nblk, out);
    uint8_t tmp[176];
    for (size_t b = 0; b < nblk; ++b) {
        ora_relayout_to_ggml(ORA_Q5K, out + b * 176, 1, tmp);
        memcpy(out + b * 176, tmp, 176);
    }
}
void ora_quantize_q6kg(const float* w, size_t nblk, uint8_t* out) {
    ora_quantize_q6k(w, nblk, out);
    for (size_t b = 0; b < nblk; ++b) {
        int8_t* sc = (int8_t*)(out + b * 210 + 192);
        for (int k = 0; k < 8; ++k) {
            const int v = sc[2 * k] + (int)((b * 5 + (size_t)k * 3) % 5) - 2;
            sc[2 * k + 1] = (int8_t)clampi(v, -127, 127);
        }
    }
}

/* Seeded weights as the device generators build them (rt_synth_*): element i
 * of the stream is w_i = stdv·N_i (f32 product), quantised per block with the
 * quantisers above. */
void ora_synth_weights(int fmt, uint64_t seed, float stdv, size_t nblk, uint8_t* out) {
    const size_t el = ora_block_elems(fmt), by = ora_block_bytes(fmt);
#pragma omp parallel
    {
        float* w = (float*)malloc(el * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t b = 0; b < (int64_t)nblk; ++b) {
            for (size_t i = 0; i < el; ++i) w[i] = stdv * ora_synth_normal(seed, (uint64_t)b * el + i);
            switch (fmt) {
            case ORA_Q8_0: ora_quantize_q8_0(w, 1, out + b * by); break;
            case ORA_Q4_0: ora_quantize_q4_0(w, 1, out + b * by); break;
            case ORA_Q4K: ora_quantize_q4k(w, 1, out + b * by); break;
            case ORA_Q6K: ora_quantize_q6k(w, 1, out + b * by); break;
            case ORA_Q5_0: ora_quantize_q5_0(w, 1, out + b * by); break;
            case ORA_Q5K: ora_quantize_q5k(w, 1, out + b * by); break;
            default: memset(out + b * by, 0, by); break;
            }
        }
        free(w);
    }
}

/* ───────────────── whole decode step, f32 (CPU baseline) ───────────────── */

static void rms_norm_f32(const float* x, const float* g, float eps, size_t n, float* y) {
    float ss = 0.0f; /* cpu_rms_norm: f32 sum of squares, then /n + eps, sqrt */
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const float rms = sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; ++i) y[i] = x[i] / rms * g[i];
}

static void rope_f32(float* v, size_t heads, size_t hd, uint32_t pos, float theta) {
    const size_t half = hd / 2;
    for (size_t d = 0; d < half; ++d) {
        const float freq = 1.0f / powf(theta, (float)(2 * d) / (float)hd);
        const float ang = (float)pos * freq, c = cosf(ang), s = sinf(ang);
        for (size_t h = 0; h < heads; ++h) {
            float* x = v + h * hd;
            const float r = x[d], i = x[d + half];
            x[d] = r * c - i * s;
            x[d + half] = r * s + i * c;
        }
    }
}

uint32_t ora_decode_step_ref_f32(const ora_model_t* m, uint32_t token, uint32_t pos,
                                 float* logits, int threads) {
    const size_t h = m->hidden, hd = m->head_dim, H = m->heads, KVH = m->kv_heads;
    const size_t qd = H * hd, kvd = KVH * hd, ff = m->ff, S = m->max_seq, kv_len = (size_t)pos + 1;
    float* x = (float*)malloc(h * sizeof(float));
    float* xn = (float*)malloc((h > ff ? h : ff) * sizeof(float));
    float* q = (float*)malloc(qd * sizeof(float));
    float* k = (float*)malloc(kvd * sizeof(float));
    float* v = (float*)malloc(kvd * sizeof(float));
    float* att = (float*)malloc(qd * sizeof(float));
    float* g = (float*)malloc(ff * sizeof(float));
    float* u = (float*)malloc(ff * sizeof(float));
    float* t = (float*)malloc((h > ff ? h : ff) * sizeof(float));
    float* sc = (float*)malloc(kv_len * sizeof(float));
    {
        const size_t nb = h / ora_block_elems(m->f_embd);
        ora_dequant(m->f_embd, m->embd + (size_t)token * nb * ora_block_bytes(m->f_embd), nb, x);
    }
    const float scale = 1.0f / sqrtf((float)hd);
    for (uint32_t li = 0; li < m->layers; ++li) {
        const ora_layer_t* L = &m->layer[li];
        rms_norm_f32(x, L->attn_norm, m->eps, h, xn);
        ora_gemv_ref_f32(L->fq, L->wq, xn, qd, h, q, threads);
        ora_gemv_ref_f32(L->fk, L->wk, xn, kvd, h, k, threads);
        ora_gemv_ref_f32(L->fv, L->wv, xn, kvd, h, v, threads);
        for (size_t i = 0; i < qd; ++i) q[i] += ora_h2f(L->bq[i]);
        for (size_t i = 0; i < kvd; ++i) { k[i] += ora_h2f(L->bk[i]); v[i] += ora_h2f(L->bv[i]); }
        rope_f32(q, H, hd, pos, m->theta);
        rope_f32(k, KVH, hd, pos, m->theta);
        for (size_t j = 0; j < KVH; ++j) {
            memcpy(L->kc + (j * S + pos) * hd, k + j * hd, hd * sizeof(float));
            memcpy(L->vc + (j * S + pos) * hd, v + j * hd, hd * sizeof(float));
        }
        for (size_t hh = 0; hh < H; ++hh) {
            const size_t kvh = hh / (H / KVH);
            const float* qh = q + hh * hd;
            float mx = -INFINITY;
            for (size_t j = 0; j < kv_len; ++j) {
                const float* kr = L->kc + (kvh * S + j) * hd;
                float dot = 0.0f;
                for (size_t d = 0; d < hd; ++d) dot += qh[d] * kr[d];
                sc[j] = dot * scale;
                mx = fmaxf(mx, sc[j]);
            }
            float sum = 0.0f;
            for (size_t j = 0; j < kv_len; ++j) { sc[j] = expf(sc[j] - mx); sum += sc[j]; }
            float* o = att + hh * hd;
            for (size_t d = 0; d < hd; ++d) o[d] = 0.0f;
            for (size_t j = 0; j < kv_len; ++j) {
                const float p = sc[j] / sum;
                const float* vr = L->vc + (kvh * S + j) * hd;
                for (size_t d = 0; d < hd; ++d) o[d] += p * vr[d];
            }
        }
        ora_gemv_ref_f32(L->fo, L->wo, att, h, qd, t, threads);
        for (size_t i = 0; i < h; ++i) x[i] += t[i];
        rms_norm_f32(x, L->ffn_norm, m->eps, h, xn);
        ora_gemv_ref_f32(L->fg, L->wg, xn, ff, h, g, threads);
        ora_gemv_ref_f32(L->fu, L->wu, xn, ff, h, u, threads);
        for (size_t i = 0; i < ff; ++i) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
        ora_gemv_ref_f32(L->fd, L->wd, g, h, ff, t, threads);
        for (size_t i = 0; i < h; ++i) x[i] += t[i];
    }
    rms_norm_f32(x, m->final_norm, m->eps, h, xn);
    ora_gemv_ref_f32(m->f_lm, m->lm_head, xn, m->vocab, h, logits, threads);
    const uint32_t tok = ora_argmax_f32(logits, m->vocab);
    free(x); free(xn); free(q); free(k); free(v); free(att); free(g); free(u); free(t); free(sc);
    return tok;
}
