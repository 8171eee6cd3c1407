// rt_gemv.h — M=1 quantized GEMV, fused QKV(+bias) and fused gate+up+SiLU
// kernel bodies for gfx950 (instantiated by the kg_*.hip files).
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
#pragma once
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
    uint32_t ksw;        // matrix-core path: waves sharing one row-quad group (K split)
    uint32_t x_rec;      // x already holds activation records (built by k_act_limbs)
    const float* gamma;  // non-null: RMSNorm(x)·γ is staged instead of x (f32 x, whole K)
    float eps;
    uint32_t xb_chunk;   // activation records staged per LDS pass (multiple of 8)
    uint64_t row_bytes;
    // matrix-core path, K split over workgroups: chunk ks of kc_units units
    // goes to workgroups ≡ ks (mod ksplit); partial sums meet in `part`
    uint32_t ksplit;     // 1: whole K per workgroup
    uint32_t kc_units;
    float* part;         // [ksplit][nvrows]
    uint32_t* counters;  // [tiles] arrival counters (reset by the last arriver)
    uint32_t cstride;    // u32 slots between two tiles' counters (own cache lines)
    // x given as split-attention partials (XT = AttnX): x = o[H][nsp][hd],
    // xml = (m, l)[H][nsp]; staging merges them as the attention kernel does
    const float* xml;
    uint32_t xnsp, xhd;
    uint32_t ls_rs;      // LDS-streamed body: LDS bytes between two rows of a slot
    uint32_t ls_res;     // LDS-streamed body: result slots per wave (items)
    uint32_t ls_xcd;     // LDS-streamed body: neighbouring quads to workgroups of one XCD
    // matrix-core body in a two-part launch: this part owns workgroups
    // [blk0, blk0 + nblk) (nblk = 0: the whole grid)
    uint32_t blk0, nblk;
    // activation rows of a multi-row launch (the _x8 kernels; 0 otherwise):
    // x holds their limb records row after row, output / residual row m of
    // a matrix starts m rows of that matrix's length further on
    uint32_t nx;
    // Σy² of the outputs, one float per row quad, for the next launch's
    // RMSNorm (null: not written) ...
    float* ssq_out;
    // ... and the same as input: Σx² of x as ssq_n partial sums (null: the
    // staging reduces x itself)
    const float* ssq_in;
    uint32_t ssq_n;
};

// Σ over the four rows of a row quad of the stored outputs' squares, written
// to ssq_out[quad] by the quad's first lane (lanes 4b..4b+3 hold rows 0..3;
// rows past the launch count 0).
RT_DEV void quad_ssq_store(float* ssq_out, uint32_t quad, float y, bool valid, uint32_t q) {
    float sq = valid ? y * y : 0.0f;
    sq += dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(sq);
    sq += dpp_f<DPP_QUAD_PERM(2, 3, 0, 1)>(sq);
    if (q == 0) ssq_out[quad] = sq;
}

// Tiles one workgroup may own in a K-split launch (the host keeps the grid's
// rounds below this).
constexpr uint32_t kMaxSplitTiles = 256;

// Items (weight loads of one step) in flight per wave in the matrix-core
// body, for one and two row quads per wave.
#define GEMV_PF1 2
#define GEMV_PF2 2

enum Epi : int {
    EPI_F32 = 0,      // y = v                     (f32 out)
    EPI_F32_ADD = 1,  // y = v + res               (f32 out, f32 residual)
    EPI_F16 = 2,      // y = half(v)
    EPI_F16_ADD = 3,  // y = half(v + float(res16))
    EPI_QKV = 4,      // 3 matrices, no bias
    EPI_QKV_BIAS = 5, // 3 matrices, + float(bias16)
    EPI_FFN = 6,      // act = silu(gate)·up, rows interleaved
    // EPI_COH | e: the same epilogue inside a persistent kernel, whose
    // activations are produced and consumed by other workgroups of the same
    // launch: the residual is read and the outputs are written at device
    // scope (dev_load / dev_store), so no cache holds a stale copy
    EPI_COH = 16,
};
constexpr int epi_base(int e) { return e & 15; }
constexpr bool epi_coh(int e) { return (e & EPI_COH) != 0; }
// f32 store of an epilogue output (device scope inside a persistent kernel)
template <int EPI, typename T>
RT_DEV void out_store(T* p, T v) {
    if constexpr (epi_coh(EPI)) dev_store(p, v); else *p = v;
}
template <int EPI, typename T>
RT_DEV T aux_load(const T* p) {
    if constexpr (epi_coh(EPI)) return dev_load(p); else return *p;
}

template <int EPI>
RT_DEV void vrow_map(const GemvArgs& a, uint32_t vr, uint32_t& mat, uint32_t& r) {
    if (epi_base(EPI) == EPI_FFN) {
        mat = vr & 1;
        r = vr >> 1;
    } else if (epi_base(EPI) == EPI_QKV || epi_base(EPI) == EPI_QKV_BIAS) {
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

// Matrix selection by value (select chains): indexing the by-value argument
// arrays with a runtime index would move the whole argument block to scratch.
template <typename T>
RT_DEV T pick3(T a0, T a1, T a2, uint32_t m) {
    return m == 0 ? a0 : (m == 1 ? a1 : a2);
}
RT_DEV const uint8_t* mat_w(const GemvArgs& a, uint32_t m) { return pick3(a.w[0], a.w[1], a.w[2], m); }
RT_DEV void* mat_out(const GemvArgs& a, uint32_t m) { return pick3(a.out[0], a.out[1], a.out[2], m); }
RT_DEV const void* mat_aux(const GemvArgs& a, uint32_t m) {
    return pick3(a.aux[0], a.aux[1], a.aux[2], m);
}

RT_DEV float silu_ref(float g) {
    // x / (1 + exp(-x))  (fused_ffn.metal:24-26; dispatch.rs:1684-1686)
    return g / (1.0f + expf(-g));
}

// Output length of matrix `mat` (the distance between two activation rows'
// outputs in a multi-row launch).
template <int EPI>
RT_DEV uint32_t out_len(const GemvArgs& a, uint32_t mat) {
    if (epi_base(EPI) == EPI_FFN) return a.nvrows >> 1;
    if (epi_base(EPI) == EPI_QKV || epi_base(EPI) == EPI_QKV_BIAS) return pick3(a.n[0], a.n[1], a.n[2], mat);
    return a.nvrows;
}

// Epilogue operand (residual or bias) of virtual row vr (activation row m),
// loaded early so the epilogue does not wait on a dependent load.
template <int EPI>
RT_DEV float load_aux(const GemvArgs& a, uint32_t vr, uint32_t m = 0) {
    uint32_t mat, r;
    vrow_map<EPI>(a, vr, mat, r);
    if (epi_base(EPI) == EPI_F32_ADD) return aux_load<EPI>((const float*)a.aux[0] + r + (size_t)m * a.nvrows);
    if (epi_base(EPI) == EPI_F16_ADD) return h2f(((const uint16_t*)a.aux[0])[r]);
    if (epi_base(EPI) == EPI_QKV_BIAS) return h2f(((const uint16_t*)mat_aux(a, mat))[r]);
    return 0.0f;
}
template <int EPI>
constexpr bool has_aux() {
    return epi_base(EPI) == EPI_F32_ADD || epi_base(EPI) == EPI_F16_ADD || epi_base(EPI) == EPI_QKV_BIAS;
}
// Stores v (+ the preloaded epilogue operand) for virtual row vr.  With an
// output aliasing the residual, the value was read by this same lane first.
template <int EPI>
RT_DEV void store_row(const GemvArgs& a, uint32_t vr, float v, uint32_t m);
// (m: activation row of a multi-row launch)
template <int EPI>
RT_DEV void store_row_pre(const GemvArgs& a, uint32_t vr, float v, float aux, uint32_t m = 0) {
    uint32_t mat, r;
    vrow_map<EPI>(a, vr, mat, r);
    const size_t ro = (size_t)m * out_len<EPI>(a, mat);
    if (epi_base(EPI) == EPI_F32_ADD) {
        out_store<EPI>((float*)a.out[0] + ro + r, v + aux);
    } else if (epi_base(EPI) == EPI_F16_ADD) {
        ((uint16_t*)a.out[0])[r] = f2h(v + aux);
    } else if (epi_base(EPI) == EPI_QKV_BIAS) {
        out_store<EPI>((float*)mat_out(a, mat) + ro + r, v + aux);
    } else {
        store_row<EPI>(a, vr, v, m);
    }
}

template <int EPI>
RT_DEV void store_row(const GemvArgs& a, uint32_t vr, float v, uint32_t m) {
    uint32_t mat, r;
    vrow_map<EPI>(a, vr, mat, r);
    r += (uint32_t)(m * out_len<EPI>(a, mat));  // multi-row launch: row m's outputs
    if (epi_base(EPI) == EPI_F32) {
        out_store<EPI>((float*)a.out[0] + r, v);
    } else if (epi_base(EPI) == EPI_F32_ADD) {
        // read residual[r] then write y[r] in the same lane: y may alias res
        const float res = aux_load<EPI>((const float*)a.aux[0] + r);
        out_store<EPI>((float*)a.out[0] + r, v + res);
    } else if (epi_base(EPI) == EPI_F16) {
        ((uint16_t*)a.out[0])[r] = f2h(v);
    } else if (epi_base(EPI) == EPI_F16_ADD) {
        const float res = h2f(((const uint16_t*)a.aux[0])[r]);
        ((uint16_t*)a.out[0])[r] = f2h(v + res);
    } else if (epi_base(EPI) == EPI_QKV) {
        ((float*)mat_out(a, mat))[r] = v;
    } else if (epi_base(EPI) == EPI_QKV_BIAS) {
        out_store<EPI>((float*)mat_out(a, mat) + r, v + h2f(((const uint16_t*)mat_aux(a, mat))[r]));
    }
}

// Reduction over a row group (TL lanes, possibly several waves) followed by
// the epilogue in the group's first lane.
template <int EPI, int RPL>
RT_DEV void finish_rows(const GemvArgs& a, float* red, uint32_t tid, uint32_t TL, uint32_t grp,
                        uint32_t kl, uint32_t vr0, float acc[RPL]) {
#pragma unroll
    for (int i = 0; i < RPL; ++i) acc[i] = group_sum(acc[i], (int)min(TL, 64u));
    if (TL > 64) {
        // the row group spans TL/64 waves: combine their sums through LDS in a
        // fixed order (deterministic)
        const uint32_t wave = tid >> 6, wpr = TL / 64;
        if ((tid & 63) == 0) {
#pragma unroll
            for (int i = 0; i < RPL; ++i) red[wave * RPL + i] = acc[i];
        }
        __syncthreads();
        if (kl == 0) {
#pragma unroll
            for (int i = 0; i < RPL; ++i) {
                float t = 0.0f;
                for (uint32_t w = 0; w < wpr; ++w) t += red[(grp * wpr + w) * RPL + i];
                acc[i] = t;
            }
        }
        __syncthreads();
    }
    if (kl == 0) {
        if (epi_base(EPI) == EPI_FFN) {
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
                if (vr0 + i < a.nvrows) store_row<EPI>(a, vr0 + i, acc[i], 0);
            }
        }
    }
}

template <int EPI, int RPL>
RT_DEV void tile_rows(const GemvArgs& a, uint32_t vr0, const uint8_t* rowp[RPL]) {
#pragma unroll
    for (int i = 0; i < RPL; ++i) {
        uint32_t vr = vr0 + i;
        if (vr >= a.nvrows) vr = a.nvrows - 1;  // clamp loads; the store is skipped
        uint32_t mat, r;
        vrow_map<EPI>(a, vr, mat, r);
        rowp[i] = mat_w(a, mat) + (size_t)r * a.row_bytes;
    }
}

// Whole-K path (all activation records fit in LDS).  Each lane walks a flat
// sequence of (tile, step) items; a step is UNR units of RPL rows.  The weight
// loads of item n+1 are issued before item n is computed (two register
// buffers), and the loads of the first item are issued before the activation
// staging, so the staging latency hides behind HBM latency.
template <class F, int EPI, typename XT, int RPL, int UNR>
RT_DEV void gemv_body_pipelined(const GemvArgs& a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    XRec* xs = (XRec*)smem;
    float* red = (float*)(smem + (size_t)a.xb_chunk * sizeof(XRec));
    const uint32_t tid = threadIdx.x;
    const uint32_t TL = a.lpr;
    const uint32_t grp = tid / TL, kl = tid % TL;
    const uint32_t vrows_per_wg = (wg_threads() / TL) * RPL;
    const uint32_t nxb = a.K / 32;
    const uint32_t ntiles = (a.nvrows + vrows_per_wg - 1) / vrows_per_wg;
    const uint32_t units = a.K / F::UNIT_EL;
    const uint32_t nsteps = (units + UNR * TL - 1) / (UNR * TL);
    const uint32_t my_tiles =
        blockIdx.x < ntiles ? (ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    const uint32_t nitems = my_tiles * nsteps;

    typename F::Raw buf[2][UNR][RPL];
    const uint8_t* rowp[RPL];

    auto issue = [&](uint32_t item, typename F::Raw (&dst)[UNR][RPL]) {
        const uint32_t tile = blockIdx.x + (item / nsteps) * gridDim.x;
        const uint32_t step = item % nsteps;
        const uint8_t* rp[RPL];
        tile_rows<EPI, RPL>(a, tile * vrows_per_wg + grp * RPL, rp);
#pragma unroll
        for (int s = 0; s < UNR; ++s) {
            const uint32_t uu = kl + (step * UNR + s) * TL;
            if (uu < units) {
#pragma unroll
                for (int i = 0; i < RPL; ++i) F::load(rp[i], uu, dst[s][i]);
            }
        }
    };

    if (nitems > 0) issue(0, buf[0]);
    stage_x<XT, F::Q40PERM>(a.x, a.x_rec != 0, 0, nxb, xs, a.gamma, a.eps);
    __syncthreads();
    if (nitems == 0) return;
    (void)rowp;

    float acc[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) acc[i] = 0.0f;

    // two-deep pipeline, unrolled by two so the buffers are addressed statically
    for (uint32_t it = 0; it < nitems; it += 2) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t item = it + half;
            if (item < nitems) {
                if (item + 1 < nitems) issue(item + 1, buf[half ^ 1]);
                const uint32_t step = item % nsteps;
#pragma unroll
                for (int s = 0; s < UNR; ++s) {
                    const uint32_t uu = kl + (step * UNR + s) * TL;
                    if (uu < units) {
                        typename F::XU xu;
                        F::load_x(xs, uu, xu);
#pragma unroll
                        for (int i = 0; i < RPL; ++i) acc[i] += F::dot(buf[half][s][i], xu);
                    }
                }
                if (step == nsteps - 1) {
                    const uint32_t tile = blockIdx.x + (item / nsteps) * gridDim.x;
                    finish_rows<EPI, RPL>(a, red, tid, TL, grp, kl,
                                          tile * vrows_per_wg + grp * RPL, acc);
#pragma unroll
                    for (int i = 0; i < RPL; ++i) acc[i] = 0.0f;
                }
            }
        }
    }
}

// Long-K path: the activation records are staged in chunks, once per tile.
template <class F, int EPI, typename XT, int RPL, int UNR>
RT_DEV void gemv_body_chunked(const GemvArgs& a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    XRec* xs = (XRec*)smem;
    float* red = (float*)(smem + (size_t)a.xb_chunk * sizeof(XRec));
    const uint32_t tid = threadIdx.x;
    const uint32_t TL = a.lpr;
    const uint32_t grp = tid / TL, kl = tid % TL;
    const uint32_t vrows_per_wg = (wg_threads() / TL) * RPL;
    const uint32_t nxb = a.K / 32;
    const uint32_t ntiles = (a.nvrows + vrows_per_wg - 1) / vrows_per_wg;

    for (uint32_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const uint32_t vr0 = tile * vrows_per_wg + grp * RPL;
        const uint8_t* rowp[RPL];
        tile_rows<EPI, RPL>(a, vr0, rowp);
        float acc[RPL];
#pragma unroll
        for (int i = 0; i < RPL; ++i) acc[i] = 0.0f;
        for (uint32_t xc = 0; xc < nxb; xc += a.xb_chunk) {
            const uint32_t nx = min(a.xb_chunk, nxb - xc);
            __syncthreads();
            stage_x<XT, F::Q40PERM>(a.x, a.x_rec != 0, xc, nx, xs);
            __syncthreads();
            const uint32_t units = nx * 32 / F::UNIT_EL;
            const uint32_t u0 = xc * 32 / F::UNIT_EL;
            for (uint32_t ub = kl; ub < units; ub += UNR * TL) {
                typename F::Raw raw[UNR][RPL];
#pragma unroll
                for (int s = 0; s < UNR; ++s) {
                    const uint32_t uu = ub + s * TL;
                    if (uu < units) {
#pragma unroll
                        for (int i = 0; i < RPL; ++i) F::load(rowp[i], u0 + uu, raw[s][i]);
                    }
                }
#pragma unroll
                for (int s = 0; s < UNR; ++s) {
                    const uint32_t uu = ub + s * TL;
                    if (uu < units) {
                        typename F::XU xu;
                        F::load_x(xs, uu, xu);
#pragma unroll
                        for (int i = 0; i < RPL; ++i) acc[i] += F::dot(raw[s][i], xu);
                    }
                }
            }
        }
        finish_rows<EPI, RPL>(a, red, tid, TL, grp, kl, vr0, acc);
    }
}

// One activation row staged by one wave (multi-row launches with K ≤ 1024):
// lane l takes slices l, l + 64, ... (≤ XSTAGE_UNR rounds), loads them (and
// γ) before the caller issues its weight loads, then RMS-normalises the row
// with a wave-wide sum (x̂ = x · rsqrt(Σx²/K + eps) · γ, products rounded in
// f32 as stage_x_convert rounds them) and writes its limb records.
RT_DEV void stage_row_load(const float* __restrict__ x, const float* __restrict__ gamma,
                           uint32_t nxb, XPre& p) {
    const uint32_t total = nxb * 8, lane = threadIdx.x & 63;
#pragma unroll
    for (int s = 0; s < XSTAGE_UNR; ++s) {
        const uint32_t t = lane + 64 * s;
        if (64 * s >= total) break;  // uniform
        const uint32_t i = t < total ? (t >> 3) * 32 + (t & 7) * 4 : 0;
        const f32x4 v = *(const f32x4*)(x + i);
        p.v[s][0] = v.x; p.v[s][1] = v.y; p.v[s][2] = v.z; p.v[s][3] = v.w;
        if (gamma) {
            const f32x4 g = *(const f32x4*)(gamma + i);
            p.g[s][0] = g.x; p.g[s][1] = g.y; p.g[s][2] = g.z; p.g[s][3] = g.w;
        }
    }
}
RT_DEV void stage_row_convert(XPre& p, const float* gamma, float eps, uint32_t nxb,
                              XRec* __restrict__ recs) {
    const uint32_t total = nxb * 8, lane = threadIdx.x & 63;
    if (gamma) {
        float ss = 0.0f;
#pragma unroll
        for (int s = 0; s < XSTAGE_UNR; ++s) {
            if (64 * s >= total) break;
            const float sq = p.v[s][0] * p.v[s][0] + p.v[s][1] * p.v[s][1] +
                             p.v[s][2] * p.v[s][2] + p.v[s][3] * p.v[s][3];
            ss += lane + 64 * s < total ? sq : 0.0f;
        }
        ss = group_sum(ss, 64);
        const float rms = rsqrtf(ss / (float)(nxb * 32) + eps);
#pragma unroll
        for (int s = 0; s < XSTAGE_UNR; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i) p.v[s][i] = p.v[s][i] * rms * p.g[s][i];
    }
#pragma unroll
    for (int s = 0; s < XSTAGE_UNR; ++s) {
        const uint32_t t = lane + 64 * s;
        if (64 * s >= total) break;
        if (t < total) limb_slice<false>(p.v[s], t & 7, recs + (t >> 3));  // whole 8-lane groups
    }
}

// Matrix-core path (whole K in LDS).  Lane 4·slot + q works on row q of the
// wave's current row quad and on unit `slot` (+16 per step) of that row, so
// the 16 lanes of a row read 16 consecutive units (coalesced) and the four
// lanes of a quad feed one 4×4×4 block of v_mfma_i32_4x4x4i8 (rt_formats.h).
// Each lane walks a flat sequence of (tile, step) items and issues the loads
// of item n+1 before computing item n; the first item's loads are issued
// before the activation staging.
// NX > 1: up to NX activation rows (a.nx of them) against each weight row:
// x holds their limb records (k_act_limbs_rows), every loaded weight unit is
// dotted with each row's records, and each row gets its own epilogue.
template <class F, int EPI, typename XT, int RQ, int PF, class Hook = NoHook, int NX = 1>
RT_DEV void gemv_mq_body(const GemvArgs& a, const Hook& hook = Hook()) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6, nwaves = wg_threads() >> 6;
    const uint32_t q = lane & 3, slot = lane >> 2;
    const uint32_t lq = q < 3 ? q : 2;  // the A row of lane q = 3 is a don't-care
    // K chunk of this workgroup (the whole K when ksplit = 1)
    const uint32_t S = a.ksplit;
    const uint32_t bid = blockIdx.x - a.blk0, gdim = a.nblk ? a.nblk : gridDim.x;
    const uint32_t ks = bid % S, wg = bid / S, nwg = gdim / S;
    const uint32_t cu0 = ks * a.kc_units;  // first unit of the chunk
    const uint32_t units = min(a.K / F::UNIT_EL - cu0, a.kc_units);
    XRec* xs = (XRec*)smem;  // the chunk's records (NX rows: row after row)
    float* red = (float*)(smem + (size_t)NX * (a.kc_units * F::UNIT_EL / 32) * sizeof(XRec));
    const uint32_t nx = NX > 1 ? a.nx : 1;  // activation rows (uniform)
    // ksw waves share one group of RQ row quads and split its K steps
    const uint32_t ksw = a.ksw;
    const uint32_t wgrp = wave / ksw, wk = wave % ksw;
    const uint32_t vrows_per_wg = (nwaves / ksw) * 4 * RQ;
    const uint32_t ntiles = (a.nvrows + vrows_per_wg - 1) / vrows_per_wg;
    const uint32_t nsteps = (units + 15) / 16;
    const uint32_t spw = (nsteps + ksw - 1) / ksw;  // steps per wave per tile
    const uint32_t my_tiles = wg < ntiles ? (ntiles - wg + nwg - 1) / nwg : 0;
    const uint32_t nitems = my_tiles * spw;
    // first virtual row of the wave's rows in the workgroup's tile number t
    auto rows_of = [&](uint32_t t) -> uint32_t { return (wg + t * nwg) * vrows_per_wg + wgrp * 4 * RQ; };

    typename F::Raw buf[PF][RQ];  // PF items in flight per wave
    auto issue = [&](uint32_t item, typename F::Raw (&dst)[RQ]) {
        const uint32_t vb = rows_of(item / spw);
        const uint32_t step = wk + ksw * (item % spw);
        uint32_t u = slot + 16 * step;
        if (u >= units) u = 0;  // clamped: loads stay in bounds, result is discarded
#pragma unroll
        for (int rq = 0; rq < RQ; ++rq) {
            uint32_t vr = vb + 4 * rq + q;
            if (vr >= a.nvrows) vr = a.nvrows - 1;
            uint32_t mat, r;
            vrow_map<EPI>(a, vr, mat, r);
            F::load(mat_w(a, mat) + (size_t)r * a.row_bytes, cu0 + u, dst[rq]);
        }
    };

    float acc[RQ][NX], aux[RQ][NX];
#pragma unroll
    for (int rq = 0; rq < RQ; ++rq)
#pragma unroll
        for (int m = 0; m < NX; ++m) acc[rq][m] = aux[rq][m] = 0.0f;
    // (every lane loads, unconditionally: a load on only some control paths
    // would make the compiler's wait for the x loads a wait for all loads)
    auto load_tile_aux = [&](uint32_t item) {
        // (device-scope operands: only the waves that run the epilogue)
        if (has_aux<EPI>() && (!epi_coh(EPI) || wk == 0)) {
            const uint32_t vb = rows_of(item / spw);
#pragma unroll
            for (int rq = 0; rq < RQ; ++rq) {
                const uint32_t vr = vb + 4 * rq + q;
#pragma unroll
                for (int m = 0; m < NX; ++m)
                    if (m < (int)nx) aux[rq][m] = load_aux<EPI>(a, vr < a.nvrows ? vr : a.nvrows - 1, m);
            }
        }
    };

    // Memory order of the prologue: x (and γ), the first tile's epilogue
    // operand, the weights of the first two items; the conversion of x then
    // waits only for x.
    const uint32_t nxb = units * F::UNIT_EL / 32, xb0 = cu0 * F::UNIT_EL / 32;
    const bool one_pass = !a.x_rec && stage_one_pass(nxb);
    XPre xp;
    XPreAttn xa;
    auto load_x = [&] {
        if constexpr (is_attn_x<XT>()) {
            // (the host launches this form with one slice round, whole K, nsp ≤ 8)
            stage_attn_load<__is_same(XT, AttnXC)>(a.x, a.xml, a.xnsp, a.xhd, nxb, xa);
        } else if constexpr (NX > 1) {
            // f32 rows staged here (K ≤ 1024): wave w takes activation row w
            if (!a.x_rec && wave < nx)
                stage_row_load((const float*)a.x + (size_t)wave * a.K, a.gamma, nxb, xp);
        } else {
            if (one_pass)
                stage_x_load<XT>((const XT*)a.x + (size_t)xb0 * 32,
                                 a.gamma ? a.gamma + (size_t)xb0 * 32 : nullptr, nxb, xp);
        }
        load_tile_aux(0);
    };
    if constexpr (is_hook<Hook>()) {
#pragma unroll
        for (int h = 0; h < PF; ++h) issue(h, buf[h]);
        hook();
        load_x();
    } else {
        load_x();
#pragma unroll
        for (int h = 0; h < PF; ++h) issue(h, buf[h]);  // items past nitems load clamped addresses
    }
    constexpr bool coh_x = __is_same(XT, AttnXC) || __is_same(XT, CohF32);
    if constexpr (is_attn_x<XT>()) {
        stage_attn_convert<F::Q40PERM, coh_x>(xa, a.xnsp, nxb, xs);
    } else {
        // (the host launches whole-K kernels either with x records or with a
        // K that one pass covers)
        if constexpr (NX > 1) {
            if (!a.x_rec) {
                if (wave < nx) stage_row_convert(xp, a.gamma, a.eps, nxb, xs + (size_t)wave * nxb);
            } else {
                // every row's records of the chunk, loads of all rows in flight
                const uint32_t n16 = nxb * (sizeof(XRec) / 16), kr = a.K / 32;
                for (uint32_t i = threadIdx.x; i < nx * n16; i += wg_threads()) {
                    const uint32_t m = i / n16, j = i % n16;
                    ((u32x4*)xs)[i] = ((const u32x4*)((const XRec*)a.x + (size_t)m * kr + xb0))[j];
                }
            }
        } else if (one_pass)
            stage_x_convert<F::Q40PERM, coh_x>(xp, a.gamma, a.eps, nxb, xs);
        else
            copy_x_limbs((const XRec*)a.x, xb0, nxb, xs);
    }
    lds_barrier();  // the records are in LDS; the weight loads stay in flight
    if (nitems == 0) return;

    for (uint32_t it = 0; it < nitems; it += PF) {
#pragma unroll
        for (int half = 0; half < PF; ++half) {
            const uint32_t item = it + half;
            if (item < nitems) {  // uniform across the workgroup
                if (item > 0 && item % spw == 0) load_tile_aux(item);
                const uint32_t step = wk + ksw * (item % spw);
                const uint32_t u = slot + 16 * step;
                const bool valid = u < units;
                const uint32_t uc = valid ? u : 0;
#pragma unroll
                for (int rq = 0; rq < RQ; ++rq)
#pragma unroll
                    for (int m = 0; m < NX; ++m)
                        if (m < (int)nx) {
                            const float v = F::mdot(buf[half][rq], xs + (size_t)m * nxb, uc, lq);
                            acc[rq][m] += valid ? v : 0.0f;
                        }
                if (item + PF < nitems) issue(item + PF, buf[half]);
                if (item % spw == spw - 1) {
                    const uint32_t vbase = rows_of(item / spw);
                    float rsum[RQ][NX];
#pragma unroll
                    for (int rq = 0; rq < RQ; ++rq)
#pragma unroll
                        for (int m = 0; m < NX; ++m) {
                            if (m >= (int)nx) continue;
                            // sum over the 16 slots of the row: lane bits 2..5
                            float v = acc[rq][m];
                            v += swz_xor_f<4>(v);
                            v += swz_xor_f<8>(v);
                            v += swz_xor_f<16>(v);
                            v += __shfl_xor(v, 32, 64);
                            rsum[rq][m] = v;
                            acc[rq][m] = 0.0f;
                        }
                    if (ksw > 1) {
                        // combine the K-split waves of the group in a fixed order
                        if (slot == 0) {
#pragma unroll
                            for (int rq = 0; rq < RQ; ++rq)
#pragma unroll
                                for (int m = 0; m < NX; ++m)
                                    if (m < (int)nx) red[((wave * RQ + rq) * NX + m) * 4 + q] = rsum[rq][m];
                        }
                        lds_barrier();
                        if (wk == 0) {
#pragma unroll
                            for (int rq = 0; rq < RQ; ++rq)
#pragma unroll
                                for (int m = 0; m < NX; ++m) {
                                    if (m >= (int)nx) continue;
                                    float t = 0.0f;
                                    for (uint32_t w = 0; w < ksw; ++w)
                                        t += red[(((wgrp * ksw + w) * RQ + rq) * NX + m) * 4 + q];
                                    rsum[rq][m] = t;
                                }
                        }
                        lds_barrier();
                    }
                    if (S > 1) {
                        // partial sums of this K chunk (the tiles are
                        // finished after the loop)
                        if (wk == 0 && slot == 0) {
#pragma unroll
                            for (int rq = 0; rq < RQ; ++rq) {
                                const uint32_t vr = vbase + 4 * rq + q;
#pragma unroll
                                for (int m = 0; m < NX; ++m)
                                    if (m < (int)nx && vr < a.nvrows)
                                        dev_store(a.part + ((size_t)ks * nx + m) * a.nvrows + vr, rsum[rq][m]);
                            }
                        }
                    } else if (wk == 0) {
#pragma unroll
                        for (int rq = 0; rq < RQ; ++rq) {
                            const uint32_t vr = vbase + 4 * rq + q;
#pragma unroll
                            for (int m = 0; m < NX; ++m) {
                                if (m >= (int)nx) continue;
                                const float v = rsum[rq][m];
                                if (epi_base(EPI) == EPI_FFN) {
                                    // quad holds (gate r, up r, gate r+1, up r+1)
                                    const float up = dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(v);
                                    if (slot == 0 && (q & 1) == 0 && vr + 1 < a.nvrows)
                                        out_store<EPI>((float*)a.out[0] + (size_t)m * (a.nvrows >> 1) + (vr >> 1),
                                                       silu_ref(v) * up);
                                } else {
                                    if (slot == 0 && vr < a.nvrows) store_row_pre<EPI>(a, vr, v, aux[rq][m], m);
                                }
                            }
                        }
                    }
                }
            }
        }
    }
    if (S > 1) {
        // K split: count this workgroup's chunk in for all its tiles at once
        // (the arrivals' latencies overlap); the last chunk to arrive at a
        // tile adds the chunks in order and runs the epilogue
        __shared__ uint8_t last_of[kMaxSplitTiles];
        dev_stores_done();
        __syncthreads();
        for (uint32_t t = tid; t < my_tiles; t += wg_threads())
            last_of[t] = arrive(a.counters + (size_t)(wg + t * nwg) * a.cstride) == S - 1;
        __syncthreads();
        for (uint32_t t = 0; t < my_tiles; ++t) {
            if (!last_of[t]) continue;  // uniform
            const uint32_t tile = wg + t * nwg;
            const uint32_t vt = tile * vrows_per_wg;
            const uint32_t step_r = epi_base(EPI) == EPI_FFN ? 2 : 1;
            for (uint32_t m = 0; m < nx; ++m)
            for (uint32_t i = tid * step_r; i < vrows_per_wg; i += wg_threads() * step_r) {
                const uint32_t vr = vt + i;
                if (vr >= a.nvrows) break;
                float v = 0.0f, v1 = 0.0f;
                for (uint32_t c = 0; c < S; ++c) {
                    const float* pc = a.part + ((size_t)c * nx + m) * a.nvrows;
                    v += dev_load(pc + vr);
                    if (epi_base(EPI) == EPI_FFN && vr + 1 < a.nvrows) v1 += dev_load(pc + vr + 1);
                }
                if (epi_base(EPI) == EPI_FFN) {
                    if (vr + 1 < a.nvrows)
                        out_store<EPI>((float*)a.out[0] + (size_t)m * (a.nvrows >> 1) + (vr >> 1), silu_ref(v) * v1);
                } else {
                    store_row<EPI>(a, vr, v, m);
                }
            }
            if (tid == 0) dev_store(a.counters + (size_t)tile * a.cstride, 0u);  // ready for the next call
        }
    }
}

template <class F, int EPI, typename XT, int RPL, int UNR>
RT_DEV void gemv_body(const GemvArgs& a) {
    if (a.xb_chunk >= a.K / 32)
        gemv_body_pipelined<F, EPI, XT, RPL, UNR>(a);
    else
        gemv_body_chunked<F, EPI, XT, RPL, UNR>(a);
}

// MFMA kernels: whole-K (or K-split) launches use the matrix-core body with
// unit format FM; launches whose K exceeds the LDS budget without a split use
// the chunked v_dot4 body with unit format FC.
// Items in flight per wave on the matrix-core path: a format may set PF.
// Formats whose lanes each load a long unit (Q6_K: 212 bytes, Q8_0: 68) keep
// one item in flight: with two, a wave's loads touch each cache line again
// after it has left L1 (the lines of a unit are shared by the wave's
// consecutive load instructions), and the stream slows down.
template <class F>
constexpr int fmt_pf_get(decltype(F::PF)*) { return F::PF; }
template <class F>
constexpr int fmt_pf_get(...) { return 0; }
template <class F>
constexpr int fmt_pf() { return fmt_pf_get<F>(nullptr); }

template <class FM, class FC, int EPI, typename XT, int RQ, int RPL, int UNR>
RT_DEV void gemv_mq_or_chunked(const GemvArgs& a) {
    if (a.xb_chunk >= a.K / 32)
        gemv_mq_body<FM, EPI, XT, RQ, (fmt_pf<FM>() ? fmt_pf<FM>() : (RQ == 1 ? GEMV_PF1 : GEMV_PF2))>(a);
    else
        gemv_body_chunked<FC, EPI, XT, RPL, UNR>(a);
}

// Thread bound of the GEMV kernels: 1024-thread workgroups (one per CU) serve
// the large whole-K launches, whose waves then issue their first loads
// together instead of queueing behind the weight loads of earlier
// workgroups on the CU (the register budget stays at 128 per lane).
#define RT_GEMV_LB 1024
#define RT_GEMV_KERNEL2(NAME, FMTM, FMTC, EPI, XT, UNR)                                 \
    extern "C" __global__ void __launch_bounds__(RT_GEMV_LB) NAME##_r1(GemvArgs a) {  \
        gemv_mq_or_chunked<FMTM, FMTC, EPI, XT, 1, (epi_base(EPI) == EPI_FFN ? 2 : 1), UNR>(a);  \
    }                                                                                   \
    extern "C" __global__ void __launch_bounds__(RT_GEMV_LB) NAME##_r2(GemvArgs a) {  \
        gemv_mq_or_chunked<FMTM, FMTC, EPI, XT, 2, (epi_base(EPI) == EPI_FFN ? 2 : 1), UNR>(a);  \
    }
#define RT_GEMV_KERNEL(NAME, FMT, EPI, XT, UNR) RT_GEMV_KERNEL2(NAME, FMT, FMT, EPI, XT, UNR)
// As RT_GEMV_KERNEL2, for at most 512 threads with a register budget for WPE
// waves per SIMD (Q6_K: a whole super-block per lane needs ~240 registers)
#define RT_GEMV_KERNEL2W(NAME, FMTM, FMTC, EPI, XT, UNR, WPE)                                \
    extern "C" __global__ void __launch_bounds__(512, WPE) NAME##_r1(GemvArgs a) {          \
        gemv_mq_or_chunked<FMTM, FMTC, EPI, XT, 1, (epi_base(EPI) == EPI_FFN ? 2 : 1), UNR>(a);      \
    }                                                                                       \
    extern "C" __global__ void __launch_bounds__(512, WPE) NAME##_r2(GemvArgs a) {          \
        gemv_mq_or_chunked<FMTM, FMTC, EPI, XT, 2, (epi_base(EPI) == EPI_FFN ? 2 : 1), UNR>(a);      \
    }
// Formats that never take the 1024-thread form (Q8_0): built for 512 threads
#define RT_GEMV_KERNEL512(NAME, FMT, EPI, XT, UNR)                                         \
    extern "C" __global__ void __launch_bounds__(512) NAME##_r1(GemvArgs a) {              \
        gemv_mq_or_chunked<FMT, FMT, EPI, XT, 1, (epi_base(EPI) == EPI_FFN ? 2 : 1), UNR>(a);        \
    }                                                                                       \
    extern "C" __global__ void __launch_bounds__(512) NAME##_r2(GemvArgs a) {              \
        gemv_mq_or_chunked<FMT, FMT, EPI, XT, 2, (epi_base(EPI) == EPI_FFN ? 2 : 1), UNR>(a);        \
    }
#define RT_Q6K_WPE 2
// Multi-row kernels (<name>_x8): up to 8 activation rows (records prepared by
// k_act_limbs_rows) through the matrix-core body, whole K or K split.
#define RT_GEMV_ROWS(NAME, FMT, EPI, LB)                                                  \
    extern "C" __global__ void __launch_bounds__(LB) NAME##_x8(GemvArgs a) {              \
        gemv_mq_body<FMT, EPI, float, 1, (fmt_pf<FMT>() ? fmt_pf<FMT>() : GEMV_PF1), NoHook, 8>(a); \
    }

// Single-block-unit fallback (rows with an odd number of 32-element blocks)
#define RT_GEMV_KERNEL_S(NAME, FMT, EPI, XT, UNR)                                 \
    extern "C" __global__ void __launch_bounds__(512) NAME##_s1(GemvArgs a) {    \
        gemv_body<FMT, EPI, XT, (epi_base(EPI) == EPI_FFN ? 2 : 1), UNR>(a);                \
    }

// Q8_0 (gemv_q8_0.metal, gemv_multirow.metal, fused_qkv.metal, fused_ffn.metal)

// Q, K and V projections whose matrices differ in format (Q4_K_M files keep
// V in Q6_K) in one launch: workgroups [0, b.blk0) run Q and K (format FA),
// the rest run V (format FB), each part with its own tiling of the
// matrix-core body; the reference issues three GEMVs and three bias adds
// for these (forward.rs:1561-1568).
template <class FA, class FB, int EPI>
RT_DEV void gemv_mq_pair(const GemvArgs& a, const GemvArgs& b) {
    if (blockIdx.x < b.blk0)
        gemv_mq_body<FA, EPI, float, 1, (fmt_pf<FA>() ? fmt_pf<FA>() : GEMV_PF1)>(a);
    else
        gemv_mq_body<FB, EPI, float, 1, (fmt_pf<FB>() ? fmt_pf<FB>() : GEMV_PF1)>(b);
}
#define RT_GEMV_PAIR(NAME, FA, FB, EPI)                                                        \
    extern "C" __global__ void __launch_bounds__(RT_GEMV_LB) NAME##_r1(GemvArgs a, GemvArgs b) { \
        gemv_mq_pair<FA, FB, EPI>(a, b);                                                       \
    }

// Activation pre-pass: builds the limb records of x (nxb records) in global
// memory once, for launches whose K is too long to convert per workgroup.
template <typename XT, bool Q40PERM>
RT_DEV void act_limbs_body(const XT* __restrict__ x, XRec* __restrict__ out, uint32_t nxb) {
    const uint32_t total = nxb * 8;
    for (uint32_t t = blockIdx.x * wg_threads() + threadIdx.x; t < total;
         t += gridDim.x * wg_threads()) {
        float v[4];
        load_x4<XT>(x, (t >> 3) * 32 + (t & 7) * 4, v);
        limb_slice<Q40PERM>(v, t & 7, out + (t >> 3));
    }
}

// Multi-row pre-pass: the limb records of `rows` activation rows ([rows][K]
// f32), one workgroup per row; with γ the row is RMS-normalised first,
// x̂ = x · rsqrt(Σx²/K + eps) · γ, each product rounded in f32 as the fused
// staging (stage_x_convert) computes it.
template <bool Q40PERM>
RT_DEV void act_limbs_rows_body(const float* __restrict__ x, const float* __restrict__ gamma,
                                float eps, uint32_t K, XRec* __restrict__ out) {
    const uint32_t nxb = K / 32, total = nxb * 8, nt = wg_threads();
    const float* xr = x + (size_t)blockIdx.x * K;
    XRec* o = out + (size_t)blockIdx.x * nxb;
    float rms = 1.0f;
    if (gamma) {
        __shared__ float nred[16];
        float ss = 0.0f;
        for (uint32_t t = threadIdx.x; t < total; t += nt) {
            const f32x4 v = *(const f32x4*)(xr + (t >> 3) * 32 + (t & 7) * 4);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = group_sum(ss, 64);
        if ((threadIdx.x & 63) == 0) nred[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (uint32_t w = 0; w < (nt >> 6); ++w) tot += nred[w];
        rms = rsqrtf(tot / (float)K + eps);
    }
    for (uint32_t t = threadIdx.x; t < total; t += nt) {
        const uint32_t i = (t >> 3) * 32 + (t & 7) * 4;
        const f32x4 xv = *(const f32x4*)(xr + i);
        float v[4] = {xv.x, xv.y, xv.z, xv.w};
        if (gamma) {
            const f32x4 g = *(const f32x4*)(gamma + i);
            v[0] = v[0] * rms * g.x; v[1] = v[1] * rms * g.y;
            v[2] = v[2] * rms * g.z; v[3] = v[3] * rms * g.w;
        }
        limb_slice<Q40PERM>(v, t & 7, o + (t >> 3));
    }
}

