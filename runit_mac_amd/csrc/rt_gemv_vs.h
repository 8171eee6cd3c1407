// rt_gemv_vs.h — VALU small-launch GEMV body (f32 dots, no staging barrier)
// for gfx950 (instantiated by kvs.hip).
//
// The 0.5B decode step's projections move 1-9 MB each and are bound by the
// chain from kernel start to first dot, not by their weight stream: the
// limb-record bodies stage the activation vector once per workgroup (loads,
// conversion, a workgroup barrier that waits for the slowest wave), copy
// every weight item through LDS and reduce the matrix-core results.  Here a
// lane takes one (row, 32-element block) pair and loads both the block's
// bytes and the block's activations itself; the four lanes of a block (rows
// 0..3 of a row quad) read the same activation addresses in one instruction.
// The dot is 32 f32 fused multiply-adds on the dequantised codes, scaled by
// the block's f16 scale; 16 blocks' partial sums meet by cross-lane adds,
// the waves sharing a row quad (rows longer than 16 blocks) through LDS.
// RMSNorm (γ given) is computed by every wave from the whole x (K ≤ 1024:
// 16 floats per lane), so no wave waits for another before its first dot.
//
// Error: per row ≤ (32 + 1 + log2(16) + waves) roundings of 2^-24 relative
// to Σ|w·x| (≈ 2.6e-6·Σ|w·x| at K = 4864), inside the 1e-4·Σ|w·x| bound for
// any input range (no block-floating-point activation form).
#pragma once
#include "rt_gemv.h"

constexpr uint32_t kVsMaxNormK = 1024;  // RMSNorm in the body: whole x, ≤ 16 floats per lane

// Q8_0 block b of a row: d·Σ q_i·y_i over its 32 elements, y from the lane's
// activations (already normalised where the launch has γ).
RT_DEV float vs_q8_0_block(const FmtQ8_0S::Raw& r, const f32x4 y[8]) {
    // block bytes from the 4-byte floor: d at byte sh, codes at sh + 2
    const uint32_t d16 = alignb(r.w[1], r.w[0], r.sh);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t q = r.sh ? r.w[i + 1] : alignb(r.w[i + 1], r.w[i], 2);
        const f32x4 v = y[i];
        acc = __builtin_fmaf((float)(int8_t)(q & 255u), v.x, acc);
        acc = __builtin_fmaf((float)(int8_t)((q >> 8) & 255u), v.y, acc);
        acc = __builtin_fmaf((float)(int8_t)((q >> 16) & 255u), v.z, acc);
        acc = __builtin_fmaf((float)(int8_t)(q >> 24), v.w, acc);
    }
    return h2f(d16) * acc;
}

// One launch: row quads of a.nvrows virtual rows; wpq waves per quad (⌈nb/16⌉
// blocks of 16), qpw = waves / wpq quads per workgroup.
template <int EPI, bool NORM>
RT_DEV void gemv_vs_body(const GemvArgs& a) {
    __shared__ float part[16][4];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t r = lane & 3, s = lane >> 2;
    const uint32_t nb = a.K / 32;
    const uint32_t wpq = (nb + 15) / 16;
    const uint32_t qpw = (wg_threads() >> 6) / wpq;
    const uint32_t nq = (a.nvrows + 3) / 4;
    const uint32_t quad = blockIdx.x * qpw + wave / wpq, sub = wave % wpq;
    const uint32_t b = sub * 16 + s;
    const bool valid = quad < nq && b < nb;
    const uint32_t vr0 = (quad < nq ? quad : nq - 1) * 4 + r;
    const uint32_t vr = vr0 < a.nvrows ? vr0 : a.nvrows - 1;
    const uint32_t bc = valid ? b : 0;
    // the block's bytes, the block's activations (and γ), then the epilogue
    // operand: all loads issued before any arithmetic
    uint32_t mat, row;
    vrow_map<EPI>(a, vr, mat, row);
    FmtQ8_0S::Raw raw;
    FmtQ8_0S::load(mat_w(a, mat) + (size_t)row * a.row_bytes, bc, raw);
    const float* x = (const float*)a.x;
    f32x4 y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = *(const f32x4*)(x + bc * 32 + 4 * i);
    f32x4 g[8];
    f32x4 xn[4];
    float sqp[4];
    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = *(const f32x4*)(a.gamma + bc * 32 + 4 * i);
        if (a.ssq_in) {
            // Σx² as the producing launch's partial sums (≤ 256)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t k = lane + 64 * i;
                sqp[i] = k < a.ssq_n ? a.ssq_in[k] : 0.0f;
            }
        } else {
            // the whole x for Σx² (K ≤ 1024: 4 float4 per lane)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t e = (lane + 64 * i) * 4;
                xn[i] = e < a.K ? *(const f32x4*)(x + e) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }
    float aux = 0.0f;
    if (has_aux<EPI>()) aux = load_aux<EPI>(a, vr);
    if constexpr (NORM) {
        // rms_norm_f32_f32_f32g (norm.metal:126-154): y = x·rsqrt(Σx²/K + eps)·γ
        float ss = 0.0f;
        if (a.ssq_in) {
            ss = sqp[0] + sqp[1] + sqp[2] + sqp[3];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ss += xn[i].x * xn[i].x + xn[i].y * xn[i].y + xn[i].z * xn[i].z + xn[i].w * xn[i].w;
        }
        ss = group_sum(ss, 64);
        const float rms = rsqrtf(ss / (float)a.K + a.eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            y[i].x = y[i].x * rms * g[i].x;
            y[i].y = y[i].y * rms * g[i].y;
            y[i].z = y[i].z * rms * g[i].z;
            y[i].w = y[i].w * rms * g[i].w;
        }
    }
    float acc = valid ? vs_q8_0_block(raw, y) : 0.0f;
    // the 16 blocks of the row in this wave (lane bits 2..5)
    acc += swz_xor_f<4>(acc);
    acc += swz_xor_f<8>(acc);
    acc += swz_xor_f<16>(acc);
    acc += __shfl_xor(acc, 32, 64);
    if (wpq > 1) {
        if (s == 0) part[wave][r] = acc;
        lds_barrier();
        if (sub != 0) return;
        acc = 0.0f;
        for (uint32_t w = 0; w < wpq; ++w) acc += part[wave + w][r];
    }
    if (quad >= nq || s != 0) return;
    if (EPI == EPI_FFN) {
        // quad rows (gate r, up r, gate r+1, up r+1)
        const float up = dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(acc);
        if ((r & 1) == 0 && vr0 + 1 < a.nvrows) ((float*)a.out[0])[vr0 >> 1] = silu_ref(acc) * up;
    } else {
        if (vr0 < a.nvrows) store_row_pre<EPI>(a, vr0, acc, aux);
        if (epi_base(EPI) == EPI_F32_ADD && a.ssq_out)
            quad_ssq_store(a.ssq_out, quad, acc + aux, vr0 < a.nvrows, r);
    }
}

#define RT_GEMV_VS(NAME, EPI, NORM) \
    extern "C" __global__ void __launch_bounds__(1024) NAME##_vs(GemvArgs a) { gemv_vs_body<EPI, NORM>(a); }

