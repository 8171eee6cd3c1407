// rt_device.h — device-side building blocks shared by every gfx950 kernel of
// the quantized-GEMV decode path.
//
//  * f16 helpers (IEEE binary16 ↔ binary32, round-to-nearest-even).
//  * Wave64 cross-lane sums built from DPP (quad_perm / row mirrors) and
//    ds_swizzle, instead of Metal's 32-lane simd_sum.
//  * The activation "limb" record: every 32-element block of the f32
//    activation vector x is turned, once per workgroup, into a block-floating
//    point integer form  x_i = 2^(E-22) · (65536·a_i + 256·b_i + c_i)  with
//    signed int8 limbs a, b, c.  Weights are integers inside a GGUF block
//    (int8, nibbles, 6-bit codes), so a block dot product becomes three exact
//    v_dot4_i32_i8 chains; scales are applied once per 32 elements in f32.
//    x is represented to 22 bits below the block's power-of-two bound, i.e.
//    |x_i − x̂_i| ≤ 2^(E−23) ≤ 2^-22·max|x_block|.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define RT_DEV __device__ __forceinline__

// Threads per workgroup: one scalar load of the implicit-argument dword at
// byte 12 (group_size_x in its low half), which arrives with the kernel
// arguments.  blockDim.x compiles to a 16-bit vector load issued only after
// the kernel arguments have arrived (a second round trip that every wave
// waits for before its first load of real data).
RT_DEV uint32_t wg_threads() {
    const uint32_t* ia = (const uint32_t*)__builtin_amdgcn_implicitarg_ptr();
    return ia[3] & 0xFFFFu;
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS (and
// scalar) operations, not for its global loads.  __syncthreads() also waits
// for every outstanding global load, which stalls a kernel that has weight
// loads in flight across the barrier until they all return.
RT_DEV void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16 bytes at base + off through a raw buffer descriptor.  none = true gives
// the descriptor no records: the hardware's range check then drops the
// request (no memory access) and returns zeros.  The same instruction either
// way, so a loop that issues it every iteration keeps exact load counts.
RT_DEV u32x4 load16_or_none(const void* base, uint32_t off, bool none) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, none ? 0 : 0x7FFFFFFF, 0x00020000);
    return (u32x4)__builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
}

// ───────────────────────────── f16 ─────────────────────────────

RT_DEV float h2f(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
    return (float)h;  // exact
}
RT_DEV uint16_t f2h(float f) {
    _Float16 h = (_Float16)f;  // IEEE round-to-nearest-even
    return __builtin_bit_cast(uint16_t, h);
}

// ───────────────────────────── cross-lane ─────────────────────────────

// DPP controls (GCN/CDNA encoding).
#define DPP_QUAD_PERM(a, b, c, d) ((a) | ((b) << 2) | ((c) << 4) | ((d) << 6))
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_HALF_MIRROR 0x141

template <int CTRL>
RT_DEV float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
RT_DEV int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// ds_swizzle bit-mode: lane' = ((lane & and) | or) ^ xor, within 32 lanes.
template <int XORM>
RT_DEV float swz_xor_f(float v) {
    constexpr int pat = 0x1F | (XORM << 10);
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), pat));
}

// Sum over aligned groups of `n` lanes (n ∈ {1,2,4,...,64}, wave-uniform).
// Every lane of a group receives the group total.
RT_DEV float group_sum(float v, int n) {
    if (n >= 2) v += dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(v);
    if (n >= 4) v += dpp_f<DPP_QUAD_PERM(2, 3, 0, 1)>(v);
    if (n >= 8) v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    if (n >= 16) v += dpp_f<DPP_ROW_MIRROR>(v);
    if (n >= 32) v += swz_xor_f<16>(v);
    if (n >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}
RT_DEV float group_max(float v, int n) {  // as group_sum, with max
    if (n >= 2) v = fmaxf(v, dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(v));
    if (n >= 4) v = fmaxf(v, dpp_f<DPP_QUAD_PERM(2, 3, 0, 1)>(v));
    if (n >= 8) v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    if (n >= 16) v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    if (n >= 32) v = fmaxf(v, swz_xor_f<16>(v));
    if (n >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}
RT_DEV float max8(float v) {  // max over aligned groups of 8 lanes
    v = fmaxf(v, dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_PERM(2, 3, 0, 1)>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    return v;
}
RT_DEV int sum8_i(int v) {
    v += dpp_i<DPP_QUAD_PERM(1, 0, 3, 2)>(v);
    v += dpp_i<DPP_QUAD_PERM(2, 3, 0, 1)>(v);
    v += dpp_i<DPP_ROW_HALF_MIRROR>(v);
    return v;
}
RT_DEV int sum4_i(int v) {
    v += dpp_i<DPP_QUAD_PERM(1, 0, 3, 2)>(v);
    v += dpp_i<DPP_QUAD_PERM(2, 3, 0, 1)>(v);
    return v;
}

RT_DEV int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ───────────────────── cross-workgroup hand-off ─────────────────────
//
// Partial results that another workgroup (possibly on another XCD) combines
// are written with device-scope stores (written through to the coherent
// level instead of staying in this XCD's L2) and read back with device-scope
// loads.  arrive() waits until this thread's stores have completed and then
// counts the workgroup in; callers put a __syncthreads() between every
// thread's dev_store()s and the one thread that calls arrive().  No L2
// write-back or invalidate of whole caches is involved.
template <typename T>
RT_DEV void dev_store(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
RT_DEV T dev_load(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RT_DEV void dev_stores_done() { __builtin_amdgcn_s_waitcnt(0); }
RT_DEV uint32_t arrive(uint32_t* counter) {
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Hook of a kernel body run as one phase of a persistent kernel: the wait
// for the previous phase (grid barrier).  With one, a body issues the loads
// that do not depend on the previous phase (weights, KV-cache rows) first,
// then waits, then loads the activations: those loads arrive while the grid
// waits.
struct NoHook {
    RT_DEV void operator()() const {}
};
template <class Hook>
constexpr bool is_hook() { return !__is_same(Hook, NoHook); }

// ───────────────────────────── activation limbs ─────────────────────────────
//
// One record per 32 activations, 112 bytes (a stride of 28 dwords keeps eight
// consecutive records' ds_read_b128 on distinct bank groups):
//   limb[0][32] (×65536), limb[1][32] (×256), limb[2][32] (×1)  — int8
//   e        : int16, block exponent E (x̂ = 2^(E-22)·(...))
//   s[2][3]  : int16, Σ of each limb over elements 0-15 and 16-31
//   pad      : int16
struct __attribute__((aligned(16))) XRec {
    uint32_t limb[3][8];
    int16_t e;
    int16_t s[2][3];
    int16_t pad;
};
static_assert(sizeof(XRec) == 112, "XRec layout");

constexpr int XREC_BYTES = 112;
constexpr int XE_NONFINITE = 300;  // marks a block that holds Inf/NaN

// Position of element j (0..31) of a block inside its record.  The Q4_0
// layout of the reference packs element 2i in the low nibble and 2i+1 in the
// high nibble of byte i (gemv_q4_0.metal:13-14, forward.rs:974-976); a dword
// of nibbles therefore yields elements {0,2,4,6} (low) and {1,3,5,7} (high),
// and its records store each 8-group as evens then odds.
template <bool Q40PERM>
RT_DEV int xpos(int j) {
    if (!Q40PERM) return j;
    return (j & ~7) | ((j & 1) << 2) | ((j >> 1) & 3);
}

template <typename XT>
RT_DEV void load_x4(const XT* x, uint32_t idx, float v[4]);
template <>
RT_DEV void load_x4<float>(const float* x, uint32_t idx, float v[4]) {
    f32x4 t = *(const f32x4*)(x + idx);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
// f32 activations written by other workgroups of the same (persistent)
// launch: read at device scope, so no cache returns a stale copy
struct CohF32 {};
template <>
RT_DEV void load_x4<CohF32>(const CohF32* x, uint32_t idx, float v[4]) {
    const float* p = (const float*)x + idx;
    v[0] = dev_load(p); v[1] = dev_load(p + 1); v[2] = dev_load(p + 2); v[3] = dev_load(p + 3);
}
template <>
RT_DEV void load_x4<uint16_t>(const uint16_t* x, uint32_t idx, float v[4]) {
    uint2 t = *(const uint2*)(x + idx);
    v[0] = h2f(t.x); v[1] = h2f(t.x >> 16); v[2] = h2f(t.y); v[3] = h2f(t.y >> 16);
}

// Converts one 4-element slice (lane q of the 8 lanes of x-block b) into
// limbs and writes them to the block's record.  The 8 lanes of a block are
// 8 consecutive, 8-aligned lanes, all active.  Straight-line code: the
// non-finite cases are selects, and every lane stores whole dwords (limb
// dword q of each limb plane, and meta dword q % 4, which lanes q and q + 4
// write with the same value).
// Block exponent and balanced base-256 digits of one 4-element slice (lane q
// of the 8 consecutive, 8-aligned, active lanes of an x-block): e is the
// block's frexp exponent (XE_NONFINITE if it holds Inf/NaN, 0 if all zero)
// and x_i ≈ 2^(e-22)·(65536·l[0][i] + 256·l[1][i] + l[2][i]).
RT_DEV void limb_digits(const float v[4], int& e, int l[3][4]) {
    constexpr float FMAX = 3.40282347e38f;
    bool nf[4];
    bool any_nf = false;
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float av = fabsf(v[i]);
        nf[i] = !(av <= FMAX);  // ±Inf or NaN
        any_nf |= nf[i];
        a = fmaxf(a, av);
    }
    // a non-finite element makes the whole block non-finite
    a = max8(any_nf ? __builtin_huge_valf() : a);
    const bool finite = a <= FMAX;
    const int ef = __builtin_amdgcn_frexp_expf(a);  // a < 2^ef
    e = !finite ? XE_NONFINITE : (a == 0.0f ? 0 : ef);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // finite block: round(x · 2^(22-e)), |xi| ≤ 2^22.  Non-finite block:
        // ±2^22 on non-finite elements (NaN as +), 0 elsewhere; with e = 300
        // their products overflow to ±Inf (or NaN).
        const int xf = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(v[i], 22 - ef));
        const int xn = nf[i] ? ((v[i] < 0.0f) ? -(1 << 22) : (1 << 22)) : 0;
        const int xi = finite ? xf : xn;
        const int c = ((xi + 128) & 255) - 128;
        const int r1 = (xi - c) >> 8;
        const int bb = ((r1 + 128) & 255) - 128;
        l[0][i] = (r1 - bb) >> 8;
        l[1][i] = bb;
        l[2][i] = c;
    }
}
RT_DEV uint32_t pack_i8x4(const int l[4]) {
    return (uint32_t)(l[0] & 255) | ((uint32_t)(l[1] & 255) << 8) |
           ((uint32_t)(l[2] & 255) << 16) | ((uint32_t)l[3] << 24);
}

// Converts one 4-element slice (lane q of the 8 lanes of x-block b) into
// limbs and writes them to the block's record.  Straight-line code: the
// non-finite cases are selects, and every lane stores whole dwords (limb
// dword q of each limb plane, and meta dword q % 4, which lanes q and q + 4
// write with the same value).
template <bool Q40PERM>
RT_DEV void limb_slice(const float v[4], uint32_t q, XRec* __restrict__ rec) {
    int e;
    int l[3][4];
    limb_digits(v, e, l);
    uint32_t* recw = (uint32_t*)rec;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const uint32_t own = pack_i8x4(l[k]);
        uint32_t w = own;
        if (Q40PERM) {
            // 8-group as evens then odds: lane 2m stores elements
            // {8m, 8m+2, 8m+4, 8m+6}, lane 2m+1 stores {8m+1, 8m+3, 8m+5, 8m+7}
            const uint32_t par = (uint32_t)dpp_i<DPP_QUAD_PERM(1, 0, 3, 2)>((int)own);
            w = __builtin_amdgcn_perm(par, own, (q & 1) ? 0x03010705u : 0x06040200u);
        }
        recw[8 * k + q] = w;
    }
    // limb sums per 16-element half (lanes 0-3 → half 0, 4-7 → half 1)
    int hs[2][3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int sq = sum4_i(l[k][0] + l[k][1] + l[k][2] + l[k][3]);
        const int sm = dpp_i<DPP_ROW_HALF_MIRROR>(sq);  // the other half's sum
        hs[0][k] = q < 4 ? sq : sm;
        hs[1][k] = q < 4 ? sm : sq;
    }
    // meta dwords: (e, s00) (s01, s02) (s10, s11) (s12, pad)
    const uint32_t m0 = (uint32_t)(e & 0xFFFF) | ((uint32_t)hs[0][0] << 16);
    const uint32_t m1 = (uint32_t)(hs[0][1] & 0xFFFF) | ((uint32_t)hs[0][2] << 16);
    const uint32_t m2 = (uint32_t)(hs[1][0] & 0xFFFF) | ((uint32_t)hs[1][1] << 16);
    const uint32_t m3 = (uint32_t)(hs[1][2] & 0xFFFF);
    const uint32_t qm = q & 3;
    recw[24 + qm] = qm == 0 ? m0 : (qm == 1 ? m1 : (qm == 2 ? m2 : m3));
}

// Builds records for x-blocks [xb0, xb0+nxb) into recs[0..nxb).  Eight lanes
// per block, four activations per lane; each thread first issues the loads of
// up to XSTAGE_UNR slices, then converts them (one memory round trip per
// XSTAGE_UNR slices instead of one per slice).  All threads of the workgroup
// call it; callers follow it with a barrier.
constexpr int XSTAGE_UNR = 4;
template <typename XT, bool Q40PERM>
RT_DEV void stage_x_limbs(const XT* __restrict__ x, uint32_t xb0, uint32_t nxb,
                          XRec* __restrict__ recs) {
    const uint32_t total = nxb * 8;
    const uint32_t step = wg_threads();
    for (uint32_t t0 = threadIdx.x; t0 < total; t0 += XSTAGE_UNR * step) {
        float v[XSTAGE_UNR][4];
#pragma unroll
        for (int s = 0; s < XSTAGE_UNR; ++s) {
            const uint32_t t = t0 + s * step;
            if (t < total) load_x4<XT>(x, (xb0 + (t >> 3)) * 32 + (t & 7) * 4, v[s]);
        }
#pragma unroll
        for (int s = 0; s < XSTAGE_UNR; ++s) {
            const uint32_t t = t0 + s * step;
            if (t < total) limb_slice<Q40PERM>(v[s], t & 7, recs + (t >> 3));
        }
    }
}

// Copies nxb pre-built records (global) into LDS.
RT_DEV void copy_x_limbs(const XRec* __restrict__ src, uint32_t xb0, uint32_t nxb,
                         XRec* __restrict__ recs) {
    const u32x4* s = (const u32x4*)(src + xb0);
    u32x4* d = (u32x4*)recs;
    const uint32_t n16 = nxb * (sizeof(XRec) / 16);
    for (uint32_t i = threadIdx.x; i < n16; i += wg_threads()) d[i] = s[i];
}

// RMSNorm fused into the staging (rms_norm_f32_f32_f32g, norm.metal:126-154,
// followed by the GEMV): x̂ = x · rsqrt(Σx²/K + eps) · γ, element by element in
// f32 as the separate kernel computes it, then converted to limbs.  Every
// workgroup recomputes Σx² over the whole vector (K is the hidden size).
template <bool Q40PERM>
RT_DEV void stage_x_norm(const float* __restrict__ x, const float* __restrict__ gamma, float eps,
                         uint32_t K, XRec* __restrict__ recs) {
    __shared__ float nred[16];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x * 4; i < K; i += wg_threads() * 4) {
        const f32x4 v = *(const f32x4*)(x + i);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) nred[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (uint32_t w = 0; w < (wg_threads() >> 6); ++w) tot += nred[w];
    const float rms = rsqrtf(tot / (float)K + eps);
    const uint32_t total = (K / 32) * 8;
    const uint32_t step = wg_threads();
    for (uint32_t t0 = threadIdx.x; t0 < total; t0 += XSTAGE_UNR * step) {
        float v[XSTAGE_UNR][4];
#pragma unroll
        for (int s = 0; s < XSTAGE_UNR; ++s) {
            const uint32_t t = t0 + s * step;
            if (t < total) {
                const uint32_t i = (t >> 3) * 32 + (t & 7) * 4;
                const f32x4 a = *(const f32x4*)(x + i);
                const f32x4 g = *(const f32x4*)(gamma + i);
                v[s][0] = a.x * rms * g.x;
                v[s][1] = a.y * rms * g.y;
                v[s][2] = a.z * rms * g.z;
                v[s][3] = a.w * rms * g.w;
            }
        }
#pragma unroll
        for (int s = 0; s < XSTAGE_UNR; ++s) {
            const uint32_t t = t0 + s * step;
            if (t < total) limb_slice<Q40PERM>(v[s], t & 7, recs + (t >> 3));
        }
    }
}

// Two-phase staging for the whole-K launches whose vector fits in one pass
// (nxb·8 ≤ XSTAGE_UNR·blockDim slices): stage_x_load issues the loads of x
// (and γ), the caller issues its weight loads, and stage_x_convert then
// converts while those are in flight.
//
// Slice handled by this thread in round s: t = threadIdx.x + s·wg_threads().
// Threads past the end take slice q of block 0: their 8-lane groups rebuild
// record 0 exactly as its owners do (the same values into the same words),
// so no lane needs a branch.
RT_DEV uint32_t stage_slice(int s, uint32_t total) {
    const uint32_t t = threadIdx.x + s * wg_threads();
    return t < total ? t : (t & 7);
}
// U slices per thread (XSTAGE_UNR unless a body holds more registers for it)
template <int U>
struct XPreU {
    float v[U][4];
    float g[U][4];
    float sq[4];  // Σx² partials of the producing launch (≤ 256, 4 per lane)
};
constexpr uint32_t kMaxSsqParts = 256;
using XPre = XPreU<XSTAGE_UNR>;
template <int U = XSTAGE_UNR>
RT_DEV bool stage_one_pass(uint32_t nxb) { return nxb * 8 <= U * wg_threads(); }

// SKIP: lanes past the end load and convert nothing (whole 8-lane groups; a
// workgroup of many such lanes otherwise rebuilds record 0 many times over)
// ssq: the Σx² of x as nssq partial sums written by the launch that
// produced x (≤ kMaxSsqParts; null: the staging reduces x itself).
template <typename XT, int U, bool SKIP = false>
RT_DEV void stage_x_load(const XT* __restrict__ x, const float* __restrict__ gamma, uint32_t nxb,
                         XPreU<U>& p, const float* __restrict__ ssq = nullptr, uint32_t nssq = 0) {
    const uint32_t total = nxb * 8;
    if (ssq) {
        const uint32_t lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t k = lane + 64 * i;
            p.sq[i] = k < nssq ? ssq[k] : 0.0f;
        }
    }
#pragma unroll
    for (int s = 0; s < U; ++s) {
        // rounds past the vector are skipped (workgroup-uniform: no lane of a
        // later load is conditional); lanes past the end load clamped addresses
        if (s * wg_threads() >= total) break;
        // device-scope activations (a persistent kernel's): lanes past the
        // end load nothing (their clamped copies would all hit the same few
        // addresses at device scope) and convert nothing
        if ((SKIP || __is_same(XT, CohF32)) && threadIdx.x + s * wg_threads() >= total) continue;
        const uint32_t t = stage_slice(s, total);
        const uint32_t i = (t >> 3) * 32 + (t & 7) * 4;
        load_x4<XT>(x, i, p.v[s]);
        if (gamma) {
            const f32x4 g = *(const f32x4*)(gamma + i);
            p.g[s][0] = g.x; p.g[s][1] = g.y; p.g[s][2] = g.z; p.g[s][3] = g.w;
        }
    }
}

// With γ: x̂ = x · rsqrt(Σx²/K + eps) · γ (rms_norm_f32_f32_f32g,
// norm.metal:126-154), each product rounded in f32 as in stage_x_norm.
template <bool Q40PERM, bool SKIP = false, int U>
RT_DEV void stage_x_convert(XPreU<U>& p, const float* gamma, float eps, uint32_t nxb,
                            XRec* __restrict__ recs, bool have_ssq = false) {
    const uint32_t total = nxb * 8;
    if (gamma) {
        float tot;
        if (have_ssq) {
            // the producer's partial sums: every wave adds them itself, in
            // the same order, so no wave waits at a barrier for the others
            tot = group_sum(p.sq[0] + p.sq[1] + p.sq[2] + p.sq[3], 64);
        } else {
            __shared__ float nred[16];
            float ss = 0.0f;
#pragma unroll
            for (int s = 0; s < U; ++s) {
                const float sq = p.v[s][0] * p.v[s][0] + p.v[s][1] * p.v[s][1] +
                                 p.v[s][2] * p.v[s][2] + p.v[s][3] * p.v[s][3];
                ss += (threadIdx.x + s * wg_threads() < total) ? sq : 0.0f;
            }
            ss = group_sum(ss, 64);
            if ((threadIdx.x & 63) == 0) nred[threadIdx.x >> 6] = ss;
            lds_barrier();
            tot = 0.0f;
            for (uint32_t w = 0; w < (wg_threads() >> 6); ++w) tot += nred[w];
        }
        const float rms = rsqrtf(tot / (float)(nxb * 32) + eps);
#pragma unroll
        for (int s = 0; s < U; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i) p.v[s][i] = p.v[s][i] * rms * p.g[s][i];
    }
#pragma unroll
    for (int s = 0; s < U; ++s) {
        // rounds past the vector are skipped (workgroup-uniform); inside a
        // round, lanes past the end convert a copy of block 0 (see stage_slice)
        if (s * wg_threads() < total) {
            // (SKIP: lanes past the end loaded nothing; whole 8-lane groups)
            if (SKIP && threadIdx.x + s * wg_threads() >= total) continue;
            const uint32_t t = stage_slice(s, total);
            limb_slice<Q40PERM>(p.v[s], t & 7, recs + (t >> 3));
        }
    }
}

// x as split-attention partials: the slice of round 0 (one round only) loads
// (o, m, l) of up to 8 splits, and the conversion merges them exactly as the
// attention kernel's last workgroup does (o = Σ o_s·e^(m_s−M) / Σ l_s·e^(m_s−M),
// splits in order), then builds the slice's limbs.
struct AttnX {};
struct AttnXC {};  // the same, produced inside a persistent launch (device-scope loads)
template <typename XT>
constexpr bool is_attn_x() { return __is_same(XT, AttnX) || __is_same(XT, AttnXC); }
constexpr uint32_t kAttnXMaxSplits = 8;
struct XPreAttn {
    f32x4 o[kAttnXMaxSplits];
    float m[kAttnXMaxSplits], l[kAttnXMaxSplits];
};
template <bool COH = false>
RT_DEV void stage_attn_load(const void* part, const float* ml, uint32_t nsp, uint32_t hd,
                            uint32_t nxb, XPreAttn& p) {
    if (COH && threadIdx.x >= nxb * 8) return;  // (as stage_x_load for CohF32)
    const uint32_t t = stage_slice(0, nxb * 8);
    const uint32_t i = (t >> 3) * 32 + (t & 7) * 4;  // 4 elements of one head
    const uint32_t h = i / hd, d = i % hd;
#pragma unroll
    for (uint32_t j = 0; j < kAttnXMaxSplits; ++j) {
        // splits past nsp load split nsp − 1 again (unconditional loads; the
        // merge ignores them)
        const uint32_t jj = j < nsp ? j : nsp - 1;
        const size_t row = (size_t)h * nsp + jj;
        const float* po = (const float*)part + row * hd + d;
        if constexpr (COH) {
            p.o[j] = f32x4{dev_load(po), dev_load(po + 1), dev_load(po + 2), dev_load(po + 3)};
            p.m[j] = dev_load(ml + row * 2);
            p.l[j] = dev_load(ml + row * 2 + 1);
        } else {
            p.o[j] = *(const f32x4*)po;
            const float2 v = *(const float2*)(ml + row * 2);
            p.m[j] = v.x;
            p.l[j] = v.y;
        }
    }
}
template <bool Q40PERM, bool SKIP = false>
RT_DEV void stage_attn_convert(const XPreAttn& p, uint32_t nsp, uint32_t nxb,
                               XRec* __restrict__ recs) {
    if (SKIP && threadIdx.x >= nxb * 8) return;
    const uint32_t t = stage_slice(0, nxb * 8);
    float M = -__builtin_huge_valf();
#pragma unroll
    for (uint32_t j = 0; j < kAttnXMaxSplits; ++j)
        if (j < nsp) M = fmaxf(M, p.m[j]);
    float L = 0.0f;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t j = 0; j < kAttnXMaxSplits; ++j) {
        if (j < nsp) {
            const float f = expf(p.m[j] - M);
            L += p.l[j] * f;
            o += p.o[j] * f;
        }
    }
    o = o * (L > 0.0f ? 1.0f / L : 0.0f);
    float v[4] = {o.x, o.y, o.z, o.w};
    limb_slice<Q40PERM>(v, t & 7, recs + (t >> 3));
}

// Stages activations for x-blocks [xb0, xb0+nxb): from f32/f16 values, from
// RMSNorm(x) (gamma != null, whole K only), or from records that an earlier
// kernel already built (x_rec).
template <typename XT, bool Q40PERM>
RT_DEV void stage_x(const void* x, bool x_rec, uint32_t xb0, uint32_t nxb, XRec* recs,
                    const float* gamma = nullptr, float eps = 0.0f) {
    if (x_rec)
        copy_x_limbs((const XRec*)x, xb0, nxb, recs);
    else if (gamma)
        stage_x_norm<Q40PERM>((const float*)x, gamma, eps, nxb * 32, recs);
    else
        stage_x_limbs<XT, Q40PERM>((const XT*)x, xb0, nxb, recs);
}

// Registers holding one record (all three limbs + meta).
struct XRegs {
    uint32_t l[3][8];
    int e;
    int s[3];  // full-block limb sums
};
RT_DEV void load_xregs(const XRec* rec, XRegs& r) {
    const u32x4* p = (const u32x4*)rec;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        u32x4 a = p[2 * k], b = p[2 * k + 1];
        r.l[k][0] = a.x; r.l[k][1] = a.y; r.l[k][2] = a.z; r.l[k][3] = a.w;
        r.l[k][4] = b.x; r.l[k][5] = b.y; r.l[k][6] = b.z; r.l[k][7] = b.w;
    }
    u32x4 m = p[6];
    r.e = (int)(int16_t)(m.x & 0xFFFF);
    const int s00 = (int16_t)(m.x >> 16), s01 = (int16_t)(m.y & 0xFFFF),
              s02 = (int16_t)(m.y >> 16);
    const int s10 = (int16_t)(m.z & 0xFFFF), s11 = (int16_t)(m.z >> 16),
              s12 = (int16_t)(m.w & 0xFFFF);
    r.s[0] = s00 + s10;
    r.s[1] = s01 + s11;
    r.s[2] = s02 + s12;
}

// Σ over limbs of an exact limb-dot triple, as f32: 65536·t0 + 256·t1 + t2.
RT_DEV float limb_combine(int t0, int t1, int t2) {
    return __builtin_fmaf((float)t0, 65536.0f, (float)(t1 * 256 + t2));
}
