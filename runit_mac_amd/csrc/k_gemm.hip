// k_gemm.hip — batched Q8_0 GEMM, Y[M,N] = X[M,K]·W[N,K]ᵀ, for M ≥ 2 (new:
// the reference's only M > 1 path is gemm_f16 on f16-dequantised weights,
// gemm.metal:39-190, called from verify_draft, forward.rs:2193-2271).
//
// One v_mfma_i32_16x16x32_i8 per (Q8_0 block, 4 activation rows, 16 weight
// rows): its K of 32 is exactly one block, so the block's scales apply to the
// MFMA's integer result.
//   A (16×32): row 4·mm + limb = limb plane `limb` (0..2; row 3 is zero) of
//              activation row 4g + mm, i.e. the same exact base-256 digits as
//              the GEMV path (rt_device.h);
//   B (32×16): the block's int8 quants of weight rows n0 .. n0+15, as stored;
//   D (16×16): lane l holds D[4·(l/16) + r][l % 16], r = 0..3 — the three
//              limb dots of activation row 4g + l/16 against weight row
//              n0 + l%16 (r = 3 is zero).
// The lane combines its limbs and adds ldexp(d · (65536·c0 + 256·c1 + c2),
// E − 22) to its f32 accumulator, as the GEMV's matrix-core path does.
//
// Activations are prepared once per launch by k_gemm_x_prep into the A
// operand order ([chunk][block][group][lane] 8-byte entries, one coalesced
// dwordx2 per lane) plus the block exponents ([chunk][block][mm][group]).
#include "rt_formats.h"
#include "rt_shared.h"

typedef long i64_t;

struct GemmArgs {
    const uint8_t* w;     // N rows of nxb Q8_0 blocks
    const uint2* aops;    // prepared activations
    const int* etab;      // block exponents
    float* y;             // [M][N]
    uint32_t M, N, K, nxb, ksw;
    uint64_t row_bytes;
};

// Activation preparation: thread t → (chunk row r, block b, slice q of 4
// elements); 8 consecutive threads hold one block (limb_digits' lane group).
// Rows past M are zero.
template <int MG>
RT_DEV void gemm_prep_body(const float* __restrict__ x, uint32_t M, uint32_t K, uint32_t nchunks,
                           uint32_t* __restrict__ aops, int* __restrict__ etab,
                           float* __restrict__ stab) {
    const uint32_t nxb = K / 32;
    constexpr uint32_t ROWS = 4 * MG;
    const uint64_t total = (uint64_t)nchunks * ROWS * nxb * 8;
    for (uint64_t t = (uint64_t)blockIdx.x * wg_threads() + threadIdx.x; t < total;
         t += (uint64_t)gridDim.x * wg_threads()) {
        const uint32_t q = t & 7;
        const uint64_t rb = t >> 3;  // (chunk row, block) pair
        const uint32_t b = (uint32_t)(rb % nxb);
        const uint32_t rr = (uint32_t)(rb / nxb);  // chunk·ROWS + row
        const uint32_t ch = rr / ROWS, row = rr % ROWS;
        const uint32_t m = ch * ROWS + row;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (m < M) {
            const f32x4 xv = *(const f32x4*)(x + (size_t)m * K + (size_t)b * 32 + 4 * q);
            v[0] = xv.x; v[1] = xv.y; v[2] = xv.z; v[3] = xv.w;
        }
        int e;
        int l[3][4];
        limb_digits(v, e, l);
        const uint32_t g = row / 4, mm = row % 4;
        const uint32_t cq = q / 2;  // 8-element chunk of the block = MFMA k-group
        uint32_t* base = aops + (((size_t)ch * nxb + b) * MG + g) * 128;  // 64 lanes × 2 dwords
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lane = (4 * mm + k) + 16 * cq;
            base[lane * 2 + (q & 1)] = k < 3 ? pack_i8x4(l[k]) : 0u;
        }
        if (q == 0) etab[(((size_t)ch * nxb + b) * 4 + mm) * MG + g] = e;
        if (stab) {
            // Σx over the record as its limbs represent it (for formats with a
            // per-sub-block min): the 8 lanes of the record reduce their sums
            int sk[3];
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                int v2 = l[k][0] + l[k][1] + l[k][2] + l[k][3];
                v2 += __shfl_xor(v2, 1, 64);
                v2 += __shfl_xor(v2, 2, 64);
                v2 += __shfl_xor(v2, 4, 64);
                sk[k] = v2;
            }
            if (q == 0)
                stab[(((size_t)ch * nxb + b) * 4 + mm) * MG + g] =
                    __builtin_amdgcn_ldexpf(limb_combine(sk[0], sk[1], sk[2]), e - 22);
        }
    }
}
#define RT_GEMM_PREP(MG)                                                                       \
    extern "C" __global__ void __launch_bounds__(256) k_gemm_x_prep_mg##MG(                    \
        const float* x, uint32_t M, uint32_t K, uint32_t nchunks, uint32_t* aops, int* etab,   \
        float* stab) {                                                                         \
        gemm_prep_body<MG>(x, M, K, nchunks, aops, etab, stab);                                \
    }
RT_GEMM_PREP(1)
RT_GEMM_PREP(2)
RT_GEMM_PREP(4)
RT_GEMM_PREP(8)

template <int MG, int CT>
struct GemmBlk {
    uint32_t wq[CT][3];  // aligned dwords covering the lane's 8 quants
    uint32_t wd[CT];     // aligned dword holding the block scale
    uint2 A[MG];
    int E[MG];
};

// Workgroup = ksw waves sharing one group of 16·CT weight rows and one chunk
// of 4·MG activation rows; wave wk takes blocks wk, wk + ksw, ... and the
// waves' partial sums are added in wave order.
template <int MG, int CT, int DEPTH>
RT_DEV void gemm_body(const GemmArgs& a) {
    __shared__ float red[8][MG * CT][64];
    const uint32_t lane = threadIdx.x & 63, wk = threadIdx.x >> 6, ksw = a.ksw;
    const uint32_t j = lane & 15, c = lane >> 4;
    const uint32_t ch = blockIdx.y, n0 = blockIdx.x * 16 * CT;
    const uint32_t nxb = a.nxb;
    const uint2* ap = a.aops + (size_t)ch * nxb * MG * 64;
    const int* ep = a.etab + (size_t)ch * nxb * 4 * MG;
    const uint8_t* wrow[CT];
#pragma unroll
    for (int t = 0; t < CT; ++t) {
        const uint32_t n = min(n0 + 16 * t + j, a.N - 1);  // clamped rows are not stored
        wrow[t] = a.w + (size_t)n * a.row_bytes;
    }
    auto load = [&](uint32_t b, GemmBlk<MG, CT>& k) {
#pragma unroll
        for (int t = 0; t < CT; ++t) {
            const uint8_t* blk = wrow[t] + (size_t)b * 34;
            const uintptr_t p = (uintptr_t)(blk + 2 + 8 * c);
            const uint32_t* pq = (const uint32_t*)(p & ~(uintptr_t)3);
            k.wq[t][0] = pq[0];
            k.wq[t][1] = pq[1];
            // the third dword is needed only for a 2-byte offset; otherwise it
            // could lie past the end of the weights, so re-read the second
            k.wq[t][2] = pq[(p & 3) ? 2 : 1];
            k.wd[t] = *(const uint32_t*)((uintptr_t)blk & ~(uintptr_t)3);
        }
#pragma unroll
        for (int g = 0; g < MG; ++g) k.A[g] = ap[((size_t)b * MG + g) * 64 + lane];
        const int* e = ep + ((size_t)b * 4 + c) * MG;
#pragma unroll
        for (int g = 0; g < MG; ++g) k.E[g] = e[g];
    };
    float acc[MG][CT];
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int t = 0; t < CT; ++t) acc[g][t] = 0.0f;
    auto compute = [&](uint32_t b, const GemmBlk<MG, CT>& k) {
#pragma unroll
        for (int t = 0; t < CT; ++t) {
            const uintptr_t blk = (uintptr_t)(wrow[t] + (size_t)b * 34);
            const uint32_t sh = (uint32_t)((blk + 2) & 3);  // 0 or 2
            const uint32_t q0 = alignb(k.wq[t][1], k.wq[t][0], sh);
            const uint32_t q1 = alignb(k.wq[t][2], k.wq[t][1], sh);
            const i64_t B = (i64_t)(((uint64_t)q1 << 32) | q0);
            const float d = h2f((blk & 3) ? (k.wd[t] >> 16) : k.wd[t]);
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                const i64_t A = (i64_t)(((uint64_t)k.A[g].y << 32) | k.A[g].x);
                const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, v4i{0, 0, 0, 0}, 0, 0, 0);
                acc[g][t] += __builtin_amdgcn_ldexpf(d * comb4(C), k.E[g] - 22);
            }
        }
    };
    // DEPTH blocks in flight per wave; loads past the end are clamped (every
    // lane issues the same loads, so waits stay partial)
    GemmBlk<MG, CT> buf[DEPTH];
    const uint32_t last = nxb - 1;
#pragma unroll
    for (int h = 0; h < DEPTH; ++h) load(min(wk + h * ksw, last), buf[h]);
    for (uint32_t b0 = wk; b0 < nxb; b0 += DEPTH * ksw) {
#pragma unroll
        for (int h = 0; h < DEPTH; ++h) {
            const uint32_t b = b0 + h * ksw;
            if (b < nxb) {
                compute(b, buf[h]);
                load(min(b + DEPTH * ksw, last), buf[h]);
            }
        }
    }
    if (ksw > 1) {
#pragma unroll
        for (int g = 0; g < MG; ++g)
#pragma unroll
            for (int t = 0; t < CT; ++t) red[wk][g * CT + t][lane] = acc[g][t];
        __syncthreads();
        if (wk != 0) return;
#pragma unroll
        for (int g = 0; g < MG; ++g)
#pragma unroll
            for (int t = 0; t < CT; ++t) {
                float s = 0.0f;
                for (uint32_t w = 0; w < ksw; ++w) s += red[w][g * CT + t][lane];
                acc[g][t] = s;
            }
    }
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
        for (int t = 0; t < CT; ++t) {
            const uint32_t m = ch * 4 * MG + 4 * g + c, n = n0 + 16 * t + j;
            if (m < a.M && n < a.N) a.y[(size_t)m * a.N + n] = acc[g][t];
        }
}

// DEPTH: blocks in flight per wave (registers per block grow with MG)
#define RT_GEMM_KERNEL(MG, CT, DEPTH)                                                       \
    extern "C" __global__ void __launch_bounds__(512) k_gemm_q8_0_mg##MG##_ct##CT(GemmArgs a) { \
        gemm_body<MG, CT, DEPTH>(a);                                                        \
    }
RT_GEMM_KERNEL(1, 1, 8)
RT_GEMM_KERNEL(2, 1, 8)
RT_GEMM_KERNEL(4, 1, 4)
RT_GEMM_KERNEL(8, 1, 4)
RT_GEMM_KERNEL(1, 2, 8)
RT_GEMM_KERNEL(2, 2, 6)
RT_GEMM_KERNEL(4, 2, 4)
RT_GEMM_KERNEL(8, 2, 3)

// ───────────────────── LDS-staged variant (nxb % 8 == 0) ─────────────────────
//
// Workgroup of 4 waves = one tile of 64 weight rows (16 per wave).  The K
// range is streamed in stages of NB blocks (8, or 4 for large batches, which
// keeps the stage's activation operands small enough for 2+ workgroups per
// CU): the 64 row segments (NB·34 contiguous bytes each, 16- or 8-byte
// aligned), the stage's prepared activation operands and block exponents are
// loaded with coalesced loads, written to LDS, and consumed from there; the
// next stage's loads are in flight while the current one is computed (two
// LDS buffers).
//
// Work items (row tile, K split, activation chunk) are spread over a
// persistent grid.  With more than one K split, each item writes its partial
// sums; the last item of a (tile, chunk) to finish (arrival counter, reset by
// that item) adds the splits in split order and stores Y.
constexpr uint32_t GB_ROWS = 64;  // weight rows per tile

struct Gemm2Args {
    const uint8_t* w;
    const uint2* aops;
    const int* etab;
    const float* stab;    // per-record activation sums (formats with a min)
    float* y;
    float* part;          // [chunk][split][chunk rows][N] partial sums (splits > 1)
    uint32_t* counters;   // [chunk][tile], cstride u32 slots apart
    uint32_t M, N, nxb, tiles, splits, kbs, nchunks;  // nxb, kbs: in weight blocks
    uint64_t row_bytes;
    uint32_t cstride;
    // f16 form, unsplit launches: y = acc (+ f32(bias[n])) (+ res as res + y)
    const uint16_t* bias;
    const float* res;
};

// Block formats of the staged GEMM.  decode() gives, for record r of a
// stage (32 elements) and lane group c (elements 8c..8c+7), the 8 int8
// weight values in element order (the B operand), the record's scale and,
// for formats with a per-sub-block min, dmin·m (y += dsc·q·x − mn·Σx).
struct GemmQ8_0 {  // gemv_q8_0.metal:11-17
    static constexpr uint32_t BLK_BYTES = 34, RECS = 1;
    static constexpr bool HAS_MIN = false;
    RT_DEV static void decode(const uint8_t* row, uint32_t r, uint32_t c, i64_t& B, float& dsc,
                              float& mn, float&) {
        const uint32_t o = r * 34 + 2 + 8 * c;  // (row is 4-byte aligned)
        const uint32_t* pw = (const uint32_t*)(row + (o & ~3u));
        const uint32_t sh = o & 3;
        const uint32_t w0 = pw[0], w1 = pw[1], w2 = pw[sh ? 2 : 1];
        const uint32_t q0 = alignb(w1, w0, sh), q1 = alignb(w2, w1, sh);
        B = (i64_t)(((uint64_t)q1 << 32) | q0);
        dsc = h2f(*(const uint16_t*)(row + r * 34));
        mn = 0.0f;
    }
};
struct GemmQ4_0 {  // reference layout: byte i = elements 2i (low), 2i+1 (high)
    static constexpr uint32_t BLK_BYTES = 18, RECS = 1;
    static constexpr bool HAS_MIN = false;
    RT_DEV static void decode(const uint8_t* row, uint32_t r, uint32_t c, i64_t& B, float& dsc,
                              float& mn, float&) {
        const uint32_t off = r * 18 + 2 + 4 * c;  // bytes 4c..4c+3 of the quants
        const uint32_t* pw = (const uint32_t*)(row + (off & ~3u));
        const uint32_t w = alignb(pw[(off & 3) ? 1 : 0], pw[0], off & 3);
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
        // interleave (lo0 hi0 lo1 hi1) (lo2 hi2 lo3 hi3), then nib − 8 per byte
        const uint32_t e0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        const uint32_t e1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
        const uint32_t q0 = (e0 + 0x78787878u) ^ 0x80808080u;
        const uint32_t q1 = (e1 + 0x78787878u) ^ 0x80808080u;
        B = (i64_t)(((uint64_t)q1 << 32) | q0);
        dsc = h2f(*(const uint16_t*)(row + r * 18));
        mn = 0.0f;
    }
};
// Q4_K: record 2j = low nibbles of qs[32j..32j+31], record 2j+1 = high
// nibbles; reference layout: sub-blocks j and j + 4 (dequant.metal:77-95);
// ggml layout (G): sub-blocks 2j and 2j + 1.
template <bool G>
struct GemmQ4KT {
    static constexpr uint32_t BLK_BYTES = 144, RECS = 8;
    static constexpr bool HAS_MIN = true;
    RT_DEV static void decode(const uint8_t* row, uint32_t r, uint32_t c, i64_t& B, float& dsc,
                              float& mn, float&) {
        const uint8_t* blk = row + (r / 8) * 144;
        const uint32_t rec = r % 8, j = rec / 2, hi = rec & 1;
        const uint2 q = *(const uint2*)(blk + 16 + 32 * j + 8 * c);
        const uint32_t q0 = hi ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
        const uint32_t q1 = hi ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
        B = (i64_t)(((uint64_t)q1 << 32) | q0);
        const u32x4 hdr = *(const u32x4*)blk;
        uint32_t sc, m;
        kq_scale_min(G ? 2 * j + hi : (hi ? j + 4 : j), hdr.y, hdr.z, hdr.w, sc, m);
        dsc = h2f(hdr.x) * (float)sc;
        mn = h2f(hdr.x >> 16) * (float)m;
    }
};
using GemmQ4K = GemmQ4KT<false>;
using GemmQ4KG = GemmQ4KT<true>;

// Eight consecutive bytes at any 2-byte-aligned offset o of a 4-byte-aligned
// row (three aligned dwords and alignbyte).
RT_DEV void gemm_bytes8(const uint8_t* row, uint32_t o, uint32_t& q0, uint32_t& q1) {
    const uint32_t* pw = (const uint32_t*)(row + (o & ~3u));
    const uint32_t sh = o & 3;
    const uint32_t w0 = pw[0], w1 = pw[1], w2 = pw[sh ? 2 : 1];
    q0 = alignb(w1, w0, sh);
    q1 = alignb(w2, w1, sh);
}

// Q4_0, ggml layout: element j < 16 = qs[j] & 15, 16 + j = qs[j] >> 4 (d·(q − 8)).
struct GemmQ4_0G {
    static constexpr uint32_t BLK_BYTES = 18, RECS = 1;
    static constexpr bool HAS_MIN = false;
    RT_DEV static void decode(const uint8_t* row, uint32_t r, uint32_t c, i64_t& B, float& dsc,
                              float& mn, float&) {
        uint32_t w0, w1;
        gemm_bytes8(row, r * 18 + 2 + 8 * (c & 1), w0, w1);
        const uint32_t s = 4 * (c >> 1);
        const uint32_t q0 = (((w0 >> s) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
        const uint32_t q1 = (((w1 >> s) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u;
        B = (i64_t)(((uint64_t)q1 << 32) | q0);
        dsc = h2f(*(const uint16_t*)(row + r * 18));
        mn = 0.0f;
    }
};

// Q5_0 (forward.rs:900-920): element j < 16 = (qs[j] & 15) | (qh bit j) << 4,
// 16 + j = (qs[j] >> 4) | (qh bit 16 + j) << 4, value d·(q − 16).  Lane group c
// holds elements 8c..8c+7, whose fifth bits are qh bits 8c..8c+7.
struct GemmQ5_0 {
    static constexpr uint32_t BLK_BYTES = 22, RECS = 1;
    static constexpr bool HAS_MIN = false;
    RT_DEV static void decode(const uint8_t* row, uint32_t r, uint32_t c, i64_t& B, float& dsc,
                              float& mn, float&) {
        uint32_t w0, w1, qh, unused;
        gemm_bytes8(row, r * 22 + 6 + 8 * (c & 1), w0, w1);
        gemm_bytes8(row, r * 22 + 2, qh, unused);
        const uint32_t s = 4 * (c >> 1);
        const uint32_t hb = (qh >> (8 * c)) & 255u;
        const uint32_t q0 = ((w0 >> s) & 0x0F0F0F0Fu) | (spread4(hb & 15u) << 4);
        const uint32_t q1 = ((w1 >> s) & 0x0F0F0F0Fu) | (spread4(hb >> 4) << 4);
        // q − 16 per byte (q ≤ 31: no carry between bytes)
        B = (i64_t)(((uint64_t)((q1 + 0x70707070u) ^ 0x80808080u) << 32) |
                    ((q0 + 0x70707070u) ^ 0x80808080u));
        dsc = h2f(*(const uint16_t*)(row + r * 22));
        mn = 0.0f;
    }
};

// Q5_K (176 B: d, dmin @0, scales[12] @4, qh[32] @16, qs[128] @48): record
// 2j = low nibbles of qs[32j..], 2j+1 = high nibbles, v = d·sc·q − dmin·m.
// Fifth bit of element e = 64j + 32·hi + l: reference layout bit e%8 of
// qh[e/8] (forward.rs:979-1012), sub-blocks (j, j+4); ggml layout (G) bit
// 2j + hi of qh[l], sub-blocks (2j, 2j+1).
template <bool G>
struct GemmQ5KT {
    static constexpr uint32_t BLK_BYTES = 176, RECS = 8;
    static constexpr bool HAS_MIN = true;
    RT_DEV static void decode(const uint8_t* row, uint32_t r, uint32_t c, i64_t& B, float& dsc,
                              float& mn, float&) {
        const uint8_t* blk = row + (r / 8) * 176;
        const uint32_t rec = r % 8, j = rec / 2, hi = rec & 1;
        const uint2 q = *(const uint2*)(blk + 48 + 32 * j + 8 * c);
        const uint32_t n0 = hi ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
        const uint32_t n1 = hi ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
        uint32_t h0, h1;
        if (G) {
            const uint2 h = *(const uint2*)(blk + 16 + 8 * c);  // qh[l], l = 8c..8c+7
            h0 = ((h.x >> (2 * j + hi)) & 0x01010101u) << 4;
            h1 = ((h.y >> (2 * j + hi)) & 0x01010101u) << 4;
        } else {
            const uint32_t hb = blk[16 + 8 * j + 4 * hi + c];  // bits of elements 8c..8c+7
            h0 = spread4(hb & 15u) << 4;
            h1 = spread4(hb >> 4) << 4;
        }
        B = (i64_t)(((uint64_t)(n1 | h1) << 32) | (n0 | h0));
        const u32x4 hdr = *(const u32x4*)blk;
        uint32_t sc, m;
        kq_scale_min(G ? 2 * j + hi : (hi ? j + 4 : j), hdr.y, hdr.z, hdr.w, sc, m);
        dsc = h2f(hdr.x) * (float)sc;
        mn = h2f(hdr.x >> 16) * (float)m;
    }
};
using GemmQ5K = GemmQ5KT<false>;
using GemmQ5KG = GemmQ5KT<true>;

// Q6_K (210 B: ql[128] @0, qh[64] @128, sc[16] @192, d @208), staged two
// super-blocks at a time (420 bytes keep 4-byte alignment).  Record r = 4·hs
// + t of a super-block holds elements 128·hs + 32t + l:
//   ((ql[64hs + l + 32(t&1)] >> 4(t>>1)) & 15) | (((qh[32hs + l] >> 2t) & 3) << 4)
// minus 32, times d·sc[8hs + 2t] (reference layout, forward.rs:921-950); the
// ggml layout (G) scales elements 16..31 of the record by sc[8hs + 2t + 1].
template <bool G>
struct GemmQ6KT {
    static constexpr uint32_t BLK_BYTES = 210, RECS = 8;
    static constexpr bool HAS_MIN = false;
    static constexpr bool SPLIT16 = G;
    RT_DEV static void decode(const uint8_t* row, uint32_t r, uint32_t c, i64_t& B, float& dsc,
                              float& mn, float& dsc2) {
        const uint32_t b = r / 8, rec = r % 8, hs = rec / 4, t = rec % 4;
        const uint32_t o = b * 210;  // block start (2-byte aligned)
        uint32_t l0, l1, h0, h1;
        gemm_bytes8(row, o + 64 * hs + 32 * (t & 1) + 8 * c, l0, l1);
        gemm_bytes8(row, o + 128 + 32 * hs + 8 * c, h0, h1);
        const uint32_t s = 4 * (t >> 1);
        const uint32_t q0 = ((l0 >> s) & 0x0F0F0F0Fu) | (((h0 >> (2 * t)) & 0x03030303u) << 4);
        const uint32_t q1 = ((l1 >> s) & 0x0F0F0F0Fu) | (((h1 >> (2 * t)) & 0x03030303u) << 4);
        // q − 32 per byte (q ≤ 63: no carry between bytes)
        B = (i64_t)(((uint64_t)((q1 + 0x60606060u) ^ 0x80808080u) << 32) |
                    ((q0 + 0x60606060u) ^ 0x80808080u));
        uint32_t sw, unused;
        gemm_bytes8(row, o + 192 + 8 * hs + 2 * t, sw, unused);  // sc[8hs + 2t], sc[8hs + 2t + 1]
        uint32_t dw;
        gemm_bytes8(row, o + 208, dw, unused);
        const float d = h2f(dw);
        dsc = d * (float)(int8_t)(sw & 255u);
        dsc2 = G ? d * (float)(int8_t)((sw >> 8) & 255u) : dsc;
        mn = 0.0f;
    }
    // Records 4·r4 .. 4·r4 + 3 (super-block r4 / 2, half r4 % 2, t = 0..3) at
    // once: they share their qh bytes, t and t + 2 their ql bytes, and all
    // four their scale window and d, so the bytes are read once (5 reads of
    // 8 bytes instead of 16).
    static constexpr bool DECODE4 = true;
    RT_DEV static void decode4(const uint8_t* row, uint32_t r4, uint32_t c, i64_t B[4], float dsc[4],
                               float dsc2[4]) {
        const uint32_t b = r4 / 2, hs = r4 % 2;
        const uint32_t o = b * 210;
        uint32_t la0, la1, lb0, lb1, h0, h1, sw0, sw1, dw, unused;
        gemm_bytes8(row, o + 64 * hs + 8 * c, la0, la1);        // ql of t = 0, 2
        gemm_bytes8(row, o + 64 * hs + 32 + 8 * c, lb0, lb1);   // ql of t = 1, 3
        gemm_bytes8(row, o + 128 + 32 * hs + 8 * c, h0, h1);    // qh of t = 0..3
        gemm_bytes8(row, o + 192 + 8 * hs, sw0, sw1);           // sc[8hs .. 8hs + 7]
        gemm_bytes8(row, o + 208, dw, unused);
        const float d = h2f(dw);
#pragma unroll
        for (uint32_t t = 0; t < 4; ++t) {
            const uint32_t l0 = (t & 1) ? lb0 : la0, l1 = (t & 1) ? lb1 : la1;
            const uint32_t s = 4 * (t >> 1);
            const uint32_t q0 = ((l0 >> s) & 0x0F0F0F0Fu) | (((h0 >> (2 * t)) & 0x03030303u) << 4);
            const uint32_t q1 = ((l1 >> s) & 0x0F0F0F0Fu) | (((h1 >> (2 * t)) & 0x03030303u) << 4);
            B[t] = (i64_t)(((uint64_t)((q1 + 0x60606060u) ^ 0x80808080u) << 32) |
                           ((q0 + 0x60606060u) ^ 0x80808080u));
            const uint32_t sw = (t >> 1) ? sw1 : sw0;           // sc[8hs + 2t] at byte 2(t & 1)
            const uint32_t sb = sw >> (16 * (t & 1));
            dsc[t] = d * (float)(int8_t)(sb & 255u);
            dsc2[t] = G ? d * (float)(int8_t)((sb >> 8) & 255u) : dsc[t];
        }
    }
};
using GemmQ6K = GemmQ6KT<false>;
using GemmQ6KG = GemmQ6KT<true>;

// Formats whose record carries one scale per 16 elements (ggml Q6_K) set
// SPLIT16: the record then takes two MFMAs, each with the other half's
// weights zeroed, scaled by dsc and dsc2.
template <class P, class = void>
struct GemmSplit16 {
    static constexpr bool value = false;
};
template <class P>
struct GemmSplit16<P, decltype((void)P::SPLIT16)> {
    static constexpr bool value = P::SPLIT16;
};
// formats whose records come four at a time from shared bytes (decode4)
template <class P, class = void>
struct GemmDecode4 {
    static constexpr bool value = false;
};
template <class P>
struct GemmDecode4<P, decltype((void)P::DECODE4)> {
    static constexpr bool value = P::DECODE4;
};

template <class P, int MG, int NB, int WAVES = 4>
RT_DEV void gemm2_body(const Gemm2Args& a) {
    // WAVES waves of 16 weight rows each share one stage of activation operands
    constexpr uint32_t T = 64 * WAVES, ROWS = 16 * WAVES;
    constexpr uint32_t NR = NB * P::RECS;                  // records per stage
    constexpr uint32_t SEG = NB * P::BLK_BYTES;            // bytes of a row segment
    constexpr uint32_t VB = SEG % 16 == 0 ? 16 : (SEG % 8 == 0 ? 8 : 4);  // bytes per W load
    typedef typename std::conditional<VB == 16, u32x4,
                                      typename std::conditional<VB == 8, uint2, uint32_t>::type>::type WV;
    constexpr uint32_t WPR = SEG / VB;                     // W loads per row segment
    constexpr uint32_t WV_N = ROWS * WPR;               // W loads per stage
    constexpr uint32_t AV4 = NR * MG * 64 * 8 / 16;        // dwordx4 of A per stage
    constexpr uint32_t EV4 = NR * 4 * MG * 4 / 16;         // dwordx4 of E (and of S) per stage
    constexpr uint32_t WPT = (WV_N + T - 1) / T;           // W loads per thread
    constexpr uint32_t APT = (AV4 + T - 1) / T;
    static_assert(SEG % VB == 0 && EV4 <= T, "segment alignment");
    __shared__ WV lw[2][WV_N];
    __shared__ u32x4 la[2][AV4];
    __shared__ u32x4 le[2][EV4 > 0 ? EV4 : 1];
    __shared__ u32x4 ls[P::HAS_MIN ? 2 : 1][P::HAS_MIN ? EV4 : 1];
    __shared__ uint32_t last_flag;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t j = lane & 15, c = lane >> 4;
    const uint32_t nitems = a.tiles * a.splits * a.nchunks;

    for (uint32_t item = blockIdx.x; item < nitems; item += gridDim.x) {
        const uint32_t tile = item % a.tiles;
        const uint32_t split = (item / a.tiles) % a.splits;
        const uint32_t ch = item / (a.tiles * a.splits);
        const uint32_t kb0 = split * a.kbs;
        const uint32_t kb1 = min(a.nxb, kb0 + a.kbs);
        const uint32_t nst = (kb1 - kb0) / NB;
        const uint32_t row0 = tile * ROWS;
        const uint32_t nrec = a.nxb * P::RECS;
        const uint2* ap = a.aops + (size_t)ch * nrec * MG * 64;
        const int* ep = a.etab + (size_t)ch * nrec * 4 * MG;
        const float* sp = P::HAS_MIN ? a.stab + (size_t)ch * nrec * 4 * MG : nullptr;

        WV rw[WPT];
        u32x4 ra[APT], re, rs;
        auto gload = [&](uint32_t st) {
            const uint32_t b0 = kb0 + st * NB;  // first block of the stage
            const uint32_t r0 = b0 * P::RECS;   // its first record
#pragma unroll
            for (uint32_t i = 0; i < WPT; ++i) {
                uint32_t f = tid + T * i;
                if (f >= WV_N) f = WV_N - 1;  // duplicate load, not stored
                const uint32_t r = f / WPR, col = f % WPR;
                const uint32_t n = min(row0 + r, a.N - 1);
                rw[i] = *(const WV*)(a.w + (size_t)n * a.row_bytes + (size_t)b0 * P::BLK_BYTES + col * VB);
            }
            const u32x4* as = (const u32x4*)(ap + (size_t)r0 * MG * 64);
#pragma unroll
            for (uint32_t i = 0; i < APT; ++i) ra[i] = as[min(tid + T * i, AV4 - 1)];
            re = ((const u32x4*)(ep + (size_t)r0 * 4 * MG))[min(tid, EV4 - 1)];
            if (P::HAS_MIN) rs = ((const u32x4*)(sp + (size_t)r0 * 4 * MG))[min(tid, EV4 - 1)];
        };
        auto lstore = [&](uint32_t buf) {
#pragma unroll
            for (uint32_t i = 0; i < WPT; ++i)
                if (tid + T * i < WV_N) lw[buf][tid + T * i] = rw[i];
#pragma unroll
            for (uint32_t i = 0; i < APT; ++i)
                if (tid + T * i < AV4) la[buf][tid + T * i] = ra[i];
            if (tid < EV4) le[buf][tid] = re;
            if (P::HAS_MIN && tid < EV4) ls[P::HAS_MIN ? buf : 0][tid] = rs;
        };
        float acc[MG];
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[g] = 0.0f;
        const uint32_t wrow = (16 * wv + j) * SEG;  // this lane's row in a W buffer
        auto compute = [&](uint32_t buf) {
            const uint8_t* wb = (const uint8_t*)lw[buf] + wrow;
            const uint2* ab = (const uint2*)la[buf];
            const int* eb = (const int*)le[buf];
            const float* sb = (const float*)ls[P::HAS_MIN ? buf : 0];
            // record r of the stage from its decoded codes B and scales
            auto record = [&](uint32_t r, i64_t B, float dsc, float mn, float dsc2) {
                // all of the record's matrix-core products first, then their
                // epilogues (independent MFMAs overlap in the pipeline)
                v4i C[MG], C2[GemmSplit16<P>::value ? MG : 1];
                const i64_t Blo = (GemmSplit16<P>::value && c >= 2) ? 0 : B;  // elements 0..15
#pragma unroll
                for (int g = 0; g < MG; ++g) {
                    const uint2 av = ab[(r * MG + g) * 64 + lane];
                    const i64_t A = (i64_t)(((uint64_t)av.y << 32) | av.x);
                    C[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, Blo, v4i{0, 0, 0, 0}, 0, 0, 0);
                    if (GemmSplit16<P>::value)
                        C2[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, c >= 2 ? B : 0, v4i{0, 0, 0, 0},
                                                                      0, 0, 0);
                }
#pragma unroll
                for (int g = 0; g < MG; ++g) {
                    const uint32_t ei = (r * 4 + c) * MG + g;
                    float t = dsc * comb4(C[g]);
                    if (GemmSplit16<P>::value) t += dsc2 * comb4(C2[GemmSplit16<P>::value ? g : 0]);
                    float v = __builtin_amdgcn_ldexpf(t, eb[ei] - 22);
                    if (P::HAS_MIN) v -= mn * sb[ei];
                    acc[g] += v;
                }
            };
            if constexpr (GemmDecode4<P>::value) {
#pragma unroll 1
                for (uint32_t r4 = 0; r4 < NR / 4; ++r4) {
                    i64_t B4[4];
                    float ds4[4], ds24[4];
                    P::decode4(wb, r4, c, B4, ds4, ds24);
#pragma unroll
                    for (uint32_t q = 0; q < 4; ++q) record(4 * r4 + q, B4[q], ds4[q], 0.0f, ds24[q]);
                }
            } else {
#pragma unroll 2
                for (uint32_t r = 0; r < NR; ++r) {
                    i64_t B;
                    float dsc, mn, dsc2 = 0.0f;
                    P::decode(wb, r, c, B, dsc, mn, dsc2);
                    record(r, B, dsc, mn, dsc2);
                }
            }
        };
        if (nst > 0) {
            gload(0);
            lstore(0);
        }
        __syncthreads();
        for (uint32_t st = 0; st < nst; ++st) {
            const bool more = st + 1 < nst;
            if (more) gload(st + 1);
            compute(st & 1);
            if (more) lstore((st + 1) & 1);
            __syncthreads();
        }
        // results: lane holds (activation row ch·4MG + 4g + c, weight row row0 + 16wv + j)
        const uint32_t n = row0 + 16 * wv + j;
        if (a.splits == 1) {
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                const uint32_t m = ch * 4 * MG + 4 * g + c;
                if (m < a.M && n < a.N) a.y[(size_t)m * a.N + n] = acc[g];
            }
            continue;
        }
        const size_t crow = (size_t)4 * MG;  // rows of a chunk
#pragma unroll
        for (int g = 0; g < MG; ++g) {
            const size_t pr = ((size_t)(ch * a.splits + split) * crow + 4 * g + c);
            if (n < a.N) {
                if (a.counters) dev_store(a.part + pr * a.N + n, acc[g]);
                else a.part[pr * a.N + n] = acc[g];
            }
        }
        if (!a.counters) continue;  // partial sums only: k_gemm_split_sum adds them
        dev_stores_done();
        __syncthreads();
        uint32_t* counter = a.counters + ((size_t)ch * a.tiles + tile) * a.cstride;
        if (tid == 0) last_flag = arrive(counter) == a.splits - 1;
        __syncthreads();
        if (!last_flag) continue;
        if (n < a.N) {
#pragma unroll
            for (int g = 0; g < MG; ++g) {
                const uint32_t m = ch * 4 * MG + 4 * g + c;
                float s = 0.0f;
                for (uint32_t sp = 0; sp < a.splits; ++sp)
                    s += dev_load(a.part + ((size_t)(ch * a.splits + sp) * crow + 4 * g + c) * a.N + n);
                if (m < a.M) a.y[(size_t)m * a.N + n] = s;
            }
        }
        if (tid == 0) dev_store(counter, 0u);  // ready for the next call (also under graph replay)
        __syncthreads();
    }
}
// ───────────── f16 matrix-core variant (v_mfma_f32_16x16x32_f16) ─────────────
//
// Same stages, tiles, splits and decode policies as gemm2_body; the dot runs
// on f16 operands with f32 accumulation, 8 activation rows per MFMA:
//   A (16×32): row 2·mm + part = part (0: hi, 1: lo) of activation row
//              8g + mm, scaled by 2^-e per activation row so that the row's
//              largest |x| lies in [2^14, 2^15): hi = f16(x·2^-e), lo =
//              f16(x·2^-e − hi), which together carry ~22 bits of each
//              element (elements below 2^-24·2^e in the scaled units are
//              carried to 2^-24·2^e absolute: f16 subnormals);
//   B (32×16): the record's integer weight codes (|q| ≤ 128) as f16, exact;
//   D (16×16): lane l holds D[4·(l/16) + r][l % 16]: hi and lo dots of
//              activation rows 8g + 2·(l/16) (r = 0, 1) and 8g + 2·(l/16) + 1
//              (r = 2, 3) against weight row l % 16.
// Per record the lane adds dsc·(hi + lo) − mn·Σx for its two activation
// rows; the row's 2^e scales the sum once, after the last record (a per-row
// exponent removes the per-record scaling: Q8_0 18944×3584 at M = 32
// 44.5 → 40.0 µs).
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// 8 signed int8 codes → 8 exact f16: byte u = q + 128 becomes the f16 bits
// 0x64uu = 1024 + u, then 1152 is subtracted (both exact in f16).
RT_DEV h8_t gemm_i8x8_to_h8(i64_t B) {
    const uint32_t lo = (uint32_t)(uint64_t)B ^ 0x80808080u;
    const uint32_t hi = (uint32_t)((uint64_t)B >> 32) ^ 0x80808080u;
    uint32_t w[4];
    w[0] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);
    w[1] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);
    w[2] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);
    w[3] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);
    h8_t r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2_t v = __builtin_bit_cast(h2_t, w[i]) - h2_t{(_Float16)1152.0f, (_Float16)1152.0f};
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

// Activation preparation of the f16 variant: workgroup (m, q) takes padded
// activation row m and the q-th of its gridDim.y record ranges.  The row's
// largest |x| (read whole by every workgroup of the row) sets its exponent e
// (etab[m], written by q = 0): 2^-e brings it into [2^14, 2^15).  Then thread
// t → (record, k-group of 8 elements), the 4 threads of a record neighbours:
// hi = f16(x·2^-e), lo = f16(x·2^-e − hi) in the A order ([chunk][record]
// [group][lane] 16-byte entries) and, for formats with a min, the records'
// sums of the scaled values ([chunk][record][row][group]).  Rows past M are
// zero (e = 0).
template <int MG>
RT_DEV void gemm_xh_prep_body(const float* __restrict__ x, uint32_t M, uint32_t K, uint32_t nchunks,
                              u32x4* __restrict__ aops, int* __restrict__ etab,
                              float* __restrict__ stab) {
    constexpr uint32_t ROWS = 8 * MG;
    __shared__ float red[16];
    const uint32_t nrec = K / 32;
    const uint32_t m = blockIdx.x;  // padded row
    const uint32_t ch = m / ROWS, rr = m % ROWS, g = rr / 8, mm = rr % 8;
    const uint32_t tid = threadIdx.x, T = wg_threads();
    const float* xr = x + (size_t)(m < M ? m : 0) * K;
    float mx = 0.0f;
    if (m < M)
        for (uint32_t i0 = tid * 4; i0 < K; i0 += T * 32) {  // 8 loads in flight per thread
            f32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t i = i0 + u * T * 4;
                v[u] = i < K ? *(const f32x4*)(xr + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
        }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = 0.0f;
    for (uint32_t w = 0; w < (T >> 6); ++w) mx = fmaxf(mx, red[w]);
    const int e = mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) - 15 : 0;
    if (tid == 0 && blockIdx.y == 0) etab[m] = e;
    const uint32_t per = (nrec + gridDim.y - 1) / gridDim.y;
    const uint32_t r0 = blockIdx.y * per, r1 = min(nrec, r0 + per);
    for (uint32_t t = r0 * 4 + tid; t < r1 * 4; t += T) {  // (groups of 4 lanes share a trip count)
        const uint32_t kc = t & 3, rec = t >> 2;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (m < M) {
            const f32x4* xp = (const f32x4*)(xr + (size_t)rec * 32 + 8 * kc);
            const f32x4 a = xp[0], b = xp[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
        h8_t hv, lv;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xs = __builtin_amdgcn_ldexpf(v[i], -e);
            const _Float16 h = (_Float16)xs;
            hv[i] = h;
            lv[i] = (_Float16)(xs - (float)h);
            sum += xs;
        }
        u32x4* base = aops + (((size_t)ch * nrec + rec) * MG + g) * 64;
        base[2 * mm + 16 * kc] = __builtin_bit_cast(u32x4, hv);
        base[2 * mm + 1 + 16 * kc] = __builtin_bit_cast(u32x4, lv);
        if (stab) {
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            if (kc == 0) stab[(((size_t)ch * nrec + rec) * 8 + mm) * MG + g] = sum;
        }
    }
}
#define RT_GEMM_XH_PREP(MG)                                                                    \
    extern "C" __global__ void __launch_bounds__(1024) k_gemm_xh_prep_mg##MG(                  \
        const float* x, uint32_t M, uint32_t K, uint32_t nchunks, u32x4* aops, int* etab,      \
        float* stab) {                                                                         \
        gemm_xh_prep_body<MG>(x, M, K, nchunks, aops, etab, stab);                             \
    }
// One-pass form (K ≤ 20,480): workgroup m holds its row in registers
// (thread t: float4s t, t + 1024, ...), reduces the row's largest |x|, then
// writes each float4 as half of a 16-byte A entry (hi, lo) — one round trip
// to memory instead of three.
// The row of a preparation given as the K-split partial sums of the GEMM
// that produced it ([chunk][split][crow][K], as k_gemm_split_sum reads
// them): x = Σ part (SILU: silu(Σ part)·Σ part2), then res + x; written to y
// when given.
struct PrepSum {
    const float* part;
    const float* part2;
    const float* res;
    float* y;
    uint32_t splits, crow;
};

// The row of a preparation given as the split partials of the multi-query
// attention (k_attn_mq_f32_hd*, parts-only, one sequence): element (head h,
// d) of row r is column qi = r·G + h mod G of KV head h / G, merged over the
// nsp key ranges as that kernel's last workgroup merges them.
struct PrepAttn {
    const float* part;
    const float* ml;
    uint32_t nsp, G, hd, cgs;
};

template <int MG, bool NORM = false, bool SUM = false, bool ATT = false>
RT_DEV void gemm_xh_prep1_body(const float* __restrict__ x, uint32_t M, uint32_t K,
                               uint2* __restrict__ aops, int* __restrict__ etab,
                               float* __restrict__ stab, const float* __restrict__ gamma = nullptr,
                               float eps = 0.0f, float* __restrict__ xn = nullptr,
                               const PrepSum* ps = nullptr, const PrepAttn* pa = nullptr) {
    constexpr uint32_t ROWS = 8 * MG, T = 1024, NPT = 5;
    __shared__ float red[16];
    const uint32_t nrec = K / 32, nf = K / 4;
    const uint32_t m = blockIdx.x;
    const uint32_t ch = m / ROWS, rr = m % ROWS, g = rr / 8, mm = rr % 8;
    const uint32_t tid = threadIdx.x;
    f32x4 v[NPT];
    float mx = 0.0f;
    if constexpr (ATT) {
        const float NEG = -__builtin_huge_valf();
#pragma unroll
        for (uint32_t i = 0; i < NPT; ++i) {
            const uint32_t f = tid + T * i;
            f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
            if (m < M && f < nf) {
                const uint32_t h = 4 * f / pa->hd, d = 4 * f % pa->hd, kvh = h / pa->G;
                const uint32_t qi = m * pa->G + h % pa->G, cg = qi / 16, col = qi % 16;
                const size_t pair = (size_t)kvh * pa->cgs + cg;
                const float* mlv = pa->ml + (pair * pa->nsp * 16 + col) * 2;
                // every range's (max, sum) and partial issued before the
                // first is used (ranges past nsp read range 0, weight 0)
                float mj[RT_ATTN_MQ_NSP_MAX], lj[RT_ATTN_MQ_NSP_MAX];
                f32x4 pj[RT_ATTN_MQ_NSP_MAX];
#pragma unroll
                for (uint32_t j = 0; j < RT_ATTN_MQ_NSP_MAX; ++j) {
                    const uint32_t jj = j < pa->nsp ? j : 0;
                    mj[j] = mlv[32 * jj];
                    lj[j] = mlv[32 * jj + 1];
                    pj[j] = *(const f32x4*)(pa->part + ((pair * pa->nsp + jj) * 16 + col) * pa->hd + d);
                }
                float Mx = NEG;
#pragma unroll
                for (uint32_t j = 0; j < RT_ATTN_MQ_NSP_MAX; ++j) Mx = fmaxf(Mx, mj[j]);
                float L = 0.0f;
#pragma unroll
                for (uint32_t j = 0; j < RT_ATTN_MQ_NSP_MAX; ++j) {
                    const float w = (j >= pa->nsp || mj[j] == NEG) ? 0.0f : expf(mj[j] - Mx);
                    L += w * lj[j];
                    o += w * pj[j];
                }
                o = o / L;
            }
            v[i] = o;
        }
    } else if constexpr (SUM) {
        const uint32_t mc = m < M ? m : 0, sch = mc / ps->crow, sr = mc % ps->crow;
        const size_t off = ((size_t)sch * ps->splits * ps->crow + sr) * K, ss = (size_t)ps->crow * K;
#pragma unroll
        for (uint32_t i = 0; i < NPT; ++i) {
            const uint32_t f = tid + T * i;
            f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
            if (m < M && f < nf) {
                t = *(const f32x4*)(ps->part + off + 4 * f);
                for (uint32_t sp = 1; sp < ps->splits; ++sp) t += *(const f32x4*)(ps->part + off + sp * ss + 4 * f);
                if (ps->part2) {
                    f32x4 u = *(const f32x4*)(ps->part2 + off + 4 * f);
                    for (uint32_t sp = 1; sp < ps->splits; ++sp)
                        u += *(const f32x4*)(ps->part2 + off + sp * ss + 4 * f);
                    t = f32x4{t.x / (1.0f + expf(-t.x)) * u.x, t.y / (1.0f + expf(-t.y)) * u.y,
                              t.z / (1.0f + expf(-t.z)) * u.z, t.w / (1.0f + expf(-t.w)) * u.w};
                }
                if (ps->res) t = *(const f32x4*)(ps->res + (size_t)m * K + 4 * f) + t;
                if (ps->y) *(f32x4*)(ps->y + (size_t)m * K + 4 * f) = t;
            }
            v[i] = t;
        }
    } else {
        const float* xr = x + (size_t)(m < M ? m : 0) * K;
#pragma unroll
        for (uint32_t i = 0; i < NPT; ++i) {
            const uint32_t f = tid + T * i;
            v[i] = (m < M && f < nf) ? *(const f32x4*)(xr + 4 * f) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    if constexpr (NORM) {
        // rms_norm_f32_f32_f32g of the row first: x · rsqrt(mean(x²) + eps) · γ,
        // also written to xn (the rows past M stay zero)
        __shared__ float red2[16];
        float ss = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < NPT; ++i)
            ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if ((tid & 63) == 0) red2[tid >> 6] = ss;
        __syncthreads();
        ss = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < T / 64; ++w) ss += red2[w];
        const float rms = rsqrtf(ss / (float)K + eps);
#pragma unroll
        for (uint32_t i = 0; i < NPT; ++i) {
            const uint32_t f = tid + T * i;
            if (m < M && f < nf) {
                const f32x4 gv = *(const f32x4*)(gamma + 4 * f);
                v[i] = f32x4{v[i].x * rms * gv.x, v[i].y * rms * gv.y, v[i].z * rms * gv.z,
                             v[i].w * rms * gv.w};
                if (xn) *(f32x4*)(xn + (size_t)m * K + 4 * f) = v[i];
            }
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < NPT; ++i)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < T / 64; ++w) mx = fmaxf(mx, red[w]);
    const int e = mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) - 15 : 0;
    if (tid == 0) etab[m] = e;
#pragma unroll
    for (uint32_t i = 0; i < NPT; ++i) {
        const uint32_t f = tid + T * i;
        if (f >= nf) break;  // (the 8 lanes of a record share this)
        const uint32_t rec = f >> 3, qf = f & 7, kc = qf >> 1, half = qf & 1;
        const float xs[4] = {__builtin_amdgcn_ldexpf(v[i].x, -e), __builtin_amdgcn_ldexpf(v[i].y, -e),
                             __builtin_amdgcn_ldexpf(v[i].z, -e), __builtin_amdgcn_ldexpf(v[i].w, -e)};
        _Float16 h[4], l[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            h[u] = (_Float16)xs[u];
            l[u] = (_Float16)(xs[u] - (float)h[u]);
        }
        // 16-byte entries 2·mm (hi) and 2·mm + 1 (lo) of k-group kc: this
        // float4 is their half `half`
        uint2* base = aops + ((((size_t)ch * nrec + rec) * MG + g) * 64 + 16 * kc + 2 * mm) * 2 + half;
        base[0] = uint2{(uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16),
                        (uint32_t)__builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16)};
        base[2] = uint2{(uint32_t)__builtin_bit_cast(uint16_t, l[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, l[1]) << 16),
                        (uint32_t)__builtin_bit_cast(uint16_t, l[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, l[3]) << 16)};
        if (stab) {
            float sum = xs[0] + xs[1] + xs[2] + xs[3];
            sum += __shfl_xor(sum, 1, 64);
            sum += __shfl_xor(sum, 2, 64);
            sum += __shfl_xor(sum, 4, 64);
            if (qf == 0) stab[(((size_t)ch * nrec + rec) * 8 + mm) * MG + g] = sum;
        }
    }
}
#define RT_GEMM_XH_PREP1(MG)                                                                   \
    extern "C" __global__ void __launch_bounds__(1024) k_gemm_xh_prep1_mg##MG(                 \
        const float* x, uint32_t M, uint32_t K, uint2* aops, int* etab, float* stab) {         \
        gemm_xh_prep1_body<MG>(x, M, K, aops, etab, stab);                                     \
    }
RT_GEMM_XH_PREP1(1)
RT_GEMM_XH_PREP1(2)
RT_GEMM_XH_PREP1(4)
// the same preparation of RMSNorm(x)·γ, the normalised rows also written to
// xn (when given)
#define RT_GEMM_XH_PREP1N(MG)                                                                  \
    extern "C" __global__ void __launch_bounds__(1024) k_gemm_xh_prep1n_mg##MG(                \
        const float* x, uint32_t M, uint32_t K, uint2* aops, int* etab, float* stab,           \
        const float* gamma, float eps, float* xn) {                                            \
        gemm_xh_prep1_body<MG, true>(x, M, K, aops, etab, stab, gamma, eps, xn);               \
    }
RT_GEMM_XH_PREP1N(1)
RT_GEMM_XH_PREP1N(2)
RT_GEMM_XH_PREP1N(4)
// the preparation of a row given as a GEMM's partial sums (PrepSum), plain or
// RMS-normalised
#define RT_GEMM_XH_PREP1S(MG)                                                                  \
    extern "C" __global__ void __launch_bounds__(1024) k_gemm_xh_prep1s_mg##MG(                \
        PrepSum ps, uint32_t M, uint32_t K, uint2* aops, int* etab, float* stab) {             \
        gemm_xh_prep1_body<MG, false, true>(nullptr, M, K, aops, etab, stab, nullptr, 0.0f,    \
                                            nullptr, &ps);                                     \
    }                                                                                          \
    extern "C" __global__ void __launch_bounds__(1024) k_gemm_xh_prep1sn_mg##MG(               \
        PrepSum ps, uint32_t M, uint32_t K, uint2* aops, int* etab, float* stab,               \
        const float* gamma, float eps) {                                                       \
        gemm_xh_prep1_body<MG, true, true>(nullptr, M, K, aops, etab, stab, gamma, eps,        \
                                           nullptr, &ps);                                      \
    }
RT_GEMM_XH_PREP1S(1)
RT_GEMM_XH_PREP1S(2)
RT_GEMM_XH_PREP1S(4)
// the preparation of rows given as multi-query attention partials (PrepAttn)
#define RT_GEMM_XH_PREP1A(MG)                                                                  \
    extern "C" __global__ void __launch_bounds__(1024) k_gemm_xh_prep1a_mg##MG(                \
        PrepAttn pa, uint32_t M, uint32_t K, uint2* aops, int* etab, float* stab) {            \
        gemm_xh_prep1_body<MG, false, false, true>(nullptr, M, K, aops, etab, stab, nullptr,   \
                                                   0.0f, nullptr, nullptr, &pa);               \
    }
RT_GEMM_XH_PREP1A(1)
RT_GEMM_XH_PREP1A(2)
RT_GEMM_XH_PREP1A(4)
RT_GEMM_XH_PREP(1)
RT_GEMM_XH_PREP(2)
RT_GEMM_XH_PREP(4)

// ABUF = 1: the activation operands of a stage in one LDS buffer (the
// weights keep two), refilled after a barrier that ends every wave's reads —
// the Q6_K form at 32 rows, whose two buffers would not fit the LDS.
// WBUF = 1: the weights in one LDS buffer as well (the same barrier ends
// the stage's reads of both) — the Q6_K 128-row tiles at 32 rows.
// bid / nbk: the workgroup's index and the number of workgroups working on
// this GEMM (the whole grid, or its range of a multi-matrix launch).
template <class P, int MG, int NB, int WAVES = 4, int ABUF = 2, int WBUF = 2>
RT_DEV void gemm3_body(const Gemm2Args& a, uint32_t bid = blockIdx.x, uint32_t nbk = gridDim.x) {
    static_assert(WBUF == 2 || ABUF == 1, "one weight buffer needs the operand barrier");
    constexpr uint32_t T = 64 * WAVES, ROWS = 16 * WAVES;
    constexpr uint32_t NR = NB * P::RECS;
    constexpr uint32_t SEG = NB * P::BLK_BYTES;
    constexpr uint32_t VB = SEG % 16 == 0 ? 16 : (SEG % 8 == 0 ? 8 : 4);
    typedef typename std::conditional<VB == 16, u32x4,
                                      typename std::conditional<VB == 8, uint2, uint32_t>::type>::type WV;
    constexpr uint32_t WPR = SEG / VB;
    constexpr uint32_t WV_N = ROWS * WPR;
    constexpr uint32_t AV4 = NR * MG * 64;               // 16-byte A entries per stage
    constexpr uint32_t SV4 = NR * 8 * MG / 4;            // dwordx4 of S per stage
    constexpr uint32_t WPT = (WV_N + T - 1) / T;
    constexpr uint32_t APT = (AV4 + T - 1) / T;
    static_assert(SEG % VB == 0 && SV4 <= T, "segment alignment");
    // one LDS block, activation operands first: their reads then take
    // 16-bit immediate offsets
    __shared__ u32x4 g3lds[ABUF * AV4 + (WBUF * WV_N * sizeof(WV) + 15) / 16];
    u32x4 (*la)[AV4] = (u32x4 (*)[AV4])g3lds;
    WV (*lw)[WV_N] = (WV (*)[WV_N])(g3lds + ABUF * AV4);
    __shared__ u32x4 ls[P::HAS_MIN ? 2 : 1][P::HAS_MIN ? SV4 : 1];
    __shared__ uint32_t last_flag;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t j = lane & 15, c = lane >> 4;
    const uint32_t nitems = a.tiles * a.splits * a.nchunks;

    for (uint32_t item = bid; item < nitems; item += nbk) {
        const uint32_t tile = item % a.tiles;
        const uint32_t split = (item / a.tiles) % a.splits;
        const uint32_t ch = item / (a.tiles * a.splits);
        const uint32_t kb0 = split * a.kbs;
        const uint32_t kb1 = min(a.nxb, kb0 + a.kbs);
        const uint32_t nst = (kb1 - kb0) / NB;
        const uint32_t row0 = tile * ROWS;
        const uint32_t nrec = a.nxb * P::RECS;
        const u32x4* ap = (const u32x4*)a.aops + (size_t)ch * nrec * MG * 64;
        const float* sp = P::HAS_MIN ? a.stab + (size_t)ch * nrec * 8 * MG : nullptr;

        WV rw[WPT];
        u32x4 ra[APT], rs;
        auto gload = [&](uint32_t st) {
            const uint32_t b0 = kb0 + st * NB;
            const uint32_t r0 = b0 * P::RECS;
            // many loads per thread at 8 waves (Q6_K: 27): the load offsets
            // recomputed per stage, not held in registers across the item
            // loop (held, they spilled: Q6_K M = 32 74 µs against 50 µs)
            uint32_t tidw = tid;
            if (WAVES >= 8 && WPT > 16) asm volatile("" : "+v"(tidw));
#pragma unroll
            for (uint32_t i = 0; i < WPT; ++i) {
                uint32_t f = tidw + T * i;
                if (f >= WV_N) f = WV_N - 1;  // duplicate load, not stored
                const uint32_t r = f / WPR, col = f % WPR;
                const uint32_t n = min(row0 + r, a.N - 1);
                rw[i] = *(const WV*)(a.w + (size_t)n * a.row_bytes + (size_t)b0 * P::BLK_BYTES + col * VB);
            }
            const u32x4* as = ap + (size_t)r0 * MG * 64;
#pragma unroll
            for (uint32_t i = 0; i < APT; ++i) ra[i] = as[min(tid + T * i, AV4 - 1)];
            if (P::HAS_MIN) rs = ((const u32x4*)(sp + (size_t)r0 * 8 * MG))[min(tid, SV4 - 1)];
        };
        auto lstore = [&](uint32_t buf) {
#pragma unroll
            for (uint32_t i = 0; i < WPT; ++i)
                if (tid + T * i < WV_N) lw[WBUF == 2 ? buf : 0][tid + T * i] = rw[i];
#pragma unroll
            for (uint32_t i = 0; i < APT; ++i)
                if (tid + T * i < AV4) la[ABUF == 2 ? buf : 0][tid + T * i] = ra[i];
            if (P::HAS_MIN && tid < SV4) ls[P::HAS_MIN ? buf : 0][tid] = rs;
        };
        float acc[MG][2];
#pragma unroll
        for (int g = 0; g < MG; ++g) acc[g][0] = acc[g][1] = 0.0f;
        const uint32_t wrow = (16 * wv + j) * SEG;
        auto compute = [&](uint32_t buf) {
            const uint8_t* wb = (const uint8_t*)lw[WBUF == 2 ? buf : 0] + wrow;
            const u32x4* ab = la[ABUF == 2 ? buf : 0];
            const float* sb = (const float*)ls[P::HAS_MIN ? buf : 0];
            // record r of the stage from its decoded codes B and scales
            auto record = [&](uint32_t r, i64_t B, float dsc, float mn, float dsc2) {
                const h8_t Bh = gemm_i8x8_to_h8(B);
                const h8_t Z = h8_t{0, 0, 0, 0, 0, 0, 0, 0};
                // ggml Q6_K: elements 0..15 (k-groups c < 2) and 16..31 take
                // their own scales: one MFMA per half, the other half zeroed
                const h8_t B1 = (GemmSplit16<P>::value && c >= 2) ? Z : Bh;
                f4_t C[MG], C2[GemmSplit16<P>::value ? MG : 1];
#pragma unroll
                for (int g = 0; g < MG; ++g) {
                    const h8_t A = __builtin_bit_cast(h8_t, ab[(r * MG + g) * 64 + lane]);
                    C[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B1, f4_t{0, 0, 0, 0}, 0, 0, 0);
                    if (GemmSplit16<P>::value)
                        C2[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, c >= 2 ? Bh : Z,
                                                                       f4_t{0, 0, 0, 0}, 0, 0, 0);
                }
#pragma unroll
                for (int g = 0; g < MG; ++g) {
                    // acc += dsc·(hi + lo) − mn·Σx, as fused multiply-adds
                    float a0 = __builtin_fmaf(dsc, C[g][0], acc[g][0]);
                    float a1 = __builtin_fmaf(dsc, C[g][2], acc[g][1]);
                    a0 = __builtin_fmaf(dsc, C[g][1], a0);
                    a1 = __builtin_fmaf(dsc, C[g][3], a1);
                    if (GemmSplit16<P>::value) {
                        const f4_t& D = C2[GemmSplit16<P>::value ? g : 0];
                        a0 = __builtin_fmaf(dsc2, D[0], a0);
                        a1 = __builtin_fmaf(dsc2, D[2], a1);
                        a0 = __builtin_fmaf(dsc2, D[1], a0);
                        a1 = __builtin_fmaf(dsc2, D[3], a1);
                    }
                    if (P::HAS_MIN) {
                        const uint32_t i0 = (r * 8 + 2 * c) * MG + g, i1 = i0 + MG;
                        a0 = __builtin_fmaf(-mn, sb[i0], a0);
                        a1 = __builtin_fmaf(-mn, sb[i1], a1);
                    }
                    acc[g][0] = a0;
                    acc[g][1] = a1;
                }
            };
            if constexpr (GemmDecode4<P>::value) {
#pragma unroll 1
                for (uint32_t r4 = 0; r4 < NR / 4; ++r4) {
                    i64_t B4[4];
                    float ds4[4], ds24[4];
                    P::decode4(wb, r4, c, B4, ds4, ds24);
#pragma unroll
                    for (uint32_t q = 0; q < 4; ++q) record(4 * r4 + q, B4[q], ds4[q], 0.0f, ds24[q]);
                }
            } else {
#pragma unroll 2
                for (uint32_t r = 0; r < NR; ++r) {
                    i64_t B;
                    float dsc, mn, dsc2 = 0.0f;
                    P::decode(wb, r, c, B, dsc, mn, dsc2);
                    record(r, B, dsc, mn, dsc2);
                }
            }
        };
        if (nst > 0) {
            gload(0);
            lstore(0);
        }
        __syncthreads();
        for (uint32_t st = 0; st < nst; ++st) {
            const bool more = st + 1 < nst;
            if (more) gload(st + 1);
            compute(st & 1);
            if (ABUF == 1) __syncthreads();  // every wave done with the one operand buffer
            if (more) lstore((st + 1) & 1);
            __syncthreads();
        }
        // lane holds activation rows ch·8MG + 8g + 2c + {0, 1} of weight row
        // n; the rows' exponents scale the sums
#pragma unroll
        for (int g = 0; g < MG; ++g)
#pragma unroll
            for (int i = 0; i < 2; ++i)
                acc[g][i] = __builtin_amdgcn_ldexpf(acc[g][i], a.etab[ch * 8 * MG + 8 * g + 2 * c + i]);
        const uint32_t n = row0 + 16 * wv + j;
        if (a.splits == 1) {
            const float b = (a.bias && n < a.N) ? h2f(a.bias[n]) : 0.0f;
#pragma unroll
            for (int g = 0; g < MG; ++g)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t m = ch * 8 * MG + 8 * g + 2 * c + i;
                    if (m < a.M && n < a.N) {
                        float v = acc[g][i];
                        if (a.bias) v += b;
                        if (a.res) v = a.res[(size_t)m * a.N + n] + v;
                        a.y[(size_t)m * a.N + n] = v;
                    }
                }
            continue;
        }
        const size_t crow = (size_t)8 * MG;  // rows of a chunk
#pragma unroll
        for (int g = 0; g < MG; ++g)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const size_t pr = ((size_t)(ch * a.splits + split) * crow + 8 * g + 2 * c + i);
                if (n < a.N) {
                    if (a.counters) dev_store(a.part + pr * a.N + n, acc[g][i]);
                    else a.part[pr * a.N + n] = acc[g][i];
                }
            }
        if (!a.counters) continue;  // partial sums only: k_gemm_split_sum adds them
        dev_stores_done();
        __syncthreads();
        uint32_t* counter = a.counters + ((size_t)ch * a.tiles + tile) * a.cstride;
        if (tid == 0) last_flag = arrive(counter) == a.splits - 1;
        __syncthreads();
        if (!last_flag) continue;
        if (n < a.N) {
#pragma unroll
            for (int g = 0; g < MG; ++g)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t m = ch * 8 * MG + 8 * g + 2 * c + i;
                    float s = 0.0f;
                    for (uint32_t sp2 = 0; sp2 < a.splits; ++sp2)
                        s += dev_load(a.part + ((size_t)(ch * a.splits + sp2) * crow + 8 * g + 2 * c + i) * a.N + n);
                    if (m < a.M) a.y[(size_t)m * a.N + n] = s;
                }
        }
        if (tid == 0) dev_store(counter, 0u);  // ready for the next call (also under graph replay)
        __syncthreads();
    }
}
// Sum of the K splits' partial sums ([chunk][split][crow][N]) into
// Y[M][N], split by split in split order.  A launch of its own after the
// GEMM: the kernel boundary makes the partials visible, where an in-kernel
// hand-off (device-scope stores, an arrival counter, device-scope loads by
// the last split) cost ~9 µs of a 40 µs GEMM.
extern "C" __global__ void __launch_bounds__(256) k_gemm_split_sum(const float* __restrict__ part, float* __restrict__ y,
                                                                 uint32_t M, uint32_t N, uint32_t splits,
                                                                 uint32_t crow) {
    // grid (⌈N / 1024⌉, M): thread → 4 consecutive outputs of row m
    const uint32_t m = blockIdx.y, n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (n >= N) return;
    const uint32_t ch = m / crow, r = m % crow;
    const float* p = part + ((size_t)ch * splits * crow + r) * N + n;
    const size_t ss = (size_t)crow * N;
    if (n + 4 <= N && N % 4 == 0) {
        f32x4 v = *(const f32x4*)p;
        for (uint32_t sp = 1; sp < splits; ++sp) v += *(const f32x4*)(p + sp * ss);
        *(f32x4*)(y + (size_t)m * N + n) = v;
    } else {
        for (uint32_t i = 0; i < 4 && n + i < N; ++i) {
            float v = p[i];
            for (uint32_t sp = 1; sp < splits; ++sp) v += p[sp * ss + i];
            y[(size_t)m * N + n + i] = v;
        }
    }
}
// k_gemm_split_sum with the epilogues of verify_draft's GEMMs
// (forward.rs:2199-2271) folded in: Y = Σ part, then
//   part2 given (the up projection's partial sums, same splits and layout):
//     Y = silu(Σ part) · Σ part2, silu(g) = g / (1 + e^−g)  (silu_mul_f32);
//   bias given: Y += f32(bias[n])  (add_bias_broadcast_f16);
//   res given:  Y = res + Y         (add_f32; Y may alias res).
RT_DEV void split_sum_ep(const float* __restrict__ part, const float* __restrict__ part2, float* y,
                         uint32_t N, uint32_t splits, uint32_t crow,
                         const uint16_t* __restrict__ bias, const float* res, uint32_t bx) {
    const uint32_t m = blockIdx.y, n0 = (bx * 256 + threadIdx.x) * 4;
    if (n0 >= N) return;
    const uint32_t ch = m / crow, r = m % crow;
    const size_t off = ((size_t)ch * splits * crow + r) * N, ss = (size_t)crow * N;
    if (N % 4 == 0 && (((uintptr_t)part | (uintptr_t)part2 | (uintptr_t)y | (uintptr_t)res) & 15) == 0 &&
        ((uintptr_t)bias & 7) == 0) {
        // four consecutive outputs in 16-byte loads and stores (rows of a
        // multiple of 4 keep every row aligned)
        f32x4 v = *(const f32x4*)(part + off + n0);
        for (uint32_t sp = 1; sp < splits; ++sp) v += *(const f32x4*)(part + off + sp * ss + n0);
        if (part2) {
            f32x4 u = *(const f32x4*)(part2 + off + n0);
            for (uint32_t sp = 1; sp < splits; ++sp) u += *(const f32x4*)(part2 + off + sp * ss + n0);
            v = f32x4{v.x / (1.0f + expf(-v.x)) * u.x, v.y / (1.0f + expf(-v.y)) * u.y,
                      v.z / (1.0f + expf(-v.z)) * u.z, v.w / (1.0f + expf(-v.w)) * u.w};
        }
        if (bias) {
            const uint2 b = *(const uint2*)(bias + n0);
            v += f32x4{h2f(b.x), h2f(b.x >> 16), h2f(b.y), h2f(b.y >> 16)};
        }
        if (res) v = *(const f32x4*)(res + (size_t)m * N + n0) + v;
        *(f32x4*)(y + (size_t)m * N + n0) = v;
        return;
    }
    for (uint32_t n = n0; n < n0 + 4 && n < N; ++n) {
        float v = part[off + n];
        for (uint32_t sp = 1; sp < splits; ++sp) v += part[off + sp * ss + n];
        if (part2) {
            float u = part2[off + n];
            for (uint32_t sp = 1; sp < splits; ++sp) u += part2[off + sp * ss + n];
            v = v / (1.0f + expf(-v)) * u;
        }
        if (bias) v += h2f(bias[n]);
        if (res) v = res[(size_t)m * N + n] + v;
        y[(size_t)m * N + n] = v;
    }
}
extern "C" __global__ void __launch_bounds__(256)
k_gemm_split_sum_ep(const float* __restrict__ part, const float* __restrict__ part2, float* y,
                    uint32_t M, uint32_t N, uint32_t splits, uint32_t crow,
                    const uint16_t* __restrict__ bias, const float* res) {
    split_sum_ep(part, part2, y, N, splits, crow, bias, res, blockIdx.x);
}
// The split sums (+ bias) of up to three GEMMs of one set in one launch
// (Q/K/V): workgroup columns [blk0[i], blk0[i + 1]) take output i.
struct EpSeg {
    const float* part;
    float* y;
    const uint16_t* bias;
    uint32_t n, splits, blk0;
};
struct EpSegs {
    EpSeg s[3];
    uint32_t count, crow;
};
extern "C" __global__ void __launch_bounds__(256) k_gemm_split_sum_ep3(EpSegs a) {
    uint32_t i = 0;
    while (i + 1 < a.count && blockIdx.x >= a.s[i + 1].blk0) ++i;
    const EpSeg& g = a.s[i];
    split_sum_ep(g.part, nullptr, g.y, g.n, g.splits, a.crow, g.bias, nullptr, blockIdx.x - g.blk0);
}
// k_gemm_split_sum_ep3 of the Q/K/V set with rope_kv_write_batch folded in:
// segment 0 (q) rotated and written to q, segment 1 (k) rotated and written
// to the key cache at position start_pos + row, segment 2 (v) written to the
// value cache.  A workgroup's 1024 outputs are whole heads (head_dim divides
// 1024), so each pair (d, d + hd/2) meets in the workgroup's LDS; the angle
// is rope_kv_write_batch's, pos / θ^(2d/hd).
struct RopeKv {
    float* kc;
    float* vc;
    uint32_t head_dim, start_pos, max_seq;
    float theta;
};
extern "C" __global__ void __launch_bounds__(256) k_gemm_split_sum_qkv_rope(EpSegs a, RopeKv rk) {
    __shared__ float row[1024];
    uint32_t si = 0;
    while (si + 1 < a.count && blockIdx.x >= a.s[si + 1].blk0) ++si;
    const EpSeg& g = a.s[si];
    const uint32_t m = blockIdx.y, bx = blockIdx.x - g.blk0, tid = threadIdx.x;
    const uint32_t n0 = (bx * 256 + tid) * 4;
    const bool live = n0 < g.n;
    f32x4 v = {0, 0, 0, 0};
    if (live) {
        const uint32_t ch = m / a.crow, r = m % a.crow;
        const size_t off = ((size_t)ch * g.splits * a.crow + r) * g.n, ss = (size_t)a.crow * g.n;
        v = *(const f32x4*)(g.part + off + n0);
        for (uint32_t sp = 1; sp < g.splits; ++sp) v += *(const f32x4*)(g.part + off + sp * ss + n0);
        if (g.bias) {
            const uint2 b = *(const uint2*)(g.bias + n0);
            v += f32x4{h2f(b.x), h2f(b.x >> 16), h2f(b.y), h2f(b.y >> 16)};
        }
    }
    const uint32_t hd = rk.head_dim, half = hd / 2, pos = rk.start_pos + m;
    if (si == 2) {  // v: straight to the cache
        if (live) {
            const uint32_t h = n0 / hd, d = n0 % hd;
            *(f32x4*)(rk.vc + ((size_t)h * rk.max_seq + pos) * hd + d) = v;
        }
        return;
    }
    // the row's cos / sin per pair index, once per workgroup (head_dim ≤ 512)
    __shared__ float cs[256], sn_[256];
    if (tid < half) {
        const float angle = (float)pos / powf(rk.theta, (float)(2 * tid) / (float)hd);
        sincosf(angle, &sn_[tid], &cs[tid]);
    }
    *(f32x4*)(row + 4 * tid) = v;
    __syncthreads();
    if (!live) return;
    const uint32_t h = n0 / hd, d0 = n0 % hd;
    float o[4];
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
        const uint32_t d = d0 + e, dd = d % half, lo = 4 * tid + e;
        const float c = cs[dd], sn = sn_[dd];
        if (d < half) {
            const float r = v[e], i = row[lo + half];
            o[e] = r * c - i * sn;
        } else {
            const float r = row[lo - half], i = v[e];
            o[e] = i * c + r * sn;
        }
    }
    const f32x4 ov = {o[0], o[1], o[2], o[3]};
    if (si == 0)
        *(f32x4*)(g.y + (size_t)m * g.n + n0) = ov;
    else
        *(f32x4*)(rk.kc + ((size_t)h * rk.max_seq + pos) * hd + d0) = ov;
}
// Up to three GEMMs of one kernel shape over the same prepared activations
// in one launch: workgroups [g0[i], g0[i + 1]) run matrix i.
struct Gemm3Multi {
    Gemm2Args a[3];
    uint32_t g0[4];
    uint32_t count;
};
#define RT_GEMM3_MULTI(NAME, THREADS, ...)                                                    \
    extern "C" __global__ void __launch_bounds__(THREADS) NAME##_x3(Gemm3Multi m) {          \
        uint32_t i = 0;                                                                        \
        while (i + 1 < m.count && blockIdx.x >= m.g0[i + 1]) ++i;                             \
        gemm3_body<__VA_ARGS__>(m.a[i], blockIdx.x - m.g0[i], m.g0[i + 1] - m.g0[i]);         \
    }
#define RT_GEMM3_KERNEL4(FN, P, MG, NB)                                                       \
    extern "C" __global__ void __launch_bounds__(256) k_gemm3_##FN##_mg##MG(Gemm2Args a) {    \
        gemm3_body<P, MG, NB>(a);                                                              \
    }                                                                                          \
    RT_GEMM3_MULTI(k_gemm3_##FN##_mg##MG, 256, P, MG, NB)
#define RT_GEMM3_KERNEL(FN, P, MG, NB)                                                        \
    RT_GEMM3_KERNEL4(FN, P, MG, NB)                                                            \
    extern "C" __global__ void __launch_bounds__(512) k_gemm3_##FN##_mg##MG##_w8(Gemm2Args a) { \
        gemm3_body<P, MG, NB, 8>(a);                                                           \
    }                                                                                          \
    RT_GEMM3_MULTI(k_gemm3_##FN##_mg##MG##_w8, 512, P, MG, NB, 8)
// (a group here is 8 activation rows: MG = 1, 2, 4 cover 8, 16, 32 rows with
// the stage sizes of gemm2's 4-row groups MG = 2, 4, 8)
RT_GEMM3_KERNEL(q8_0, GemmQ8_0, 1, 8)
RT_GEMM3_KERNEL(q8_0, GemmQ8_0, 2, 4)
RT_GEMM3_KERNEL(q8_0, GemmQ8_0, 4, 4)
// 8 rows with 4-block stages, for K of a multiple of 4 but not of 8 blocks
// (the 0.5B hidden size 896: 28 blocks)
RT_GEMM3_KERNEL4(q8_0_nb4, GemmQ8_0, 1, 4)
RT_GEMM3_KERNEL4(q4_0_nb4, GemmQ4_0, 1, 4)
// 256-row tiles (16 waves share each stage of activation operands)
extern "C" __global__ void __launch_bounds__(1024) k_gemm3_q8_0_mg4_w16(Gemm2Args a) {
    gemm3_body<GemmQ8_0, 4, 4, 16>(a);
}
RT_GEMM3_MULTI(k_gemm3_q8_0_mg4_w16, 1024, GemmQ8_0, 4, 4, 16)
// and for the super-block formats at 32 rows (Q4_K 18944×3584 40.7 → 33.2 µs,
// Q5_K 42.2 → 35.8; Q4_0 unchanged, Q5_0 32.3 → 33.5, so they keep 128 rows)
#define RT_GEMM3_W16(FN, P, NB)                                                               \
    extern "C" __global__ void __launch_bounds__(1024) k_gemm3_##FN##_mg4_w16(Gemm2Args a) {  \
        gemm3_body<P, 4, NB, 16>(a);                                                           \
    }                                                                                          \
    RT_GEMM3_MULTI(k_gemm3_##FN##_mg4_w16, 1024, P, 4, NB, 16)
RT_GEMM3_W16(q4k, GemmQ4K, 1)
RT_GEMM3_W16(q4kg, GemmQ4KG, 1)
RT_GEMM3_W16(q5k, GemmQ5K, 1)
RT_GEMM3_W16(q5kg, GemmQ5KG, 1)
RT_GEMM3_KERNEL(q4_0, GemmQ4_0, 1, 8)
RT_GEMM3_KERNEL(q4_0, GemmQ4_0, 2, 4)
RT_GEMM3_KERNEL(q4_0, GemmQ4_0, 4, 4)
RT_GEMM3_KERNEL(q4k, GemmQ4K, 1, 1)
RT_GEMM3_KERNEL(q4k, GemmQ4K, 2, 1)
RT_GEMM3_KERNEL(q4k, GemmQ4K, 4, 1)
RT_GEMM3_KERNEL(q4kg, GemmQ4KG, 1, 1)
RT_GEMM3_KERNEL(q4kg, GemmQ4KG, 2, 1)
RT_GEMM3_KERNEL(q4kg, GemmQ4KG, 4, 1)
RT_GEMM3_KERNEL(q4_0g, GemmQ4_0G, 1, 8)
RT_GEMM3_KERNEL(q4_0g, GemmQ4_0G, 2, 4)
RT_GEMM3_KERNEL(q4_0g, GemmQ4_0G, 4, 4)
RT_GEMM3_KERNEL(q5_0, GemmQ5_0, 1, 8)
RT_GEMM3_KERNEL(q5_0, GemmQ5_0, 2, 4)
RT_GEMM3_KERNEL(q5_0, GemmQ5_0, 4, 4)
RT_GEMM3_KERNEL(q5k, GemmQ5K, 1, 1)
RT_GEMM3_KERNEL(q5k, GemmQ5K, 2, 1)
RT_GEMM3_KERNEL(q5k, GemmQ5K, 4, 1)
RT_GEMM3_KERNEL(q5kg, GemmQ5KG, 1, 1)
RT_GEMM3_KERNEL(q5kg, GemmQ5KG, 2, 1)
RT_GEMM3_KERNEL(q5kg, GemmQ5KG, 4, 1)
RT_GEMM3_KERNEL4(q6k, GemmQ6K, 1, 2)
RT_GEMM3_KERNEL4(q6k, GemmQ6K, 2, 2)
RT_GEMM3_KERNEL4(q6kg, GemmQ6KG, 1, 2)
RT_GEMM3_KERNEL4(q6kg, GemmQ6KG, 2, 2)
// 32 rows in one chunk (one pass over the weights): 64 KB of activation
// operands per stage, single-buffered
#define RT_GEMM3_KERNEL4A1(FN, P, MG, NB)                                                     \
    extern "C" __global__ void __launch_bounds__(256) k_gemm3_##FN##_mg##MG(Gemm2Args a) {    \
        gemm3_body<P, MG, NB, 4, 1>(a);                                                        \
    }
RT_GEMM3_KERNEL4A1(q6k, GemmQ6K, 4, 2)
RT_GEMM3_KERNEL4A1(q6kg, GemmQ6KG, 4, 2)
// 128-row tiles at 8 rows, both buffers doubled (137 KB)
extern "C" __global__ void __launch_bounds__(512) k_gemm3_q6k_mg1_w8(Gemm2Args a) {
    gemm3_body<GemmQ6K, 1, 2, 8>(a);
}
extern "C" __global__ void __launch_bounds__(512) k_gemm3_q6kg_mg1_w8(Gemm2Args a) {
    gemm3_body<GemmQ6KG, 1, 2, 8>(a);
}
// 128-row tiles at 16 / 32 rows: one operand and one weight buffer (84.5 /
// 116.5 KB)
#define RT_GEMM3_KERNEL8A1(FN, P, MG, NB)                                                     \
    extern "C" __global__ void __launch_bounds__(512) k_gemm3_##FN##_mg##MG##_w8(Gemm2Args a) { \
        gemm3_body<P, MG, NB, 8, 1, 1>(a);                                                     \
    }
RT_GEMM3_KERNEL8A1(q6k, GemmQ6K, 4, 2)
RT_GEMM3_KERNEL8A1(q6kg, GemmQ6KG, 4, 2)
RT_GEMM3_KERNEL8A1(q6k, GemmQ6K, 2, 2)
RT_GEMM3_KERNEL8A1(q6kg, GemmQ6KG, 2, 2)

#define RT_GEMM2_KERNEL4(FN, P, MG, NB)                                                       \
    extern "C" __global__ void __launch_bounds__(256) k_gemm2_##FN##_mg##MG(Gemm2Args a) {    \
        gemm2_body<P, MG, NB>(a);                                                              \
    }
#define RT_GEMM2_KERNEL(FN, P, MG, NB)                                                        \
    RT_GEMM2_KERNEL4(FN, P, MG, NB)                                                            \
    extern "C" __global__ void __launch_bounds__(512) k_gemm2_##FN##_mg##MG##_w8(Gemm2Args a) { \
        gemm2_body<P, MG, NB, 8>(a);                                                           \
    }
// NB: blocks per stage (Q8_0 / Q4_0: 8 records, or 4 for large batches so
// that the stage's operands leave room for 2+ workgroups per CU; Q4_K: one
// 256-element super-block = 8 records)
RT_GEMM2_KERNEL(q8_0, GemmQ8_0, 1, 8)
RT_GEMM2_KERNEL(q8_0, GemmQ8_0, 2, 8)
RT_GEMM2_KERNEL(q8_0, GemmQ8_0, 4, 4)
RT_GEMM2_KERNEL(q8_0, GemmQ8_0, 8, 4)
RT_GEMM2_KERNEL(q4_0, GemmQ4_0, 1, 8)
RT_GEMM2_KERNEL(q4_0, GemmQ4_0, 2, 8)
RT_GEMM2_KERNEL(q4_0, GemmQ4_0, 4, 4)
RT_GEMM2_KERNEL(q4_0, GemmQ4_0, 8, 4)
RT_GEMM2_KERNEL(q4k, GemmQ4K, 1, 1)
RT_GEMM2_KERNEL(q4k, GemmQ4K, 2, 1)
RT_GEMM2_KERNEL(q4k, GemmQ4K, 4, 1)
RT_GEMM2_KERNEL(q4k, GemmQ4K, 8, 1)
RT_GEMM2_KERNEL(q4kg, GemmQ4KG, 1, 1)
RT_GEMM2_KERNEL(q4kg, GemmQ4KG, 2, 1)
RT_GEMM2_KERNEL(q4kg, GemmQ4KG, 4, 1)
RT_GEMM2_KERNEL(q4kg, GemmQ4KG, 8, 1)
RT_GEMM2_KERNEL(q4_0g, GemmQ4_0G, 1, 8)
RT_GEMM2_KERNEL(q4_0g, GemmQ4_0G, 2, 8)
RT_GEMM2_KERNEL(q4_0g, GemmQ4_0G, 4, 4)
RT_GEMM2_KERNEL(q4_0g, GemmQ4_0G, 8, 4)
RT_GEMM2_KERNEL(q5_0, GemmQ5_0, 1, 8)
RT_GEMM2_KERNEL(q5_0, GemmQ5_0, 2, 8)
RT_GEMM2_KERNEL(q5_0, GemmQ5_0, 4, 4)
RT_GEMM2_KERNEL(q5_0, GemmQ5_0, 8, 4)
RT_GEMM2_KERNEL(q5k, GemmQ5K, 1, 1)
RT_GEMM2_KERNEL(q5k, GemmQ5K, 2, 1)
RT_GEMM2_KERNEL(q5k, GemmQ5K, 4, 1)
RT_GEMM2_KERNEL(q5k, GemmQ5K, 8, 1)
RT_GEMM2_KERNEL(q5kg, GemmQ5KG, 1, 1)
RT_GEMM2_KERNEL(q5kg, GemmQ5KG, 2, 1)
RT_GEMM2_KERNEL(q5kg, GemmQ5KG, 4, 1)
RT_GEMM2_KERNEL(q5kg, GemmQ5KG, 8, 1)
// Q6_K: two super-blocks per stage; at most 4 activation-row groups (the
// stage's 16 records of operands) and 4-wave workgroups (LDS)
RT_GEMM2_KERNEL4(q6k, GemmQ6K, 1, 2)
RT_GEMM2_KERNEL4(q6k, GemmQ6K, 2, 2)
RT_GEMM2_KERNEL4(q6k, GemmQ6K, 4, 2)
RT_GEMM2_KERNEL4(q6kg, GemmQ6KG, 1, 2)
RT_GEMM2_KERNEL4(q6kg, GemmQ6KG, 2, 2)
RT_GEMM2_KERNEL4(q6kg, GemmQ6KG, 4, 2)
