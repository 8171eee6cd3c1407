// rt_formats.h — GGUF block formats as "units" for the gfx950 GEMV kernels.
//
// A unit is the slice of one weight row that one lane handles per step:
//   Q8_0 : one 34-byte block            (32 elements, 1 activation record)
//   Q4_0 : one 18-byte block            (32 elements, 1 record)
//   Q4_K : one (super-block, pair j)    (64 elements: 32 qs bytes, 2 records)
//   Q6_K : one (super-block, half, l-half) (64 elements: 48 code bytes,
//          16 elements of each of 4 records)
// Units of a row are consecutive in memory, so lane j of a row group reading
// unit j gives contiguous wave-wide loads.
//
// Every dot is exact integer arithmetic (v_dot4_i32_i8 over the activation
// limbs of rt_device.h) followed by one f32 scaling per 32 elements.
#pragma once
#include "rt_device.h"

// Loads are always 4-byte aligned: the 34- and 18-byte blocks (and the
// 210-byte Q6_K blocks) start on 2-byte boundaries, and 2-byte-aligned wide
// loads stream markedly slower on gfx950 than aligned dword loads of the same
// lines.  Misaligned fields are rebuilt in registers with v_alignbyte.
RT_DEV uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}
template <int N>
RT_DEV void load_dwords(const uint8_t* p, uint32_t (&w)[N]) {
    // p is 4-byte aligned; N dwords as dwordx4 / dwordx2 / dword loads
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        u32x4 v = *(const u32x4_a4*)(p + 4 * i);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
    constexpr int R = N & 3, B = N - R;
    if (R == 3) {
        typedef uint32_t u32x3_a4 __attribute__((ext_vector_type(3), aligned(4)));
        u32x3_a4 v = *(const u32x3_a4*)(p + 4 * B);
        w[B] = v.x; w[B + 1] = v.y; w[B + 2] = v.z;
    } else if (R == 2) {
        typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
        u32x2_a4 v = *(const u32x2_a4*)(p + 4 * B);
        w[B] = v.x; w[B + 1] = v.y;
    } else if (R == 1) {
        w[B] = *(const uint32_t*)(p + 4 * B);
    }
}

// ───────────────────────────── matrix-core dots ─────────────────────────────
// v_mfma_i32_4x4x4i8 runs 16 independent 4×4×4 int8 products per wave.  For
// block b (lanes 4b..4b+3): lane 4b+i supplies row i of A (4 int8), lane 4b+j
// supplies column j of B, and lane 4b+j receives D[0..3][j] in its 4 result
// registers.  The GEMV kernels put activation limb i in A and weight row j in
// B, so lane 4b+q ends up holding the three limb dots of ITS OWN row q for
// the unit in slot b; lane q = 3 feeds a don't-care A row.
typedef int v4i __attribute__((ext_vector_type(4)));
RT_DEV v4i mfma4(uint32_t a, uint32_t b, v4i c) {
    return __builtin_amdgcn_mfma_i32_4x4x4i8((int)a, (int)b, c, 0, 0, 0);
}
RT_DEV float comb4(v4i c) { return limb_combine(c[0], c[1], c[2]); }

// Limb `lq` of a record (8 dwords) and its exponent / limb sums.
struct XLimb {
    uint32_t l[8];
    int e;
    int s[3];      // full-block sums
    int sh[2][3];  // per-half sums
};
RT_DEV void load_xlimb(const XRec* rec, uint32_t lq, XLimb& x) {
    const u32x4* p = (const u32x4*)rec;
    u32x4 a = p[2 * lq], b = p[2 * lq + 1];
    x.l[0] = a.x; x.l[1] = a.y; x.l[2] = a.z; x.l[3] = a.w;
    x.l[4] = b.x; x.l[5] = b.y; x.l[6] = b.z; x.l[7] = b.w;
    u32x4 m = p[6];
    x.e = (int)(int16_t)(m.x & 0xFFFF);
    x.sh[0][0] = (int16_t)(m.x >> 16);
    x.sh[0][1] = (int16_t)(m.y & 0xFFFF);
    x.sh[0][2] = (int16_t)(m.y >> 16);
    x.sh[1][0] = (int16_t)(m.z & 0xFFFF);
    x.sh[1][1] = (int16_t)(m.z >> 16);
    x.sh[1][2] = (int16_t)(m.w & 0xFFFF);
#pragma unroll
    for (int i = 0; i < 3; ++i) x.s[i] = x.sh[0][i] + x.sh[1][i];
}

// ───────────────────────────── Q8_0 ─────────────────────────────
// Block: d:f16 @0, qs:int8[32] @2 (gemv_q8_0.metal:11-17; forward.rs:951-963).
RT_DEV float q8_0_block_dot(uint32_t d, const uint32_t q[8], const XRegs& x) {
    int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        t0 = sdot4(q[i], x.l[0][i], t0);
        t1 = sdot4(q[i], x.l[1][i], t1);
        t2 = sdot4(q[i], x.l[2][i], t2);
    }
    return __builtin_amdgcn_ldexpf(h2f(d) * limb_combine(t0, t1, t2), x.e - 22);
}

// Unit = two consecutive blocks (68 bytes, 4-byte aligned when a row holds
// an even number of blocks): 17 aligned dwords.
struct FmtQ8_0 {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 34, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    static constexpr int PF = 1;  // matrix-core path: one item in flight per wave
    // held as whole dwordx4 tuples: element-wise copies out of a load's
    // destination would make the compiler wait for the load right away
    struct Raw {
        u32x4 v[4];
        uint32_t t;
        RT_DEV uint32_t operator[](int i) const { return i < 16 ? v[i >> 2][i & 3] : t; }
    };
    struct XU { XRegs x[2]; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint8_t* p = row + (size_t)u * 68;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.v[i] = *(const u32x4_a4*)(p + 16 * i);
        r.t = *(const uint32_t*)(p + 64);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        load_xregs(recs + 2 * uu, xu.x[0]);
        load_xregs(recs + 2 * uu + 1, xu.x[1]);
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t qa[8], qb[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            qa[i] = alignb(r[i + 1], r[i], 2);  // bytes 2..33
            qb[i] = r[9 + i];                     // bytes 36..67
        }
        return q8_0_block_dot(r[0], qa, xu.x[0]) + q8_0_block_dot(r[8] >> 16, qb, xu.x[1]);
    }
    // matrix-core form: recs = the unit's two records, lq = this lane's limb
    static constexpr bool XPAIR = true;  // mdotx: the unit's two records' limbs given
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        XLimb xa, xb;
        load_xlimb(xs + 2 * uu, lq, xa);
        load_xlimb(xs + 2 * uu + 1, lq, xb);
        return mdotx(r, xa, xb);
    }
    RT_DEV static float mdotx(const Raw& r, const XLimb& xa, const XLimb& xb) {
        v4i ca = {0, 0, 0, 0}, cb = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ca = mfma4(xa.l[i], alignb(r[i + 1], r[i], 2), ca);  // bytes 2..33
            cb = mfma4(xb.l[i], r[9 + i], cb);                     // bytes 36..67
        }
        return __builtin_amdgcn_ldexpf(h2f(r[0]) * comb4(ca), xa.e - 22) +
               __builtin_amdgcn_ldexpf(h2f(r[8] >> 16) * comb4(cb), xb.e - 22);
    }
};

// Single-block unit for rows with an odd number of blocks: 10 aligned dwords
// from the block's 4-byte-aligned floor.
struct FmtQ8_0S {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 34, UNIT_EL = 32;
    static constexpr bool Q40PERM = false;
    // 9 aligned dwords from the block's floor cover its 34 bytes at either
    // 2-byte offset and never lie wholly past the block
    struct Raw { uint32_t w[9]; uint32_t sh; };
    struct XU { XRegs x; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uintptr_t p = (uintptr_t)(row + (size_t)u * 34);
        r.sh = (uint32_t)(p & 3);
        load_dwords<9>((const uint8_t*)(p & ~(uintptr_t)3), r.w);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) { load_xregs(recs + uu, xu.x); }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = r.sh ? r.w[i + 1] : alignb(r.w[i + 1], r.w[i], 2);
        const uint32_t d = alignb(r.w[1], r.w[0], r.sh);
        return q8_0_block_dot(d, q, xu.x);
    }
};

// ───────────────────────────── Q4_0 ─────────────────────────────
// Block: d:f16 @0, qs:u8[16] @2; element 2i = qs[i]&0xF, 2i+1 = qs[i]>>4,
// value d·(nib−8) (gemv_q4_0.metal:10-15; forward.rs:964-978).
RT_DEV float q4_0_block_dot(uint32_t d, const uint32_t q[4], const XRegs& x) {
    // −8·Σx folded into the accumulators' start values
    int t0 = -8 * x.s[0], t1 = -8 * x.s[1], t2 = -8 * x.s[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = q[i] & 0x0F0F0F0Fu;         // elements 8i+{0,2,4,6}
        const uint32_t hi = (q[i] >> 4) & 0x0F0F0F0Fu;  // elements 8i+{1,3,5,7}
        t0 = sdot4(lo, x.l[0][2 * i], t0);
        t0 = sdot4(hi, x.l[0][2 * i + 1], t0);
        t1 = sdot4(lo, x.l[1][2 * i], t1);
        t1 = sdot4(hi, x.l[1][2 * i + 1], t1);
        t2 = sdot4(lo, x.l[2][2 * i], t2);
        t2 = sdot4(hi, x.l[2][2 * i + 1], t2);
    }
    return __builtin_amdgcn_ldexpf(h2f(d) * limb_combine(t0, t1, t2), x.e - 22);
}

// Unit = two consecutive blocks (36 bytes): 9 aligned dwords.
struct FmtQ4_0 {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 18, UNIT_EL = 64;
    static constexpr bool Q40PERM = true;
    struct Raw { uint32_t w[9]; };
    struct XU { XRegs x[2]; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        load_dwords<9>(row + (size_t)u * 36, r.w);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        load_xregs(recs + 2 * uu, xu.x[0]);
        load_xregs(recs + 2 * uu + 1, xu.x[1]);
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t qa[4], qb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qa[i] = alignb(r.w[i + 1], r.w[i], 2);  // bytes 2..17
            qb[i] = r.w[5 + i];                     // bytes 20..35
        }
        return q4_0_block_dot(r.w[0], qa, xu.x[0]) + q4_0_block_dot(r.w[4] >> 16, qb, xu.x[1]);
    }
    static constexpr bool XPAIR = true;
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        XLimb xa, xb;
        load_xlimb(xs + 2 * uu, lq, xa);
        load_xlimb(xs + 2 * uu + 1, lq, xb);
        return mdotx(r, xa, xb);
    }
    RT_DEV static float mdotx(const Raw& r, const XLimb& xa, const XLimb& xb) {
        // −8·Σx folded into the accumulators' start values
        v4i ca = {-8 * xa.s[0], -8 * xa.s[1], -8 * xa.s[2], 0};
        v4i cb = {-8 * xb.s[0], -8 * xb.s[1], -8 * xb.s[2], 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t qa = alignb(r.w[i + 1], r.w[i], 2), qb = r.w[5 + i];
            ca = mfma4(xa.l[2 * i], qa & 0x0F0F0F0Fu, ca);           // elements 8i+{0,2,4,6}
            ca = mfma4(xa.l[2 * i + 1], (qa >> 4) & 0x0F0F0F0Fu, ca);  // elements 8i+{1,3,5,7}
            cb = mfma4(xb.l[2 * i], qb & 0x0F0F0F0Fu, cb);
            cb = mfma4(xb.l[2 * i + 1], (qb >> 4) & 0x0F0F0F0Fu, cb);
        }
        return __builtin_amdgcn_ldexpf(h2f(r.w[0]) * comb4(ca), xa.e - 22) +
               __builtin_amdgcn_ldexpf(h2f(r.w[4] >> 16) * comb4(cb), xb.e - 22);
    }
};

// Single-block unit for rows with an odd number of blocks.
struct FmtQ4_0S {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 18, UNIT_EL = 32;
    static constexpr bool Q40PERM = true;
    // 5 aligned dwords from the block's floor cover its 18 bytes at either
    // 2-byte offset and never lie wholly past the block
    struct Raw { uint32_t w[5]; uint32_t sh; };
    struct XU { XRegs x; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uintptr_t p = (uintptr_t)(row + (size_t)u * 18);
        r.sh = (uint32_t)(p & 3);
        load_dwords<5>((const uint8_t*)(p & ~(uintptr_t)3), r.w);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) { load_xregs(recs + uu, xu.x); }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = r.sh ? r.w[i + 1] : alignb(r.w[i + 1], r.w[i], 2);
        return q4_0_block_dot(alignb(r.w[1], r.w[0], r.sh), q, xu.x);
    }
};

// ───────────────────────────── Q4_K ─────────────────────────────
// 6-bit (scale, min) of sub-block `is` from the 12-byte table held as three
// dwords y = bytes 0..3, z = 4..7, w = 8..11 (get_scale_min_k4,
// forward.rs:359-369; ggml uses the same packing).
RT_DEV void kq_scale_min(uint32_t is, uint32_t y, uint32_t z, uint32_t w, uint32_t& sc,
                          uint32_t& m) {
    const uint32_t b = 8 * (is & 3);
    const uint32_t yb = (y >> b) & 255u, zb = (z >> b) & 255u, wb = (w >> b) & 255u;
    if (is < 4) {
        sc = yb & 63u;
        m = zb & 63u;
    } else {
        sc = (wb & 15u) | ((yb >> 6) << 4);
        m = (wb >> 4) | ((zb >> 6) << 4);
    }
}
// (scale, min) of the unit's two sub-blocks packed as bytes (sc_lo, m_lo,
// sc_hi, m_hi).  Reference layout: pair j uses sub-blocks j and j + 4
// (forward.rs:1026-1057); ggml layout: 2j and 2j + 1 (dequantize_row_q4_K).
template <bool G>
RT_DEV uint32_t k_quant_scales(uint32_t j, uint32_t y, uint32_t z, uint32_t w) {
    uint32_t a, b, c, d;
    kq_scale_min(G ? 2 * j : j, y, z, w, a, b);
    kq_scale_min(G ? 2 * j + 1 : j + 4, y, z, w, c, d);
    return a | (b << 8) | (c << 16) | (d << 24);
}

// Super-block: d:f16 @0, dmin:f16 @2, scales:u8[12] @4, qs:u8[128] @16
// (dequant.metal:9-16).  Pair j ∈ 0..3: element 64j+l = d·sc·(qs[32j+l]&0xF)
// − dmin·m of the pair's first sub-block, element 64j+32+l the high nibble
// with the second sub-block's (sc, m).  Sub-blocks per k_quant_scales<G>.
template <bool G>
struct FmtQ4KT {
    static constexpr uint32_t BLK_EL = 256, BLK_BYTES = 144, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t dd; uint32_t sc; uint32_t q[8]; };
    struct XU { XRegs lo, hi; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint32_t b = u >> 2, j = u & 3;
        const uint8_t* p = row + (size_t)b * 144;
        // 144-byte blocks keep 16-byte alignment: header = one dwordx4
        const u32x4 hdr = *(const u32x4*)p;
        r.dd = hdr.x;
        r.sc = k_quant_scales<G>(j, hdr.y, hdr.z, hdr.w);
        const u32x4* qp = (const u32x4*)(p + 16 + 32 * j);
        u32x4 a = qp[0], c = qp[1];
        r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
        r.q[4] = c.x; r.q[5] = c.y; r.q[6] = c.z; r.q[7] = c.w;
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        load_xregs(recs + 2 * uu, xu.lo);
        load_xregs(recs + 2 * uu + 1, xu.hi);
    }
    RT_DEV static void scales(const Raw& r, float& d_lo, float& m_lo, float& d_hi, float& m_hi) {
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        d_lo = d * (float)(r.sc & 255u);
        m_lo = dmin * (float)((r.sc >> 8) & 255u);
        d_hi = d * (float)((r.sc >> 16) & 255u);
        m_hi = dmin * (float)(r.sc >> 24);
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = r.q[i] & 0x0F0F0F0Fu;
            const uint32_t hi = (r.q[i] >> 4) & 0x0F0F0F0Fu;
            a0 = sdot4(lo, xu.lo.l[0][i], a0);
            a1 = sdot4(lo, xu.lo.l[1][i], a1);
            a2 = sdot4(lo, xu.lo.l[2][i], a2);
            b0 = sdot4(hi, xu.hi.l[0][i], b0);
            b1 = sdot4(hi, xu.hi.l[1][i], b1);
            b2 = sdot4(hi, xu.hi.l[2][i], b2);
        }
        float d_lo, mm_lo, d_hi, mm_hi;
        scales(r, d_lo, mm_lo, d_hi, mm_hi);
        const float vlo = d_lo * limb_combine(a0, a1, a2) -
                          mm_lo * limb_combine(xu.lo.s[0], xu.lo.s[1], xu.lo.s[2]);
        const float vhi = d_hi * limb_combine(b0, b1, b2) -
                          mm_hi * limb_combine(xu.hi.s[0], xu.hi.s[1], xu.hi.s[2]);
        return __builtin_amdgcn_ldexpf(vlo, xu.lo.e - 22) +
               __builtin_amdgcn_ldexpf(vhi, xu.hi.e - 22);
    }
    static constexpr bool XPAIR = true;
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        XLimb xl, xh;
        load_xlimb(xs + 2 * uu, lq, xl);
        load_xlimb(xs + 2 * uu + 1, lq, xh);
        return mdotx(r, xl, xh);
    }
    RT_DEV static float mdotx(const Raw& r, const XLimb& xl, const XLimb& xh) {
        v4i cl = {0, 0, 0, 0}, ch = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            cl = mfma4(xl.l[i], r.q[i] & 0x0F0F0F0Fu, cl);
            ch = mfma4(xh.l[i], (r.q[i] >> 4) & 0x0F0F0F0Fu, ch);
        }
        float d_lo, mm_lo, d_hi, mm_hi;
        scales(r, d_lo, mm_lo, d_hi, mm_hi);
        const float vlo = d_lo * comb4(cl) - mm_lo * limb_combine(xl.s[0], xl.s[1], xl.s[2]);
        const float vhi = d_hi * comb4(ch) - mm_hi * limb_combine(xh.s[0], xh.s[1], xh.s[2]);
        return __builtin_amdgcn_ldexpf(vlo, xl.e - 22) + __builtin_amdgcn_ldexpf(vhi, xh.e - 22);
    }
};
using FmtQ4K = FmtQ4KT<false>;
using FmtQ4KG = FmtQ4KT<true>;

// ───────────────────────────── Q6_K ─────────────────────────────
// Super-block: ql:u8[128] @0, qh:u8[64] @128, sc:i8[16] @192, d:f16 @208.
// For half h ∈ {0,128}, l ∈ 0..31, t ∈ 0..3: element h+32t+l =
//   d · sc[h/16 + 2t] · (code_t − 32), code_t from ql[h/2+l (+32 if t odd)]
//   (low nibble for t<2, high for t≥2) and 2 bits (qh[h/4+l] >> 2t)
// (forward.rs:921-950; only the even scale slots are read, forward.rs:935).
// The ggml layout (G) gives every 16 elements their own scale: element
// h + 32t + l uses sc[h/16 + 2t + l/16] instead of sc[h/16 + 2t]
// (dequantize_row_q6_K); its unit's scale bytes are shifted by l-half.
template <bool G>
struct FmtQ6KT {
    static constexpr uint32_t BLK_EL = 256, BLK_BYTES = 210, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t ql0[4], ql1[4], qh[4]; uint32_t sc01, sc23; uint32_t d; };
    struct XHalf { uint32_t l[3][4]; int e; int s[3]; };
    struct XU { XHalf t[4]; };
    // 16 bytes at a 2-byte-aligned address, via 5 aligned dwords + alignbyte
    RT_DEV static void load16(const uint8_t* q, uint32_t out[4]) {
        const uintptr_t pa = (uintptr_t)q;
        const uint32_t sh = (uint32_t)(pa & 3);
        uint32_t w[5];
        load_dwords<5>((const uint8_t*)(pa & ~(uintptr_t)3), w);
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = alignb(w[i + 1], w[i], sh);
    }
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint32_t b = u >> 2, hsel = (u >> 1) & 1, lh = u & 1;
        const uint8_t* p = row + (size_t)b * 210;
        const uint32_t h = hsel * 128;
        load16(p + h / 2 + 16 * lh, r.ql0);
        load16(p + h / 2 + 32 + 16 * lh, r.ql1);
        load16(p + 128 + h / 4 + 16 * lh, r.qh);
        // scales sc[h/16 .. h/16+7] and d (bytes 208-209): 5 aligned dwords
        // from the floor of byte 192 + h/16
        const uintptr_t ps = (uintptr_t)(p + 192 + h / 16);
        const uint32_t sh = (uint32_t)(ps & 3);
        uint32_t w[5];
        // dwords past the block's last byte (never used) re-read its last
        // dword instead, so the window stays inside the weights
        const uintptr_t wl = (uintptr_t)(p + 209) & ~(uintptr_t)3;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const uintptr_t a = (ps & ~(uintptr_t)3) + 4 * i;
            w[i] = *(const uint32_t*)(a <= wl ? a : wl);
        }
        r.sc01 = alignb(w[1], w[0], sh);  // bytes 0..3: sc[is+0], (odd), sc[is+2], (odd)
        r.sc23 = alignb(w[2], w[1], sh);  // bytes 4..7: sc[is+4], (odd), sc[is+6], (odd)
        if (G) {  // bytes 0 and 2 become sc[is + lh + 0|2] (and + 4|6)
            r.sc01 >>= 8 * lh;
            r.sc23 >>= 8 * lh;
        }
        // d sits 16 (h = 0) or 8 (h = 128) bytes after the scale window start
        r.d = hsel ? alignb(w[3], w[2], sh) : alignb(w[4], w[4], sh);
    }
    // the same from a row copied into LDS: the alignment is taken with
    // pointer arithmetic (integer address arithmetic would lose the LDS
    // address space and turn every read into a flat load)
    RT_DEV static void load16_ls(const uint8_t* q, uint32_t out[4]) {
        const uint32_t sh = (uint32_t)((uintptr_t)q & 3);
        uint32_t w[5];
        load_dwords<5>(q - sh, w);
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = alignb(w[i + 1], w[i], sh);
    }
    RT_DEV static void load_ls(const uint8_t* row, uint32_t u, Raw& r) {
        const uint32_t b = u >> 2, hsel = (u >> 1) & 1, lh = u & 1;
        const uint8_t* p = row + (size_t)b * 210;
        const uint32_t h = hsel * 128;
        load16_ls(p + h / 2 + 16 * lh, r.ql0);
        load16_ls(p + h / 2 + 32 + 16 * lh, r.ql1);
        load16_ls(p + 128 + h / 4 + 16 * lh, r.qh);
        const uint8_t* ps = p + 192 + h / 16;
        const uint32_t sh = (uint32_t)((uintptr_t)ps & 3);
        const uint8_t* ps4 = ps - sh;
        // (in LDS the slot holds whole 16-byte granules around the chunk, so
        // the window's last dword never leaves the slot)
        uint32_t w[5];
        load_dwords<5>(ps4, w);
        r.sc01 = alignb(w[1], w[0], sh);
        r.sc23 = alignb(w[2], w[1], sh);
        if (G) {
            r.sc01 >>= 8 * lh;
            r.sc23 >>= 8 * lh;
        }
        r.d = hsel ? alignb(w[3], w[2], sh) : alignb(w[4], w[4], sh);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        // unit uu (chunk-relative) → super-block b = uu>>2, half, l-half
        const uint32_t b = uu >> 2, hsel = (uu >> 1) & 1, lh = uu & 1;
        const XRec* base = recs + 8 * b + 4 * hsel;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const u32x4* p = (const u32x4*)(base + t);
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                u32x4 v = p[2 * k + lh];
                xu.t[t].l[k][0] = v.x; xu.t[t].l[k][1] = v.y;
                xu.t[t].l[k][2] = v.z; xu.t[t].l[k][3] = v.w;
            }
            u32x4 m = p[6];
            xu.t[t].e = (int)(int16_t)(m.x & 0xFFFF);
            if (lh == 0) {
                xu.t[t].s[0] = (int16_t)(m.x >> 16);
                xu.t[t].s[1] = (int16_t)(m.y & 0xFFFF);
                xu.t[t].s[2] = (int16_t)(m.y >> 16);
            } else {
                xu.t[t].s[0] = (int16_t)(m.z & 0xFFFF);
                xu.t[t].s[1] = (int16_t)(m.z >> 16);
                xu.t[t].s[2] = (int16_t)(m.w & 0xFFFF);
            }
        }
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        const float d = h2f(r.d);
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int z0 = 0, z1 = 0, z2 = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t ql = (t & 1) ? r.ql1[c] : r.ql0[c];
                const uint32_t lo4 = (t < 2) ? (ql & 0x0F0F0F0Fu) : ((ql >> 4) & 0x0F0F0F0Fu);
                const uint32_t hi2 = (r.qh[c] >> (2 * t)) & 0x03030303u;
                const uint32_t code = lo4 | (hi2 << 4);  // 0..63 per byte
                z0 = sdot4(code, xu.t[t].l[0][c], z0);
                z1 = sdot4(code, xu.t[t].l[1][c], z1);
                z2 = sdot4(code, xu.t[t].l[2][c], z2);
            }
            z0 -= 32 * xu.t[t].s[0];
            z1 -= 32 * xu.t[t].s[1];
            z2 -= 32 * xu.t[t].s[2];
            const uint32_t scw = (t < 2) ? r.sc01 : r.sc23;
            const int sc = (int)(int8_t)((scw >> (16 * (t & 1))) & 255u);
            acc += __builtin_amdgcn_ldexpf(d * (float)sc * limb_combine(z0, z1, z2),
                                           xu.t[t].e - 22);
        }
        return acc;
    }
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        const uint32_t b = uu >> 2, hsel = (uu >> 1) & 1, lh = uu & 1;
        const XRec* base = xs + 8 * b + 4 * hsel;
        const float d = h2f(r.d);
        float acc = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const u32x4* p = (const u32x4*)(base + t);
            const u32x4 lv = p[2 * lq + lh];
            const u32x4 m = p[6];
            const int e = (int)(int16_t)(m.x & 0xFFFF);
            int s0, s1, s2;
            if (lh == 0) {
                s0 = (int16_t)(m.x >> 16); s1 = (int16_t)(m.y & 0xFFFF); s2 = (int16_t)(m.y >> 16);
            } else {
                s0 = (int16_t)(m.z & 0xFFFF); s1 = (int16_t)(m.z >> 16); s2 = (int16_t)(m.w & 0xFFFF);
            }
            // codes are 0..63; −32·Σx (over this 16-element half) seeds the accumulators
            v4i c = {-32 * s0, -32 * s1, -32 * s2, 0};
            const uint32_t xl[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t ql = (t & 1) ? r.ql1[k] : r.ql0[k];
                const uint32_t lo4 = (t < 2) ? (ql & 0x0F0F0F0Fu) : ((ql >> 4) & 0x0F0F0F0Fu);
                const uint32_t hi2 = (r.qh[k] >> (2 * t)) & 0x03030303u;
                c = mfma4(xl[k], lo4 | (hi2 << 4), c);
            }
            const uint32_t scw = (t < 2) ? r.sc01 : r.sc23;
            const int sc = (int)(int8_t)((scw >> (16 * (t & 1))) & 255u);
            acc += __builtin_amdgcn_ldexpf(d * (float)sc * comb4(c), e - 22);
        }
        return acc;
    }
};

using FmtQ6K = FmtQ6KT<false>;
using FmtQ6KG = FmtQ6KT<true>;

// Q6_K for the matrix-core path: one whole 210-byte super-block (256
// elements) per lane, loaded as 53 aligned dwords (13 dwordx4 + 1) from the
// block's 4-byte floor.  The block starts 0 or 2 bytes past that floor (sh);
// every field read below sits at a 4-byte multiple of the block start, so a
// single alignbyte by sh rebuilds it.  Reference layout (forward.rs:921-950):
// for half h ∈ {0, 128} and l ∈ 0..31, element h + 32t + l (t = 0..3) is
//   ((ql[h/2 + l + 32·(t&1)] >> 4·(t>>1)) & 15) | (((qh[h/4 + l] >> 2t) & 3) << 4),
// minus 32, times d · int8(sc[h/16 + 2t]) — one scale per 32-element record.
// ggml layout (G): the two 16-element halves of each record accumulate
// separately and take sc[h/16 + 2t] and sc[h/16 + 2t + 1].
template <bool G>
struct FmtQ6KBT {
    static constexpr uint32_t BLK_EL = 256, BLK_BYTES = 210, UNIT_EL = 256;
    static constexpr bool Q40PERM = false;
    static constexpr int PF = 1;  // one item (212 bytes per lane) in flight per wave
    struct Raw { uint32_t w[53]; uint32_t sh; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uintptr_t p = (uintptr_t)(row + (size_t)u * 210);
        r.sh = (uint32_t)(p & 3);
        load_dwords<53>((const uint8_t*)(p & ~(uintptr_t)3), r.w);
    }
    // the same from a row copied into LDS (offset arithmetic on the pointer
    // keeps its address space, so the reads compile to LDS reads)
    RT_DEV static void load_ls(const uint8_t* row, uint32_t u, Raw& r) {
        const uint8_t* p = row + (size_t)u * 210;
        r.sh = (uint32_t)((uintptr_t)p & 3);
        load_dwords<53>(p - r.sh, r.w);
    }
    // bytes [off, off+4) of the block, off a multiple of 4 below 208 (a
    // constant once the callers' loops are unrolled)
    RT_DEV static uint32_t get(const Raw& r, uint32_t off) {
        return alignb(r.w[off / 4 + 1], r.w[off / 4], r.sh);
    }
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        const float d = h2f(r.w[52] >> (8 * r.sh));  // bytes 208-209
        constexpr int NH = G ? 2 : 1;  // accumulators per record
        float acc = 0.0f;
#pragma unroll 1
        for (int hs = 0; hs < 2; ++hs) {  // (rolled: one half's operands live at a time)
            const XRec* rec = xs + 8 * uu + 4 * hs;
            v4i c[4][NH];
            int e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const u32x4 m = ((const u32x4*)(rec + t))[6];
                e[t] = (int)(int16_t)(m.x & 0xFFFF);
                // codes are 0..63; −32·Σx over the record (G: over each half)
                // seeds the accumulators
                const int a0 = (int16_t)(m.x >> 16), a1 = (int16_t)(m.y & 0xFFFF),
                          a2 = (int16_t)(m.y >> 16);
                const int b0 = (int16_t)(m.z & 0xFFFF), b1 = (int16_t)(m.z >> 16),
                          b2 = (int16_t)(m.w & 0xFFFF);
                if (G) {
                    c[t][0] = v4i{-32 * a0, -32 * a1, -32 * a2, 0};
                    c[t][NH - 1] = v4i{-32 * b0, -32 * b1, -32 * b2, 0};
                } else {
                    c[t][0] = v4i{-32 * (a0 + b0), -32 * (a1 + b1), -32 * (a2 + b2), 0};
                }
            }
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                // limb dword g of the four records, read where it is used
                uint32_t xl[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) xl[t] = ((const uint32_t*)(rec + t))[8 * lq + g];
                // (both halves' offsets are constants; the rolled loop selects)
                const uint32_t ql = hs ? get(r, 64 + 4 * g) : get(r, 4 * g);
                const uint32_t ql32 = hs ? get(r, 96 + 4 * g) : get(r, 32 + 4 * g);
                const uint32_t qh = hs ? get(r, 160 + 4 * g) : get(r, 128 + 4 * g);
                const int k = (G && g >= 4) ? NH - 1 : 0;
                c[0][k] = mfma4(xl[0], (ql & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u), c[0][k]);
                c[1][k] = mfma4(xl[1], (ql32 & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u), c[1][k]);
                c[2][k] = mfma4(xl[2], ((ql >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u), c[2][k]);
                c[3][k] = mfma4(xl[3], ((ql32 >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u), c[3][k]);
            }
            // scales sc[8·hs + 2t (+1)]: bytes 192 + 8·hs + 0..7
            const uint32_t sa = hs ? get(r, 200) : get(r, 192);
            const uint32_t sb = hs ? get(r, 204) : get(r, 196);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t sw = t < 2 ? sa : sb;
                const int sh0 = 16 * (t & 1);
                const int s0 = (int8_t)((sw >> sh0) & 255u);
                float v = d * (float)s0 * comb4(c[t][0]);
                if (G) {
                    const int s1 = (int8_t)((sw >> (sh0 + 8)) & 255u);
                    v += d * (float)s1 * comb4(c[t][NH - 1]);
                }
                acc += __builtin_amdgcn_ldexpf(v, e[t] - 22);
            }
        }
        return acc;
    }
    // VALU form of mdot: every lane takes all three limbs of its records and
    // accumulates them with v_dot4_i32_i8 (no matrix core); same integer
    // sums, same f32 combination, so the same result bit for bit
    RT_DEV static float vdot(const Raw& r, const XRec* xs, uint32_t uu) {
        const float d = h2f(r.w[52] >> (8 * r.sh));
        constexpr int NH = G ? 2 : 1;
        float acc = 0.0f;
#pragma unroll 1
        for (int hs = 0; hs < 2; ++hs) {
            const XRec* rec = xs + 8 * uu + 4 * hs;
            int z[4][NH][3];
            int e[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const u32x4 m = ((const u32x4*)(rec + t))[6];
                e[t] = (int)(int16_t)(m.x & 0xFFFF);
                const int a0 = (int16_t)(m.x >> 16), a1 = (int16_t)(m.y & 0xFFFF),
                          a2 = (int16_t)(m.y >> 16);
                const int b0 = (int16_t)(m.z & 0xFFFF), b1 = (int16_t)(m.z >> 16),
                          b2 = (int16_t)(m.w & 0xFFFF);
                if (G) {
                    z[t][0][0] = -32 * a0; z[t][0][1] = -32 * a1; z[t][0][2] = -32 * a2;
                    z[t][NH - 1][0] = -32 * b0; z[t][NH - 1][1] = -32 * b1; z[t][NH - 1][2] = -32 * b2;
                } else {
                    z[t][0][0] = -32 * (a0 + b0); z[t][0][1] = -32 * (a1 + b1);
                    z[t][0][2] = -32 * (a2 + b2);
                }
            }
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const uint32_t ql = hs ? get(r, 64 + 4 * g) : get(r, 4 * g);
                const uint32_t ql32 = hs ? get(r, 96 + 4 * g) : get(r, 32 + 4 * g);
                const uint32_t qh = hs ? get(r, 160 + 4 * g) : get(r, 128 + 4 * g);
                const int k = (G && g >= 4) ? NH - 1 : 0;
                const uint32_t code[4] = {
                    (ql & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u),
                    (ql32 & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u),
                    ((ql >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u),
                    ((ql32 >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u)};
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int l = 0; l < 3; ++l)
                        z[t][k][l] = sdot4(code[t], ((const uint32_t*)(rec + t))[8 * l + g], z[t][k][l]);
            }
            const uint32_t sa = hs ? get(r, 200) : get(r, 192);
            const uint32_t sb = hs ? get(r, 204) : get(r, 196);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t sw = t < 2 ? sa : sb;
                const int sh0 = 16 * (t & 1);
                const int s0 = (int8_t)((sw >> sh0) & 255u);
                float v = d * (float)s0 * limb_combine(z[t][0][0], z[t][0][1], z[t][0][2]);
                if (G) {
                    const int s1 = (int8_t)((sw >> (sh0 + 8)) & 255u);
                    v += d * (float)s1 * limb_combine(z[t][NH - 1][0], z[t][NH - 1][1], z[t][NH - 1][2]);
                }
                acc += __builtin_amdgcn_ldexpf(v, e[t] - 22);
            }
        }
        return acc;
    }
};
using FmtQ6KB = FmtQ6KBT<false>;
using FmtQ6KGB = FmtQ6KBT<true>;

// ───────────────────────────── Q5_0 / Q5_K ─────────────────────────────
//
// The reference runs these through CPU dequantisation to f16/f32 (forward.rs:
// 900-920 Q5_0, 979-1012 Q5_K); these formats give them fused GEMVs with the
// same values.  A 5-bit code is a 4-bit nibble plus one high bit taken from a
// bit array; for four consecutive elements the four high bits are one
// nibble of that array, spread to bit 4 of each byte by spread4.
RT_DEV uint32_t spread4(uint32_t nib) {  // bit k of nib → bit 8k
    return (nib * 0x00204081u) & 0x01010101u;
}

// Q5_0 block (22 B): d f16 @0, qh u32 @2, qs[16] @6.  Element j < 16 is
// (qs[j] & 15) | (qh bit j) << 4, element 16 + j is (qs[j] >> 4) | (qh bit
// 16+j) << 4; value d·(q − 16) (forward.rs:900-920).  q[i] = qs dword i.
RT_DEV float q5_0_block_mdot(uint32_t d16, uint32_t qh, const uint32_t q[4], const XLimb& x) {
    v4i c = {-16 * x.s[0], -16 * x.s[1], -16 * x.s[2], 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c = mfma4(x.l[i], (q[i] & 0x0F0F0F0Fu) | (spread4((qh >> (4 * i)) & 15u) << 4), c);
        c = mfma4(x.l[4 + i],
                  ((q[i] >> 4) & 0x0F0F0F0Fu) | (spread4((qh >> (16 + 4 * i)) & 15u) << 4), c);
    }
    return __builtin_amdgcn_ldexpf(h2f(d16) * comb4(c), x.e - 22);
}
RT_DEV float q5_0_block_dot(uint32_t d16, uint32_t qh, const uint32_t q[4], const XRegs& x) {
    int t0 = -16 * x.s[0], t1 = -16 * x.s[1], t2 = -16 * x.s[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (spread4((qh >> (4 * i)) & 15u) << 4);
        const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (spread4((qh >> (16 + 4 * i)) & 15u) << 4);
        t0 = sdot4(lo, x.l[0][i], t0);
        t1 = sdot4(lo, x.l[1][i], t1);
        t2 = sdot4(lo, x.l[2][i], t2);
        t0 = sdot4(hi, x.l[0][4 + i], t0);
        t1 = sdot4(hi, x.l[1][4 + i], t1);
        t2 = sdot4(hi, x.l[2][4 + i], t2);
    }
    return __builtin_amdgcn_ldexpf(h2f(d16) * limb_combine(t0, t1, t2), x.e - 22);
}

// Unit = two consecutive Q5_0 blocks (44 bytes, 4-byte aligned when a row
// holds an even number of blocks): 11 aligned dwords.
struct FmtQ5_0 {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 22, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t w[11]; };
    struct XU { XRegs x[2]; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        load_dwords<11>(row + (size_t)u * 44, r.w);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        load_xregs(recs + 2 * uu, xu.x[0]);
        load_xregs(recs + 2 * uu + 1, xu.x[1]);
    }
    // block A at byte 0 (d, qh @2, qs @6), block B at byte 22 (d, qh @24, qs @28)
    RT_DEV static void split(const Raw& r, uint32_t& da, uint32_t& qha, uint32_t qa[4],
                             uint32_t& db, uint32_t& qhb, uint32_t qb[4]) {
        da = r.w[0];
        qha = alignb(r.w[1], r.w[0], 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) qa[i] = alignb(r.w[2 + i], r.w[1 + i], 2);
        db = r.w[5] >> 16;
        qhb = r.w[6];
#pragma unroll
        for (int i = 0; i < 4; ++i) qb[i] = r.w[7 + i];
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t da, qha, qa[4], db, qhb, qb[4];
        split(r, da, qha, qa, db, qhb, qb);
        return q5_0_block_dot(da, qha, qa, xu.x[0]) + q5_0_block_dot(db, qhb, qb, xu.x[1]);
    }
    static constexpr bool XPAIR = true;
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        XLimb xa, xb;
        load_xlimb(xs + 2 * uu, lq, xa);
        load_xlimb(xs + 2 * uu + 1, lq, xb);
        return mdotx(r, xa, xb);
    }
    RT_DEV static float mdotx(const Raw& r, const XLimb& xa, const XLimb& xb) {
        uint32_t da, qha, qa[4], db, qhb, qb[4];
        split(r, da, qha, qa, db, qhb, qb);
        return q5_0_block_mdot(da, qha, qa, xa) + q5_0_block_mdot(db, qhb, qb, xb);
    }
};

// Single-block unit for rows with an odd number of blocks: 6 aligned dwords
// from the block's floor (never wholly past the block).
struct FmtQ5_0S {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 22, UNIT_EL = 32;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t w[6]; uint32_t sh; };
    struct XU { XRegs x; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uintptr_t p = (uintptr_t)(row + (size_t)u * 22);
        r.sh = (uint32_t)(p & 3);
        load_dwords<6>((const uint8_t*)(p & ~(uintptr_t)3), r.w);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) { load_xregs(recs + uu, xu.x); }
    RT_DEV static void split(const Raw& r, uint32_t& d, uint32_t& qh, uint32_t q[4]) {
        d = r.sh ? (r.w[0] >> 16) : r.w[0];
        qh = r.sh ? r.w[1] : alignb(r.w[1], r.w[0], 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = r.sh ? r.w[2 + i] : alignb(r.w[2 + i], r.w[1 + i], 2);
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t d, qh, q[4];
        split(r, d, qh, q);
        return q5_0_block_dot(d, qh, q, xu.x);
    }
};

// Q5_K (176 B, 16-byte aligned): d, dmin f16 @0, scales[12] @4 (Q4_K
// packing), qh[32] @16, qs[128] @48.  Unit (block, pair j) = 64 elements:
// the low nibbles of qs[32j..32j+31] (first sub-block of the pair) and the
// high nibbles (second), v = d·sc·q − dmin·m.  The fifth bit of element e:
//   reference layout: bit e%8 of qh[e/8] (forward.rs:979-1012), so the
//     unit's 64 bits are qh bytes 8j..8j+7 and sub-blocks pair as (j, j+4);
//   ggml layout (G): bit 2j (low half) / 2j+1 (high half) of qh[l] for
//     element 64j(+32)+l (dequantize_row_q5_K), sub-blocks (2j, 2j+1).
template <bool G>
struct FmtQ5KT {
    static constexpr uint32_t BLK_EL = 256, BLK_BYTES = 176, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    static constexpr int NQH = G ? 8 : 2;
    struct Raw { uint32_t dd; uint32_t sc; uint32_t qh[NQH]; uint32_t q[8]; uint32_t j2; };
    struct XU { XRegs lo, hi; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint32_t b = u >> 2, j = u & 3;
        const uint8_t* p = row + (size_t)b * 176;
        const u32x4 hdr = *(const u32x4*)p;
        r.dd = hdr.x;
        r.sc = k_quant_scales<G>(j, hdr.y, hdr.z, hdr.w);
        r.j2 = 2 * j;
        if (G) {
            const u32x4* hp = (const u32x4*)(p + 16);
            const u32x4 h0 = hp[0], h1 = hp[1];
            r.qh[0] = h0.x; r.qh[1] = h0.y; r.qh[2] = h0.z; r.qh[3] = h0.w;
            r.qh[NQH - 4] = h1.x; r.qh[NQH - 3] = h1.y; r.qh[NQH - 2] = h1.z; r.qh[NQH - 1] = h1.w;
        } else {
            const uint2 h = *(const uint2*)(p + 16 + 8 * j);
            r.qh[0] = h.x;
            r.qh[NQH - 1] = h.y;
        }
        const u32x4* qp = (const u32x4*)(p + 48 + 32 * j);
        const u32x4 a = qp[0], c = qp[1];
        r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
        r.q[4] = c.x; r.q[5] = c.y; r.q[6] = c.z; r.q[7] = c.w;
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        load_xregs(recs + 2 * uu, xu.lo);
        load_xregs(recs + 2 * uu + 1, xu.hi);
    }
    // 5-bit codes of elements 4i..4i+3 of the low / high half
    RT_DEV static uint32_t code_lo(const Raw& r, int i) {
        const uint32_t hb = G ? ((r.qh[i] >> r.j2) & 0x01010101u) : spread4((r.qh[0] >> (4 * i)) & 15u);
        return (r.q[i] & 0x0F0F0F0Fu) | (hb << 4);
    }
    RT_DEV static uint32_t code_hi(const Raw& r, int i) {
        const uint32_t hb = G ? ((r.qh[i] >> (r.j2 + 1)) & 0x01010101u)
                              : spread4((r.qh[NQH - 1] >> (4 * i)) & 15u);
        return ((r.q[i] >> 4) & 0x0F0F0F0Fu) | (hb << 4);
    }
    RT_DEV static void scales(const Raw& r, float& d_lo, float& m_lo, float& d_hi, float& m_hi) {
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        d_lo = d * (float)(r.sc & 255u);
        m_lo = dmin * (float)((r.sc >> 8) & 255u);
        d_hi = d * (float)((r.sc >> 16) & 255u);
        m_hi = dmin * (float)(r.sc >> 24);
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = code_lo(r, i), hi = code_hi(r, i);
            a0 = sdot4(lo, xu.lo.l[0][i], a0);
            a1 = sdot4(lo, xu.lo.l[1][i], a1);
            a2 = sdot4(lo, xu.lo.l[2][i], a2);
            b0 = sdot4(hi, xu.hi.l[0][i], b0);
            b1 = sdot4(hi, xu.hi.l[1][i], b1);
            b2 = sdot4(hi, xu.hi.l[2][i], b2);
        }
        float d_lo, m_lo, d_hi, m_hi;
        scales(r, d_lo, m_lo, d_hi, m_hi);
        const float vlo = d_lo * limb_combine(a0, a1, a2) -
                          m_lo * limb_combine(xu.lo.s[0], xu.lo.s[1], xu.lo.s[2]);
        const float vhi = d_hi * limb_combine(b0, b1, b2) -
                          m_hi * limb_combine(xu.hi.s[0], xu.hi.s[1], xu.hi.s[2]);
        return __builtin_amdgcn_ldexpf(vlo, xu.lo.e - 22) +
               __builtin_amdgcn_ldexpf(vhi, xu.hi.e - 22);
    }
    static constexpr bool XPAIR = true;
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        XLimb xl, xh;
        load_xlimb(xs + 2 * uu, lq, xl);
        load_xlimb(xs + 2 * uu + 1, lq, xh);
        return mdotx(r, xl, xh);
    }
    RT_DEV static float mdotx(const Raw& r, const XLimb& xl, const XLimb& xh) {
        v4i cl = {0, 0, 0, 0}, ch = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            cl = mfma4(xl.l[i], code_lo(r, i), cl);
            ch = mfma4(xh.l[i], code_hi(r, i), ch);
        }
        float d_lo, m_lo, d_hi, m_hi;
        scales(r, d_lo, m_lo, d_hi, m_hi);
        const float vlo = d_lo * comb4(cl) - m_lo * limb_combine(xl.s[0], xl.s[1], xl.s[2]);
        const float vhi = d_hi * comb4(ch) - m_hi * limb_combine(xh.s[0], xh.s[1], xh.s[2]);
        return __builtin_amdgcn_ldexpf(vlo, xl.e - 22) + __builtin_amdgcn_ldexpf(vhi, xh.e - 22);
    }
};
using FmtQ5K = FmtQ5KT<false>;
using FmtQ5KG = FmtQ5KT<true>;

// ─────────────────────── Q4_0, ggml layout ───────────────────────
// Block as Q4_0, but element j < 16 is the low nibble of qs[j] and element
// 16 + j its high nibble (dequantize_row_q4_0), value d·(nib − 8).  The
// activation records stay in natural order (no Q4_0 permutation).
RT_DEV float q4_0g_block_dot(uint32_t d16, const uint32_t q[4], const XRegs& x) {
    int t0 = -8 * x.s[0], t1 = -8 * x.s[1], t2 = -8 * x.s[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
        t0 = sdot4(lo, x.l[0][i], t0);
        t1 = sdot4(lo, x.l[1][i], t1);
        t2 = sdot4(lo, x.l[2][i], t2);
        t0 = sdot4(hi, x.l[0][4 + i], t0);
        t1 = sdot4(hi, x.l[1][4 + i], t1);
        t2 = sdot4(hi, x.l[2][4 + i], t2);
    }
    return __builtin_amdgcn_ldexpf(h2f(d16) * limb_combine(t0, t1, t2), x.e - 22);
}
RT_DEV float q4_0g_block_mdot(uint32_t d16, const uint32_t q[4], const XLimb& x) {
    v4i c = {-8 * x.s[0], -8 * x.s[1], -8 * x.s[2], 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c = mfma4(x.l[i], q[i] & 0x0F0F0F0Fu, c);
        c = mfma4(x.l[4 + i], (q[i] >> 4) & 0x0F0F0F0Fu, c);
    }
    return __builtin_amdgcn_ldexpf(h2f(d16) * comb4(c), x.e - 22);
}
// Unit = two consecutive blocks (36 bytes): 9 aligned dwords.
struct FmtQ4_0G {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 18, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t w[9]; };
    struct XU { XRegs x[2]; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        load_dwords<9>(row + (size_t)u * 36, r.w);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        load_xregs(recs + 2 * uu, xu.x[0]);
        load_xregs(recs + 2 * uu + 1, xu.x[1]);
    }
    RT_DEV static void split(const Raw& r, uint32_t qa[4], uint32_t qb[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qa[i] = alignb(r.w[i + 1], r.w[i], 2);  // bytes 2..17
            qb[i] = r.w[5 + i];                     // bytes 20..35
        }
    }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t qa[4], qb[4];
        split(r, qa, qb);
        return q4_0g_block_dot(r.w[0], qa, xu.x[0]) + q4_0g_block_dot(r.w[4] >> 16, qb, xu.x[1]);
    }
    static constexpr bool XPAIR = true;
    RT_DEV static float mdot(const Raw& r, const XRec* xs, uint32_t uu, uint32_t lq) {
        XLimb xa, xb;
        load_xlimb(xs + 2 * uu, lq, xa);
        load_xlimb(xs + 2 * uu + 1, lq, xb);
        return mdotx(r, xa, xb);
    }
    RT_DEV static float mdotx(const Raw& r, const XLimb& xa, const XLimb& xb) {
        uint32_t qa[4], qb[4];
        split(r, qa, qb);
        return q4_0g_block_mdot(r.w[0], qa, xa) + q4_0g_block_mdot(r.w[4] >> 16, qb, xb);
    }
};
// Single-block unit for rows with an odd number of blocks.
struct FmtQ4_0GS {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 18, UNIT_EL = 32;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t w[5]; uint32_t sh; };
    struct XU { XRegs x; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uintptr_t p = (uintptr_t)(row + (size_t)u * 18);
        r.sh = (uint32_t)(p & 3);
        load_dwords<5>((const uint8_t*)(p & ~(uintptr_t)3), r.w);
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) { load_xregs(recs + uu, xu.x); }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = r.sh ? r.w[i + 1] : alignb(r.w[i + 1], r.w[i], 2);
        return q4_0g_block_dot(alignb(r.w[1], r.w[0], r.sh), q, xu.x);
    }
};
