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

// ───────────────────────────── Q8_0 ─────────────────────────────
// Block: d:f16 @0, qs:int8[32] @2 (gemv_q8_0.metal:11-17; forward.rs:951-963).
struct FmtQ8_0 {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 34, UNIT_EL = 32;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t d; uint32_t q[8]; };
    struct XU { XRegs x; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint8_t* p = row + (size_t)u * 34;
        r.d = *(const uint16_t*)p;
        u32x4 a = *(const u32x4_a2*)(p + 2);
        u32x4 b = *(const u32x4_a2*)(p + 18);
        r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
        r.q[4] = b.x; r.q[5] = b.y; r.q[6] = b.z; r.q[7] = b.w;
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) { load_xregs(recs + uu, xu.x); }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            t0 = sdot4(r.q[i], xu.x.l[0][i], t0);
            t1 = sdot4(r.q[i], xu.x.l[1][i], t1);
            t2 = sdot4(r.q[i], xu.x.l[2][i], t2);
        }
        return __builtin_amdgcn_ldexpf(h2f(r.d) * limb_combine(t0, t1, t2), xu.x.e - 22);
    }
};

// ───────────────────────────── Q4_0 ─────────────────────────────
// Block: d:f16 @0, qs:u8[16] @2; element 2i = qs[i]&0xF, 2i+1 = qs[i]>>4,
// value d·(nib−8) (gemv_q4_0.metal:10-15; forward.rs:964-978).
struct FmtQ4_0 {
    static constexpr uint32_t BLK_EL = 32, BLK_BYTES = 18, UNIT_EL = 32;
    static constexpr bool Q40PERM = true;
    struct Raw { uint32_t d; uint32_t q[4]; };
    struct XU { XRegs x; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint8_t* p = row + (size_t)u * 18;
        r.d = *(const uint16_t*)p;
        u32x4 a = *(const u32x4_a2*)(p + 2);
        r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) { load_xregs(recs + uu, xu.x); }
    RT_DEV static float dot(const Raw& r, const XU& xu) {
        int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = r.q[i] & 0x0F0F0F0Fu;         // elements 8i+{0,2,4,6}
            const uint32_t hi = (r.q[i] >> 4) & 0x0F0F0F0Fu;  // elements 8i+{1,3,5,7}
            t0 = sdot4(lo, xu.x.l[0][2 * i], t0);
            t0 = sdot4(hi, xu.x.l[0][2 * i + 1], t0);
            t1 = sdot4(lo, xu.x.l[1][2 * i], t1);
            t1 = sdot4(hi, xu.x.l[1][2 * i + 1], t1);
            t2 = sdot4(lo, xu.x.l[2][2 * i], t2);
            t2 = sdot4(hi, xu.x.l[2][2 * i + 1], t2);
        }
        t0 -= 8 * xu.x.s[0];
        t1 -= 8 * xu.x.s[1];
        t2 -= 8 * xu.x.s[2];
        return __builtin_amdgcn_ldexpf(h2f(r.d) * limb_combine(t0, t1, t2), xu.x.e - 22);
    }
};

// ───────────────────────────── Q4_K ─────────────────────────────
// Super-block: d:f16 @0, dmin:f16 @2, scales:u8[12] @4, qs:u8[128] @16
// (dequant.metal:9-16).  Pair j ∈ 0..3: element 64j+l = d·sc_j·(qs[32j+l]&0xF)
// − dmin·m_j, element 64j+32+l uses the high nibble with (sc,m)_{j+4}
// (forward.rs:1026-1057; 6-bit (sc,m) per get_scale_min_k4, forward.rs:359-369).
struct FmtQ4K {
    static constexpr uint32_t BLK_EL = 256, BLK_BYTES = 144, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t dd; uint32_t sc; uint32_t q[8]; };
    struct XU { XRegs lo, hi; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint32_t b = u >> 2, j = u & 3;
        const uint8_t* p = row + (size_t)b * 144;
        const uint32_t* pw = (const uint32_t*)p;  // 144-byte blocks keep 4-byte alignment
        r.dd = pw[0];
        const uint32_t s0 = pw[1], s1 = pw[2], s2 = pw[3];
        // bytes j, j+4, j+8 of the scale table, packed as (b0 | b1<<8 | b2<<16)
        const uint32_t sh = 8 * j;
        r.sc = ((s0 >> sh) & 255u) | (((s1 >> sh) & 255u) << 8) | (((s2 >> sh) & 255u) << 16);
        const u32x4* qp = (const u32x4*)(p + 16 + 32 * j);
        u32x4 a = qp[0], c = qp[1];
        r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
        r.q[4] = c.x; r.q[5] = c.y; r.q[6] = c.z; r.q[7] = c.w;
    }
    RT_DEV static void load_x(const XRec* recs, uint32_t uu, XU& xu) {
        load_xregs(recs + 2 * uu, xu.lo);
        load_xregs(recs + 2 * uu + 1, xu.hi);
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
        const uint32_t c0 = r.sc & 255u, c1 = (r.sc >> 8) & 255u, c2 = (r.sc >> 16) & 255u;
        const uint32_t sc_lo = c0 & 63u, m_lo = c1 & 63u;
        const uint32_t sc_hi = (c2 & 15u) | ((c0 >> 6) << 4);
        const uint32_t m_hi = (c2 >> 4) | ((c1 >> 6) << 4);
        const float d = h2f(r.dd), dmin = h2f(r.dd >> 16);
        const float d_lo = d * (float)sc_lo, mm_lo = dmin * (float)m_lo;
        const float d_hi = d * (float)sc_hi, mm_hi = dmin * (float)m_hi;
        const float vlo = d_lo * limb_combine(a0, a1, a2) -
                          mm_lo * limb_combine(xu.lo.s[0], xu.lo.s[1], xu.lo.s[2]);
        const float vhi = d_hi * limb_combine(b0, b1, b2) -
                          mm_hi * limb_combine(xu.hi.s[0], xu.hi.s[1], xu.hi.s[2]);
        return __builtin_amdgcn_ldexpf(vlo, xu.lo.e - 22) +
               __builtin_amdgcn_ldexpf(vhi, xu.hi.e - 22);
    }
};

// ───────────────────────────── Q6_K ─────────────────────────────
// Super-block: ql:u8[128] @0, qh:u8[64] @128, sc:i8[16] @192, d:f16 @208.
// For half h ∈ {0,128}, l ∈ 0..31, t ∈ 0..3: element h+32t+l =
//   d · sc[h/16 + 2t] · (code_t − 32), code_t from ql[h/2+l (+32 if t odd)]
//   (low nibble for t<2, high for t≥2) and 2 bits (qh[h/4+l] >> 2t)
// (forward.rs:921-950; only the even scale slots are read, forward.rs:935).
struct FmtQ6K {
    static constexpr uint32_t BLK_EL = 256, BLK_BYTES = 210, UNIT_EL = 64;
    static constexpr bool Q40PERM = false;
    struct Raw { uint32_t ql0[4], ql1[4], qh[4]; uint32_t sc01, sc23; uint32_t d; };
    struct XHalf { uint32_t l[3][4]; int e; int s[3]; };
    struct XU { XHalf t[4]; };
    RT_DEV static void load(const uint8_t* row, uint32_t u, Raw& r) {
        const uint32_t b = u >> 2, hsel = (u >> 1) & 1, lh = u & 1;
        const uint8_t* p = row + (size_t)b * 210;
        const uint32_t h = hsel * 128;
        u32x4 a = *(const u32x4_a2*)(p + h / 2 + 16 * lh);
        u32x4 c = *(const u32x4_a2*)(p + h / 2 + 32 + 16 * lh);
        u32x4 e = *(const u32x4_a2*)(p + 128 + h / 4 + 16 * lh);
        u32x2_a2 s = *(const u32x2_a2*)(p + 192 + h / 16);
        r.ql0[0] = a.x; r.ql0[1] = a.y; r.ql0[2] = a.z; r.ql0[3] = a.w;
        r.ql1[0] = c.x; r.ql1[1] = c.y; r.ql1[2] = c.z; r.ql1[3] = c.w;
        r.qh[0] = e.x; r.qh[1] = e.y; r.qh[2] = e.z; r.qh[3] = e.w;
        r.sc01 = s.x;  // bytes 0..3: sc[is+0], (odd), sc[is+2], (odd)
        r.sc23 = s.y;  // bytes 4..7: sc[is+4], (odd), sc[is+6], (odd)
        r.d = *(const uint16_t*)(p + 208);
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
};
