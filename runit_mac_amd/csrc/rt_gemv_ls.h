// rt_gemv_ls.h — LDS-streamed M=1 GEMV body (matrix-core dots) for gfx950
// (instantiated by the kls_*.hip files).
//
// What limits an M=1 GEMV on MI355X is how the weight bytes are requested.
// Two properties set the achieved HBM rate:
//   * coalescing: a wave load of 64 lanes × 16 consecutive bytes (1 KB) is
//     served as 8 whole 128-byte lines; lanes that each walk their own 36..212
//     byte block touch ~20 lines per load instruction and stream ~15% slower;
//   * a compact front: all waves reading a window of the stream that moves
//     through memory together run ~10% faster than waves that each own one
//     long contiguous span (≥ 16 KB per wave).
// This body therefore:
//   1. splits the launch into items of one row quad (4 rows of one K chunk);
//      item j of wave w in workgroup g is quad g + nwg·(w + nwaves·j), so the
//      waves of the whole grid move through the quads together, and every
//      workgroup gets the same number of items to within one;
//   2. loads each row of an item with coalesced dwordx4 loads (lane l reads
//      bytes 16l.. of each KB) into registers, one item ahead, and writes
//      the item into a wave-private LDS slot just before computing it,
//      keeping the row's address modulo 16 so the block formats' alignment
//      assumptions hold (no workgroup barrier after the activation staging;
//      the compiler places every wait, which it cannot do for global→LDS
//      loads whose target it cannot tell apart from the slot being read);
//   3. computes the row-quad dots with the formats' matrix-core unit code
//      (F::load on the LDS copy, F::mdot against the activation records) and
//      collects the results in LDS, stored after the last item.
// Residual/bias operands are loaded once at the start (≤ 64 items per wave).
// A K split (S > 1 chunks) writes partial sums; the last chunk to arrive at a
// quad adds them in chunk order and runs the epilogue.
#pragma once
#include "rt_gemv.h"

constexpr uint32_t kLsGroup = 16;     // items per result store instruction
constexpr uint32_t kLsMaxGroups = 4;  // ≤ 64 items per wave

// Unit loader for a row in LDS: F::load_ls where a format has one (loaders
// that round the address with integer arithmetic would lose the LDS address
// space), else F::load.
template <class F>
RT_DEV auto ls_load(const uint8_t* row, uint32_t u, typename F::Raw& r, int) -> decltype(F::load_ls(row, u, r)) {
    return F::load_ls(row, u, r);
}
template <class F>
RT_DEV void ls_load(const uint8_t* row, uint32_t u, typename F::Raw& r, long) { F::load(row, u, r); }

// The unit dot of this lane's row: matrix-core form (F::mdot, lane q feeds
// limb lq of the quad's A operand), or, VALU, the format's v_dot4 form over
// all three limbs of the records (F::vdot where the format has one, else
// F::load_x + F::dot) — the same integer sums and the same result.
template <class F>
RT_DEV auto fmt_vdot(const typename F::Raw& r, const XRec* xs, uint32_t u, int)
    -> decltype(F::vdot(r, xs, u)) {
    return F::vdot(r, xs, u);
}
template <class F>
RT_DEV float fmt_vdot(const typename F::Raw& r, const XRec* xs, uint32_t u, long) {
    typename F::XU xu;
    F::load_x(xs, u, xu);
    return F::dot(r, xu);
}
// Formats whose unit takes two whole records, with F::mdotx(raw, limbs of
// record 0, limbs of record 1) (the limbs can then be held in registers).
template <class F>
constexpr auto fmt_xpair(int) -> decltype(F::XPAIR, bool()) { return F::XPAIR; }
template <class F>
constexpr bool fmt_xpair(long) { return false; }

template <class F, bool VALU>
RT_DEV float ls_dot(const typename F::Raw& r, const XRec* xs, uint32_t u, uint32_t lq) {
    if constexpr (VALU) return fmt_vdot<F>(r, xs, u, 0);
    else return F::mdot(r, xs, u, lq);
}

template <class F, int EPI, typename XT, int NI, bool VALU = false>
RT_DEV void gemv_ls_body(const GemvArgs& a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nwaves = wg_threads() >> 6;
    const uint32_t q = lane & 3, slot = lane >> 2;
    const uint32_t lq = q < 3 ? q : 2;  // the A row of lane q = 3 is a don't-care
    const uint32_t S = a.ksplit;
    const uint32_t ks = blockIdx.x % S, nwg = gridDim.x / S;
    // Workgroups are dealt to the 8 XCDs in turn (block b → XCD b mod 8).
    // Without a K split, renumber them so that neighbouring row quads, which
    // share the cache lines at their ends, go to workgroups on one XCD (one
    // L2) instead of to eight.
    const uint32_t wg = (S == 1 && a.ls_xcd && nwg % 8 == 0)
                            ? (blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8
                            : blockIdx.x / S;
    const uint32_t cu0 = ks * a.kc_units;  // first unit of this workgroup's K chunk
    const uint32_t units = min(a.K / F::UNIT_EL - cu0, a.kc_units);
    const uint32_t cbyte0 = cu0 * F::UNIT_EL / F::BLK_EL * F::BLK_BYTES;  // chunk offset in a row
    const uint32_t cbytes = units * F::UNIT_EL / F::BLK_EL * F::BLK_BYTES;
    const uint32_t nxb = units * F::UNIT_EL / 32, xb0 = cu0 * F::UNIT_EL / 32;
    const uint32_t xcap = a.kc_units * F::UNIT_EL / 32 * XREC_BYTES;
    XRec* xs = (XRec*)smem;
    // per wave: a result buffer of a.ls_res items (a multiple of 16, ≤ 64)
    float* res = (float*)(smem + xcap) + wave * (a.ls_res * 4);
    const uint32_t RS = a.ls_rs;  // LDS bytes between two rows of the slot
    uint8_t* wslot = smem + xcap + nwaves * a.ls_res * 16 + wave * (4 * RS);
    const uint32_t nq = (a.nvrows + 3) / 4;
    const uint32_t first = wg + nwg * wave, stride = nwg * nwaves;
    const uint32_t nitems = first < nq ? (nq - first + stride - 1) / stride : 0;
    auto quad_of = [&](uint32_t j) { return first + stride * j; };

    // chunk start of virtual row vr (clamped into the launch)
    auto row_src = [&](uint32_t vr) -> const uint8_t* {
        if (vr >= a.nvrows) vr = a.nvrows - 1;
        uint32_t mat, r;
        vrow_map<EPI>(a, vr, mat, r);
        return mat_w(a, mat) + (size_t)r * a.row_bytes + cbyte0;
    };
    // coalesced loads of item j's four row chunks: NI dwordx4 per lane and
    // row from the chunk's 16-byte floor (lanes past the chunk re-read its
    // last 16 bytes).  An item past the wave's last issues the same loads
    // with no records in their descriptor (dropped, no memory access), so
    // that every loop iteration issues the same loads and the compiler's
    // waits stay exact.  (Re-reading the last item instead fetched 7% more
    // than the weight bytes: some of those lines had left the L2.)
    typedef u32x4 Item[4][NI];
    auto issue = [&](uint32_t j, Item& dst) {
        const bool none = j >= nitems;
        const uint32_t quad = quad_of(min(j, nitems - 1));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint8_t* src = row_src(quad * 4 + r);
            const uint8_t* base = src - ((uintptr_t)src & 15);
            const uint32_t last = (uint32_t)(((uintptr_t)src & 15) + cbytes - 1) & ~15u;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t off = min((uint32_t)(i * 64 + lane) * 16, last);
                dst[r][i] = load16_or_none(base, off, none);
            }
        }
    };
    // the item's bytes into the wave's LDS slot (row r at r·RS, keeping the
    // chunk's address modulo 16)
    auto commit = [&](const Item& src) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < NI; ++i) *(u32x4*)(wslot + r * RS + (i * 64 + lane) * 16) = src[r][i];
    };

    // epilogue operands of the lanes' result slots (lane l of group g: item
    // 16g + l/4, row l%4), loaded before any weight
    float aux[kLsMaxGroups];
#pragma unroll
    for (uint32_t g = 0; g < kLsMaxGroups; ++g) {
        aux[g] = 0.0f;
        if (has_aux<EPI>()) {
            const uint32_t jj = g * kLsGroup + slot;
            const uint32_t vr = (jj < nitems ? quad_of(jj) : 0) * 4 + q;
            aux[g] = load_aux<EPI>(a, vr < a.nvrows ? vr : a.nvrows - 1);
        }
    }
    auto pick_aux = [&](uint32_t g) {
        return g == 0 ? aux[0] : (g == 1 ? aux[1] : (g == 2 ? aux[2] : aux[3]));
    };

    // activation loads, then the first two items' weights, then the
    // conversion (which waits for the activations only)
    const bool one_pass = !a.x_rec && stage_one_pass(nxb);
    XPre xp;
    if (one_pass)
        stage_x_load<XT>((const XT*)a.x + (size_t)xb0 * 32,
                         a.gamma ? a.gamma + (size_t)xb0 * 32 : nullptr, nxb, xp);
    Item buf;
    issue(0, buf);
    if (one_pass)
        stage_x_convert<F::Q40PERM>(xp, a.gamma, a.eps, nxb, xs);
    else
        copy_x_limbs((const XRec*)a.x, xb0, nxb, xs);
    lds_barrier();

    // results of group g (items 16g .. 16g + n - 1): one store per lane
    auto flush = [&](uint32_t g, uint32_t n) {
        const uint32_t jj = g * kLsGroup + slot;
        const float v = res[g * 64 + lane];
        const uint32_t vr = (jj < nitems ? quad_of(jj) : 0) * 4 + q;
        const bool ok = slot < n && vr < a.nvrows;
        if (S > 1) {
            if (ok) dev_store(a.part + (size_t)ks * a.nvrows + vr, v);
        } else if (EPI == EPI_FFN) {
            // quad rows (gate r, up r, gate r+1, up r+1)
            const float up = dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(v);
            if (ok && (q & 1) == 0 && vr + 1 < a.nvrows)
                ((float*)a.out[0])[vr >> 1] = silu_ref(v) * up;
        } else {
            if (ok) store_row_pre<EPI>(a, vr, v, pick_aux(g));
        }
    };

    const uint32_t nsteps = (units + 15) / 16;
    // One item in flight: item j is written to the slot, item j+1's loads
    // are issued, item j is computed.  (Two items in flight per wave stream
    // slower: the extra outstanding requests only queue.)  Results wait in
    // LDS until the end.
    for (uint32_t j = 0; j < nitems; ++j) {
        commit(buf);
        issue(j + 1, buf);
        // this lane's row in the slot
        const uint8_t* rowl = wslot + q * RS + ((uintptr_t)row_src(quad_of(j) * 4 + q) & 15);
        float acc = 0.0f;
        for (uint32_t st = 0; st < nsteps; ++st) {
            const uint32_t u = slot + 16 * st;
            const bool valid = u < units;
            const uint32_t uc = valid ? u : 0;
            typename F::Raw raw;
            ls_load<F>(rowl, uc, raw, 0);
            const float v = ls_dot<F, VALU>(raw, xs, uc, lq);
            acc += valid ? v : 0.0f;
        }
        // sum over the 16 slots of the row (lane bits 2..5)
        acc += swz_xor_f<4>(acc);
        acc += swz_xor_f<8>(acc);
        acc += swz_xor_f<16>(acc);
        acc += __shfl_xor(acc, 32, 64);
        if (slot == 0) res[j * 4 + q] = acc;
    }
#pragma unroll
    for (uint32_t g = 0; g < kLsMaxGroups; ++g) {
        if (g * kLsGroup >= nitems) break;  // uniform
        flush(g, min(nitems - g * kLsGroup, kLsGroup));
    }

    if (S > 1) {
        // K split: count this chunk in at each of the wave's quads (lane of
        // row 0 of the item), then the last chunk to arrive sums the chunks
        // in order and runs the epilogue
        dev_stores_done();
#pragma unroll
        for (uint32_t g = 0; g < kLsMaxGroups; ++g) {
            if (g * kLsGroup >= nitems) break;  // uniform
            const uint32_t jj = g * kLsGroup + slot;
            const bool have = jj < nitems;
            const uint32_t quad = have ? quad_of(jj) : 0;
            uint32_t last = 0;
            if (have && q == 0) last = arrive(a.counters + (size_t)quad * a.cstride) == S - 1;
            last = __shfl(last, lane & ~3u, 64);
            if (!last) continue;
            const uint32_t vr = quad * 4 + q;
            float v = 0.0f;
            for (uint32_t c = 0; c < S; ++c)
                v += dev_load(a.part + (size_t)c * a.nvrows + (vr < a.nvrows ? vr : a.nvrows - 1));
            if (EPI == EPI_FFN) {
                const float up = __shfl_xor(v, 1, 64);
                if ((q & 1) == 0 && vr + 1 < a.nvrows) ((float*)a.out[0])[vr >> 1] = silu_ref(v) * up;
            } else if (vr < a.nvrows) {
                store_row_pre<EPI>(a, vr, v, pick_aux(g));
            }
            if (q == 0) dev_store(a.counters + (size_t)quad * a.cstride, 0u);  // ready for the next call
        }
    }
}

// Workgroup-local K split (rows longer than the slot, few row quads: the 7B
// down projections).  Each workgroup owns row quads g, g + nwg, ... and all K
// chunks of each; its waves take (quad, chunk) items in turn (item i: quad
// i / S, chunk i % S), so the partial sums of a row meet in LDS instead of
// through memory and arrival counters.  The activation records of the whole
// K are staged once per workgroup.  After the last item a barrier, then the
// chunks of each row are added in chunk order and the epilogue runs.
template <class F, int EPI, typename XT, int NI, bool VALU = false>
RT_DEV void gemv_lsk_body(const GemvArgs& a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nwaves = wg_threads() >> 6;
    const uint32_t q = lane & 3, slot = lane >> 2;
    const uint32_t lq = q < 3 ? q : 2;
    const uint32_t S = a.ksplit;          // K chunks of a row (all in this workgroup)
    const uint32_t kcu = a.kc_units;      // units per chunk (the last may be shorter)
    const uint32_t wg = blockIdx.x, nwg = gridDim.x;
    const uint32_t units_all = a.K / F::UNIT_EL;
    const uint32_t nxb_all = a.K / 32;
    XRec* xs = (XRec*)smem;
    const uint32_t xcap = nxb_all * XREC_BYTES;
    const uint32_t nq = (a.nvrows + 3) / 4;
    const uint32_t nql = wg < nq ? (nq - wg + nwg - 1) / nwg : 0;  // this workgroup's quads
    float* res = (float*)(smem + xcap);                              // [nql][S][4]
    const uint32_t RS = a.ls_rs;
    uint8_t* wslot = smem + xcap + a.ls_res * 16 + wave * (4 * RS);
    const uint32_t nitems_wg = nql * S;
    const uint32_t nitems = wave < nitems_wg ? (nitems_wg - wave + nwaves - 1) / nwaves : 0;
    auto item_of = [&](uint32_t j) { return wave + nwaves * j; };  // workgroup item index

    auto row_src = [&](uint32_t vr, uint32_t c) -> const uint8_t* {
        if (vr >= a.nvrows) vr = a.nvrows - 1;
        uint32_t mat, r;
        vrow_map<EPI>(a, vr, mat, r);
        return mat_w(a, mat) + (size_t)r * a.row_bytes + c * kcu * F::UNIT_EL / F::BLK_EL * F::BLK_BYTES;
    };
    auto chunk_units = [&](uint32_t c) { return min(units_all - c * kcu, kcu); };
    typedef u32x4 Item[4][NI];
    auto issue = [&](uint32_t j, Item& dst) {  // (past the last item: dropped loads)
        const bool none = j >= nitems;
        const uint32_t it = item_of(min(j, nitems - 1));
        const uint32_t quad = wg + nwg * (it / S), c = it % S;
        const uint32_t cbytes = chunk_units(c) * F::UNIT_EL / F::BLK_EL * F::BLK_BYTES;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint8_t* src = row_src(quad * 4 + r, c);
            const uint8_t* base = src - ((uintptr_t)src & 15);
            const uint32_t last = (uint32_t)(((uintptr_t)src & 15) + cbytes - 1) & ~15u;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t off = min((uint32_t)(i * 64 + lane) * 16, last);
                dst[r][i] = load16_or_none(base, off, none);
            }
        }
    };
    auto commit = [&](const Item& src) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < NI; ++i) *(u32x4*)(wslot + r * RS + (i * 64 + lane) * 16) = src[r][i];
    };

    // epilogue operand of this thread's row (thread t < 4·nql: quad t/4, row t%4)
    float aux = 0.0f;
    if (has_aux<EPI>()) {
        const uint32_t vr = (wg + nwg * min(tid >> 2, nql ? nql - 1 : 0)) * 4 + (tid & 3);
        aux = load_aux<EPI>(a, vr < a.nvrows ? vr : a.nvrows - 1);
    }
    // activation loads, then the first item's weights, then the conversion
    // (which waits for the activations only: loads complete in issue order,
    // so staging behind the weight loads would wait for HBM)
    constexpr int XU = 5;  // slices per thread: K ≤ 20,480 at 1024 threads
    const bool one_pass = !a.x_rec && stage_one_pass<XU>(nxb_all);
    XPreU<XU> xp;
    if (one_pass) stage_x_load<XT, XU, true>((const XT*)a.x, a.gamma, nxb_all, xp);
    // When the waves divide evenly over the chunks, wave w only ever takes
    // chunk w mod S (item w + nwaves·j): the activation limbs of its lanes'
    // units (≤ 2 steps of 16 units) are then read from LDS once and held in
    // registers for all its items.
    constexpr bool XP = fmt_xpair<F>(0) && !VALU;
    const bool xreg = XP && nwaves % S == 0 && kcu <= 32;
    __shared__ uint32_t qcnt[16];  // per chunk: quads taken past the dealt ones
    if (tid < 16) qcnt[tid] = 0;   // (ordered before use by the staging barrier)
    Item buf;
    issue(0, buf);
    if (one_pass)
        stage_x_convert<F::Q40PERM, true>(xp, a.gamma, a.eps, nxb_all, xs);
    else
        stage_x<XT, F::Q40PERM>(a.x, a.x_rec != 0, 0, nxb_all, xs, a.gamma, a.eps);
    lds_barrier();

    if constexpr (XP) {
        if (xreg) {
            const uint32_t c = wave % S;
            const uint32_t units = chunk_units(c);
            const XRec* xc = xs + c * kcu * F::UNIT_EL / 32;
            XLimb xa[2], xb[2];
#pragma unroll
            for (uint32_t st = 0; st < 2; ++st) {
                const uint32_t u = slot + 16 * st;
                const uint32_t uc = u < units ? u : 0;
                load_xlimb(xc + 2 * uc, lq, xa[st]);
                load_xlimb(xc + 2 * uc + 1, lq, xb[st]);
            }
            const uint32_t nsteps = (units + 15) / 16;
            // quad ql of this wave's chunk: loads of its four row chunks
            // (ql ≥ nql: dropped)
            auto issue_q = [&](uint32_t ql, Item& dst) {
                const bool none = ql >= nql;
                const uint32_t quad = wg + nwg * min(ql, nql - 1);
                const uint32_t cbytes = units * F::UNIT_EL / F::BLK_EL * F::BLK_BYTES;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint8_t* src = row_src(quad * 4 + r, c);
                    const uint8_t* base = src - ((uintptr_t)src & 15);
                    const uint32_t last = (uint32_t)(((uintptr_t)src & 15) + cbytes - 1) & ~15u;
#pragma unroll
                    for (int i = 0; i < NI; ++i) {
                        const uint32_t off = min((uint32_t)(i * 64 + lane) * 16, last);
                        dst[r][i] = load16_or_none(base, off, none);
                    }
                }
            };
            // the next quad of the wave's chunk from the workgroup's counter
            // (the first nwaves / S quads of each chunk are dealt statically)
            auto draw = [&]() -> uint32_t {
                uint32_t v = 0;
                if (lane == 0) v = __hip_atomic_fetch_add(&qcnt[c], 1u, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_WORKGROUP);
                return nwaves / S + __builtin_amdgcn_readfirstlane(v);
            };
            // quad ql from the wave's slot
            auto work = [&](uint32_t ql) {
                const uint32_t it = ql * S + c;
                const uint8_t* rowl =
                    wslot + q * RS + ((uintptr_t)row_src((wg + nwg * ql) * 4 + q, c) & 15);
                float acc = 0.0f;
#pragma unroll
                for (uint32_t st = 0; st < 2; ++st) {
                    if (st < nsteps) {  // (uniform)
                        const uint32_t u = slot + 16 * st;
                        const bool valid = u < units;
                        typename F::Raw raw;
                        ls_load<F>(rowl, valid ? u : 0, raw, 0);
                        const float v = F::mdotx(raw, xa[st], xb[st]);
                        acc += valid ? v : 0.0f;
                    }
                }
                acc += swz_xor_f<4>(acc);
                acc += swz_xor_f<8>(acc);
                acc += swz_xor_f<16>(acc);
                acc += __shfl_xor(acc, 32, 64);
                if (slot == 0) res[it * 4 + q] = acc;
            };
            // One item in flight (two per wave streamed slower: 7B Q4_K FFN
            // 18.3 → 19.8 µs, Q4_0 17.3 → 18.7 µs).  After its first quad a
            // wave takes the next quad of its chunk from the workgroup's
            // counter, drawn one item ahead: waves whose data comes back
            // sooner take more quads, instead of the workgroup waiting for
            // its slowest wave's fixed share.
            uint32_t qcur = wave / S;
            uint32_t qnext = qcur < nql ? draw() : nql;
            while (qcur < nql) {
                commit(buf);
                issue_q(qnext, buf);
                const uint32_t qnn = qnext < nql ? draw() : nql;
                work(qcur);
                qcur = qnext;
                qnext = qnn;
            }
            goto combine;
        }
    }
    for (uint32_t j = 0; j < nitems; ++j) {
        commit(buf);
        issue(j + 1, buf);
        const uint32_t it = item_of(j);
        const uint32_t ql = it / S, c = it % S;
        const uint32_t units = chunk_units(c);
        const uint8_t* rowl = wslot + q * RS + ((uintptr_t)row_src((wg + nwg * ql) * 4 + q, c) & 15);
        const XRec* xc = xs + c * kcu * F::UNIT_EL / 32;
        const uint32_t nsteps = (units + 15) / 16;
        float acc = 0.0f;
        for (uint32_t st = 0; st < nsteps; ++st) {
            const uint32_t u = slot + 16 * st;
            const bool valid = u < units;
            const uint32_t uc = valid ? u : 0;
            typename F::Raw raw;
            ls_load<F>(rowl, uc, raw, 0);
            const float v = ls_dot<F, VALU>(raw, xc, uc, lq);
            acc += valid ? v : 0.0f;
        }
        acc += swz_xor_f<4>(acc);
        acc += swz_xor_f<8>(acc);
        acc += swz_xor_f<16>(acc);
        acc += __shfl_xor(acc, 32, 64);
        if (slot == 0) res[it * 4 + q] = acc;
    }
combine:
    __syncthreads();
    if (tid < 4 * nql) {
        const uint32_t ql = tid >> 2, r = tid & 3;
        const uint32_t vr = (wg + nwg * ql) * 4 + r;
        float v = 0.0f, v1 = 0.0f;
        for (uint32_t c = 0; c < S; ++c) {
            v += res[(ql * S + c) * 4 + r];
            if (EPI == EPI_FFN && r + 1 < 4) v1 += res[(ql * S + c) * 4 + r + 1];
        }
        if (EPI == EPI_FFN) {
            // quad rows (gate r, up r, gate r+1, up r+1)
            if ((r & 1) == 0 && vr + 1 < a.nvrows) ((float*)a.out[0])[vr >> 1] = silu_ref(v) * v1;
        } else if (vr < a.nvrows) {
            store_row_pre<EPI>(a, vr, v, aux);
        }
    }
}

// Small-launch body (M = 1, whole K in one staging pass, about one row quad
// per wave: the 0.5B model's norm-fused Q/K/V, attention-merging O and
// norm-fused gate+up launches).  These launches are bound by the chain
// before their first dot, not by their 1-9 MB of weights, and per-workgroup
// timestamps show where that chain goes on the matrix-core body: its lanes'
// strided 68-byte units touch ~34 cache lines per load instruction, so
// issuing a workgroup's weight loads backs up the CU's address unit for
// ~0.7 µs, and the staging barriers then wait ~1.9 µs for the slowest wave.
// Here every row of a quad is read with NI coalesced 1 KB loads (8 lines per
// instruction), the activation loads go out first, the quad goes through the
// wave's LDS slot (as in gemv_ls_body), and the result is stored right after
// the dot: no result buffer, no second item in flight.
template <class F, int EPI, typename XT, int NI>
RT_DEV void gemv_sm_body(const GemvArgs& a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nwaves = wg_threads() >> 6;
    const uint32_t q = lane & 3, slot = lane >> 2;
    const uint32_t lq = q < 3 ? q : 2;  // the A row of lane q = 3 is a don't-care
    const uint32_t units = a.K / F::UNIT_EL;
    const uint32_t cbytes = units * F::UNIT_EL / F::BLK_EL * F::BLK_BYTES;  // a whole row
    const uint32_t nxb = a.K / 32;
    XRec* xs = (XRec*)smem;
    const uint32_t RS = a.ls_rs;
    uint8_t* wslot = smem + nxb * XREC_BYTES + wave * (4 * RS);
    const uint32_t nq = (a.nvrows + 3) / 4;
    // the waves of a workgroup take neighbouring quads (one contiguous run
    // of rows per workgroup), then the next run of the grid (in a two-part
    // launch: of this part's workgroups [blk0, blk0 + nblk))
    const uint32_t bid = a.nblk ? blockIdx.x - a.blk0 : blockIdx.x;
    const uint32_t nbid = a.nblk ? a.nblk : gridDim.x;
    const uint32_t first = bid * nwaves + wave, stride = nbid * nwaves;
    const uint32_t nitems = first < nq ? (nq - first + stride - 1) / stride : 0;
    auto row_src = [&](uint32_t vr) -> const uint8_t* {
        if (vr >= a.nvrows) vr = a.nvrows - 1;
        uint32_t mat, r;
        vrow_map<EPI>(a, vr, mat, r);
        return mat_w(a, mat) + (size_t)r * a.row_bytes;
    };
    typedef u32x4 Item[4][NI];
    auto issue = [&](uint32_t j, Item& dst) {
        const uint32_t quad = first + stride * min(j, nitems ? nitems - 1 : 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint8_t* src = row_src(quad * 4 + r);
            const uint8_t* base = src - ((uintptr_t)src & 15);
            const uint32_t last = (uint32_t)(((uintptr_t)src & 15) + cbytes - 1) & ~15u;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t off = min((uint32_t)(i * 64 + lane) * 16, last);
                dst[r][i] = *(const u32x4*)(base + off);
            }
        }
    };
    auto commit = [&](const Item& src) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < NI; ++i) *(u32x4*)(wslot + r * RS + (i * 64 + lane) * 16) = src[r][i];
    };
    // activations first, then the weights and the epilogue operand of the
    // lane's row of the first quad, then the conversion (which waits for the
    // activations only)
    XPre xp;
    XPreAttn xa;
    if constexpr (is_attn_x<XT>())
        stage_attn_load<false>(a.x, a.xml, a.xnsp, a.xhd, nxb, xa);
    else
        stage_x_load<XT>((const XT*)a.x, a.gamma, nxb, xp, a.ssq_in, a.ssq_n);
    Item buf;
    issue(0, buf);
    float aux = 0.0f;
    if (has_aux<EPI>() && nitems) {
        const uint32_t vr = first * 4 + q;
        aux = load_aux<EPI>(a, vr < a.nvrows ? vr : a.nvrows - 1);
    }
    if constexpr (is_attn_x<XT>())
        stage_attn_convert<F::Q40PERM>(xa, a.xnsp, nxb, xs);
    else
        stage_x_convert<F::Q40PERM>(xp, a.gamma, a.eps, nxb, xs, a.ssq_in != nullptr);
    lds_barrier();

    const uint32_t nsteps = (units + 15) / 16;
    for (uint32_t j = 0; j < nitems; ++j) {
        commit(buf);
        const uint32_t quad = first + stride * j;
        if (j + 1 < nitems) issue(j + 1, buf);
        const uint8_t* rowl = wslot + q * RS + ((uintptr_t)row_src(quad * 4 + q) & 15);
        float acc = 0.0f;
        for (uint32_t st = 0; st < nsteps; ++st) {
            const uint32_t u = slot + 16 * st;
            const bool valid = u < units;
            const uint32_t uc = valid ? u : 0;
            typename F::Raw raw;
            ls_load<F>(rowl, uc, raw, 0);
            const float v = F::mdot(raw, xs, uc, lq);
            acc += valid ? v : 0.0f;
        }
        // sum over the 16 slots of the row (lane bits 2..5): every lane of
        // the row gets the total
        acc += swz_xor_f<4>(acc);
        acc += swz_xor_f<8>(acc);
        acc += swz_xor_f<16>(acc);
        acc += __shfl_xor(acc, 32, 64);
        const uint32_t vr = quad * 4 + q;
        if (j > 0 && has_aux<EPI>()) aux = load_aux<EPI>(a, vr < a.nvrows ? vr : a.nvrows - 1);
        if (EPI == EPI_FFN) {
            // quad rows (gate r, up r, gate r+1, up r+1)
            const float up = dpp_f<DPP_QUAD_PERM(1, 0, 3, 2)>(acc);
            if (slot == 0 && (q & 1) == 0 && vr + 1 < a.nvrows)
                ((float*)a.out[0])[vr >> 1] = silu_ref(acc) * up;
        } else {
            if (slot == 0 && vr < a.nvrows) store_row_pre<EPI>(a, vr, acc, aux);
            if (epi_base(EPI) == EPI_F32_ADD && a.ssq_out && slot == 0)
                quad_ssq_store(a.ssq_out, quad, acc + aux, vr < a.nvrows, q);
        }
    }
}

// Kernels: one per (format, epilogue, activation type, loads per row NI).
// Built for up to 1024 threads (≤ 128 registers: 16 waves per CU share one
// copy of the activation records), except Q6_K, whose whole-super-block
// units need ~270 registers (256 threads).
#define RT_GEMV_LS1(NAME, FMT, EPI, XT, NI, LB) \
    extern "C" __global__ void __launch_bounds__(LB) NAME##_ls##NI(GemvArgs a) { gemv_ls_body<FMT, EPI, XT, NI>(a); }
#define RT_GEMV_LSB(NAME, FMT, EPI, XT, LB) \
    RT_GEMV_LS1(NAME, FMT, EPI, XT, 1, LB) RT_GEMV_LS1(NAME, FMT, EPI, XT, 2, LB) RT_GEMV_LS1(NAME, FMT, EPI, XT, 3, LB)
#define RT_GEMV_LSK(NAME, FMT, EPI, XT, LB) \
    extern "C" __global__ void __launch_bounds__(LB) NAME##_lsk1(GemvArgs a) { gemv_lsk_body<FMT, EPI, XT, 1>(a); }
#define RT_GEMV_LS(NAME, FMT, EPI, XT) RT_GEMV_LSB(NAME, FMT, EPI, XT, 1024)
// The VALU-dot twins (<name>_ls<NI>v) of a kernel set, for the A/B of the two
// dot forms (selected by the context's gemv_valu switch)
#define RT_GEMV_LS1V(NAME, FMT, EPI, XT, NI, LB)                                            \
    extern "C" __global__ void __launch_bounds__(LB) NAME##_ls##NI##v(GemvArgs a) {        \
        gemv_ls_body<FMT, EPI, XT, NI, true>(a);                                           \
    }
#define RT_GEMV_LSBV(NAME, FMT, EPI, XT, LB) \
    RT_GEMV_LS1V(NAME, FMT, EPI, XT, 1, LB) RT_GEMV_LS1V(NAME, FMT, EPI, XT, 2, LB) RT_GEMV_LS1V(NAME, FMT, EPI, XT, 3, LB)


// Small-launch kernels (gemv_sm_body): <name>_sm<NI>, 256 threads.
#define RT_GEMV_SM1(NAME, FMT, EPI, XT, NI) \
    extern "C" __global__ void __launch_bounds__(256) NAME##_sm##NI(GemvArgs a) { gemv_sm_body<FMT, EPI, XT, NI>(a); }
#define RT_GEMV_SM(NAME, FMT, EPI, XT) RT_GEMV_SM1(NAME, FMT, EPI, XT, 1) RT_GEMV_SM1(NAME, FMT, EPI, XT, 2)
