// k_step.hip — a whole decode step of a Q8_0 Qwen2-shape model as ONE
// persistent launch (embedding and every layer; the LM head and the argmax
// follow as two ordinary launches).
//
// The per-layer sequence of forward.rs:1494-1771 is a chain of dependent
// phases — RMSNorm + Q/K/V (+ bias), RoPE + KV write + attention, O
// (+ residual), RMSNorm + gate/up + SiLU, down (+ residual) — each of which
// needs the whole output of the one before.  As separate kernels each costs a
// launch, the workgroups' start skew, the first memory round trips and the
// drain, ~5.7 µs at the 0.5B shapes for 1–9 MB of weights.  Here one grid of
// workgroups (one per CU, all resident) runs every phase in turn and meets at
// a grid barrier between phases.  The weights of a phase do not depend on
// the phase before it, so each workgroup issues its first weight loads (and,
// for attention, its first KV-cache rows) BEFORE waiting at the barrier:
// they arrive while the grid waits, and after the barrier only the
// activation loads, the dot and the stores remain.
//
// Phases are described by an array of StepPhase records built by the host
// (runtime.cpp, rt_decode_step_*): the GEMV phases run the matrix-core body
// of rt_gemv.h (gemv_mq_body) and attention runs attn_split of
// rt_attn.h, with device-scope activation loads and stores (every
// activation is produced and consumed by different workgroups of the same
// launch; no cache may return a stale copy, and no cache-wide write-back or
// invalidate is needed).
//
// Grid barrier: a workgroup ends a phase by waiting for its own stores and
// adding 1 to the arrival counter of its XCD (workgroup b runs on XCD b mod
// 8; each counter on its own 128-byte line, so at most G/8 atomics meet on
// one address); the next phase waits until every XCD's counter has reached
// (phases completed) × (that XCD's workgroups), 8 lanes of one wave reading
// the 8 counters per poll.  (Measured on a grid of 256 × 1024 threads: 1.5
// µs per barrier, against 3.7 µs for one flag per workgroup polled by every
// workgroup.)  The counters only grow: `base`, the phases of all earlier
// launches, is read at the start of a launch and advanced by the last
// workgroup to leave, so nothing needs clearing.  Every wait is bounded:
// after kStepSpinTicks of the 100 MHz real-time clock (50 ms) the workgroup
// records the timeout in the status word and goes on, so the launch always
// ends; the host reports a set status as an error.
#include "rt_attn.h"
#include "rt_gemv.h"
#include "rt_shared.h"

enum StepKind : uint32_t {
    SK_EMBED_Q8_0 = 0,  // x = dequant(table row *token)
    SK_QKV_Q8_0 = 1,    // RMSNorm + fused Q/K/V + bias
    SK_ATTN_HD64 = 2,   // RoPE + KV write + split attention (partials)
    SK_OPROJ_Q8_0 = 3,  // O (staging merges the partials) + residual
    SK_FFN_Q8_0 = 4,    // RMSNorm + gate/up + SiLU
    SK_DOWN_Q8_0 = 5,   // down + residual
};

struct StepPhase {
    uint32_t kind;
    uint32_t n0, n1, n2;   // embed: k; attention: splits, (kv head, head block) pairs
    const void* p0;        // embed: table
    const void* p1;        // embed: token id (device)
    void* p2;              // embed: output
    uint64_t pad;
    GemvArgs g;            // GEMV phases
    AttnArgs at;           // attention
};
static_assert(sizeof(StepPhase) == RT_STEP_PHASE_BYTES, "StepPhase layout");

struct StepSync {
    uint32_t ctr[8][32];    // per-XCD arrival counters, one 128-byte line each
    uint32_t base;          // phases completed by all earlier launches
    uint32_t pad0[31];
    uint32_t exits;         // workgroups that have left this launch
    uint32_t pad1[31];
    uint32_t status;        // non-zero: a barrier wait timed out
};
static_assert(sizeof(StepSync) <= RT_STEP_SYNC_BYTES, "StepSync size");
static_assert(__builtin_offsetof(StepSync, status) == RT_STEP_STATUS_OFF, "StepSync layout");

// The phase records live in global memory, so the pointers read from them
// carry no address space: as generic (flat) pointers every load through them
// would also count against the LDS wait counter, and each LDS barrier of a
// body would then wait for the weight loads in flight.  A local copy whose
// pointers pass through the global address space (behind an empty asm, so
// the two casts are not folded away) lets the compiler use global loads and
// stores.
template <typename T>
RT_DEV T* as_global(T* p) {
    auto g = (__attribute__((address_space(1))) T*)p;
    asm volatile("" : "+s"(g));
    return (T*)g;
}
RT_DEV GemvArgs step_gemv_args(const GemvArgs& src) {
    GemvArgs a = src;
    for (int i = 0; i < 3; ++i) {
        a.w[i] = as_global(a.w[i]);
        a.out[i] = as_global(a.out[i]);
        a.aux[i] = as_global(a.aux[i]);
    }
    a.x = as_global(a.x);
    a.gamma = as_global(a.gamma);
    a.part = as_global(a.part);
    a.counters = as_global(a.counters);
    a.xml = as_global(a.xml);
    return a;
}
RT_DEV AttnArgs step_attn_args(const AttnArgs& src) {
    AttnArgs a = src;
    a.q = as_global(a.q);
    a.kc = as_global(a.kc);
    a.vc = as_global(a.vc);
    a.out = as_global(a.out);
    a.k_new = as_global(a.k_new);
    a.v_new = as_global(a.v_new);
    a.part = as_global(a.part);
    a.ml = as_global(a.ml);
    a.counters = as_global(a.counters);
    return a;
}

constexpr uint64_t kStepSpinTicks = 5000000ull;  // 50 ms of the 100 MHz real-time clock

// End of a phase: this workgroup's stores are complete, then it counts in.
RT_DEV void step_arrive(StepSync* sy) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) arrive(&sy->ctr[blockIdx.x % 8][0]);
}

// Start of a phase (after its first weight loads): wait until `done` phases
// are complete, i.e. every XCD's counter has reached done × its workgroups
// (serial-number comparison).  Lanes 0-7 of wave 0 poll; the other waves
// wait at the workgroup barrier, which does not wait for their outstanding
// weight loads.
RT_DEV void step_wait(StepSync* sy, uint32_t done) {
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x, G = gridDim.x;
        const uint32_t need = lane < 8 ? done * ((G - lane + 7) / 8) : 0u;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (true) {
            const bool ok = lane >= 8 || (int32_t)(dev_load(&sy->ctr[lane][0]) - need) >= 0;
            if (__all(ok)) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > kStepSpinTicks) {
                if (lane == 0) dev_store(&sy->status, 1u);
                break;
            }
        }
    }
    lds_barrier();
}

struct StepHook {
    StepSync* sy;
    uint32_t done;  // phases to wait for (all earlier launches' and this one's)
    bool wait;      // false for the first phase of a launch
    RT_DEV void operator()() const {
        if (wait) step_wait(sy, done);
    }
};

extern "C" __global__ void __launch_bounds__(RT_STEP_THREADS)
k_decode_step_q8_0(const StepPhase* __restrict__ ph, uint32_t nph, StepSync* sy) {
    constexpr int PF = fmt_pf<FmtQ8_0>() ? fmt_pf<FmtQ8_0>() : GEMV_PF1;
    __shared__ uint32_t base_s;
    if (threadIdx.x == 0) base_s = dev_load(&sy->base);
    lds_barrier();
    const uint32_t base = base_s;
    for (uint32_t p = 0; p < nph; ++p) {
        const StepPhase& f = ph[p];
        const StepHook hook{sy, base + p, p > 0};
        switch (f.kind) {
        case SK_EMBED_Q8_0: {
            hook();
            const uint32_t k = f.n0;
            const uint8_t* table = as_global((const uint8_t*)f.p0);
            float* out = as_global((float*)f.p2);
            const uint8_t* row = table + (size_t)as_global((const uint32_t*)f.p1)[0] * (k / 32) * 34;
            for (uint32_t i = blockIdx.x * wg_threads() + threadIdx.x; i < k; i += gridDim.x * wg_threads()) {
                const uint8_t* blk = row + (i / 32) * 34;
                dev_store(out + i, __fmul_rn(h2f(*(const uint16_t*)blk), (float)(int8_t)blk[2 + (i & 31)]));
            }
            break;
        }
        case SK_QKV_Q8_0:
            gemv_mq_body<FmtQ8_0, EPI_QKV_BIAS | EPI_COH, CohF32, 1, PF>(step_gemv_args(f.g), hook);
            break;
        case SK_ATTN_HD64: {
            const uint32_t nsp = f.n0, ny = f.n1;
            if (blockIdx.x < nsp * ny)
                attn_split<64, true, RT_STEP_THREADS / 256, rt_step_attn_gm(64), true>(
                    step_attn_args(f.at), blockIdx.x % nsp, nsp, blockIdx.x / nsp, 0, hook);
            else
                hook();
            break;
        }
        case SK_OPROJ_Q8_0:
            gemv_mq_body<FmtQ8_0, EPI_F32_ADD | EPI_COH, AttnXC, 1, PF>(step_gemv_args(f.g), hook);
            break;
        case SK_FFN_Q8_0:
            gemv_mq_body<FmtQ8_0, EPI_FFN | EPI_COH, CohF32, 1, PF>(step_gemv_args(f.g), hook);
            break;
        case SK_DOWN_Q8_0:
            gemv_mq_body<FmtQ8_0, EPI_F32_ADD | EPI_COH, CohF32, 1, PF>(step_gemv_args(f.g), hook);
            break;
        default:
            hook();
            break;
        }
        step_arrive(sy);
    }
    // the last workgroup to leave advances the epoch for the next launch
    if (threadIdx.x == 0 && arrive(&sy->exits) == gridDim.x - 1) {
        dev_store(&sy->exits, 0u);
        dev_store(&sy->base, base + nph);
    }
}
