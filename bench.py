#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-GEMV decode path (one GPU).

Metric: quant GEMV HBM GB/s (% of peak) + decode tok/s.

For each BASELINE configuration the hot-path kernels run on synthetic,
seeded inputs already resident in HBM:
  * every weight matrix is replicated until the working set exceeds 1 GiB
    (4× the 256 MB Infinity Cache), and consecutive launches use different
    replicas, so each launch streams its weights from HBM;
  * the launches are captured once in a HIP graph and the graph is replayed;
    HIP events on the library's stream bracket the timed replays.
GB/s uses ALGORITHMIC bytes: packed weights once + activations + outputs
(+ residual / bias), each counted once per launch.

The CPU baseline is the oracle's restatement of the reference CPU path
(dequantise row → sequential f32 dot, crates/kernels/src/dispatch.rs:
1705-1709), timed on this host on a bounded sample.

Prints ONE JSON line (the last line of stdout).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

from runit_mac_amd import dispatch as d  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
WORKSET_BYTES = 1 << 30  # ≥ 4× the 256 MB MALL


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Arena:
    """One device allocation carved into 256-byte-aligned sub-buffers: model
    weights live in one large allocation, as a loaded model's would."""

    def __init__(self, ctx, nbytes):
        self.buf = ctx.new_buffer(nbytes)
        self.base, self.off, self.size = self.buf.ptr, 0, nbytes

    def take(self, nbytes) -> int:
        p = self.base + self.off
        self.off += (nbytes + 255) & ~255
        assert self.off <= self.size, "arena overflow"
        return p

    def free(self):
        self.buf.free()


def _arena_for(ctx, sizes, reps):
    return Arena(ctx, reps * sum((b + 255) & ~255 for b in sizes) + 4096)


class Workload:
    """A set of launches over rotating weight replicas."""

    def __init__(self, ctx, name, fmt, kind, n, k, m=1, seed=1):
        self.ctx, self.name, self.fmt, self.kind, self.n, self.k, self.m = ctx, name, fmt, kind, n, k, m
        nmat = 2 if kind == "ffn" else 1
        el, _ = d.BLOCK[fmt]
        wbytes = d.weight_bytes(fmt, n, k)
        self.wbytes_per_launch = nmat * wbytes
        self.reps = max(2, min(512, -(-WORKSET_BYTES // self.wbytes_per_launch)))
        self.arena = _arena_for(ctx, [wbytes] * nmat, self.reps)
        self.w = []
        for r in range(self.reps):
            mats = []
            for j in range(nmat):
                b = self.arena.take(wbytes)
                # ggml layouts (…g) are timed on the reference layout's synthetic
                # bytes: the same block sizes and byte statistics
                sfmt = fmt[:-1] if fmt.endswith("g") else fmt
                d.synth_weights(ctx, sfmt, b, n * k // el, seed * 1000 + r * 2 + j)
                mats.append(b)
            self.w.append(mats)
        self.x = ctx.new_buffer(4 * m * k)
        d.synth_normal_f32(ctx, self.x, m * k, seed + 7)
        nout = n if kind != "qkv" else n
        self.y = ctx.new_buffer(4 * m * nout)
        self.res = ctx.new_buffer(4 * n)
        d.synth_normal_f32(ctx, self.res, n, seed + 8)
        if kind == "qkv":
            self.q_dim, self.kv_dim = self.split
        ctx.flush()

    split = None

    def algorithmic_bytes(self) -> int:
        n, k, m = self.n, self.k, self.m
        b = self.wbytes_per_launch + 4 * m * k  # weights + activations
        if self.kind == "ffn":
            b += 4 * n
        elif self.kind == "add":
            b += 4 * n + 4 * n  # output + residual read
        elif self.kind == "qkv":
            b += 4 * n + 2 * n  # outputs + f16 bias
        else:
            b += 4 * m * n
        return b

    def flops(self) -> int:
        nmat = 2 if self.kind == "ffn" else 1
        return 2 * self.m * self.n * self.k * nmat

    def launch(self, r: int):
        ctx, w, n, k = self.ctx, self.w[r % self.reps], self.n, self.k
        f = self.fmt
        if self.kind == "gemv":
            getattr(d, f"gemv_{f}_f32in_f32out")(ctx, w[0], self.x, self.y, n, k)
        elif self.kind == "add":
            getattr(d, f"gemv_{f}_add_f32_f32in")(ctx, w[0], self.x, self.y, self.res, n, k)
        elif self.kind == "ffn":
            getattr(d, f"fused_ffn_{f}_f32")(ctx, w[0], w[1], self.x, self.y, n, k)
        elif self.kind == "gemm":
            getattr(d, f"gemm_{f}_f32")(ctx, w[0], self.x, self.y, self.m, n, k)
        else:
            raise ValueError(self.kind)

    def free(self):
        self.arena.free()
        self.w = []


class QKVWorkload(Workload):
    """Fused Q/K/V (+f16 bias) launches; fmt_v: V in another format (Q4_K_M)."""

    def __init__(self, ctx, name, fmt, q_dim, kv_dim, k, seed=1, fmt_v=None):
        self.q_dim, self.kv_dim = q_dim, kv_dim
        self.ctx, self.name, self.fmt, self.kind, self.k, self.m = ctx, name, fmt, "qkv", k, 1
        self.fmt_v = fmt_v or fmt
        self.n = q_dim + 2 * kv_dim
        dims = (q_dim, kv_dim, kv_dim)
        fmts = (fmt, fmt, self.fmt_v)
        sizes = [d.weight_bytes(f, n, k) for f, n in zip(fmts, dims)]
        self.wbytes_per_launch = sum(sizes)
        self.reps = max(2, min(512, -(-WORKSET_BYTES // self.wbytes_per_launch)))
        self.arena = _arena_for(ctx, sizes, self.reps)
        self.w = []
        for r in range(self.reps):
            mats = []
            for j, (f, n) in enumerate(zip(fmts, dims)):
                b = self.arena.take(sizes[j])
                d.synth_weights(ctx, f, b, n * k // d.BLOCK[f][0], seed * 1000 + r * 3 + j)
                mats.append(b)
            self.w.append(mats)
        self.x = ctx.new_buffer(4 * k)
        d.synth_normal_f32(ctx, self.x, k, seed + 7)
        self.outs = [ctx.new_buffer(4 * n) for n in dims]
        self.bias = [ctx.new_buffer(2 * n) for n in dims]
        for i, (b, n) in enumerate(zip(self.bias, dims)):
            d.synth_normal_f16(ctx, b, n, seed + 20 + i, 0.0, 0.02)
        ctx.flush()
        fn = (f"fused_qkv_bias_{fmt}_f32" if self.fmt_v == fmt
              else f"fused_qkv_bias_{fmt}_{self.fmt_v}_f32")
        self.fn = getattr(d, fn)

    def launch(self, r: int):
        w = self.w[r % self.reps]
        self.fn(self.ctx, w[0], w[1], w[2], self.x, *self.outs, *self.bias,
                self.q_dim, self.kv_dim, self.k)


def time_workload(ctx, wl: Workload, steps: int, warmup: int) -> dict:
    """Graph of `reps` launches (one per replica), replayed; returns µs/launch."""
    launches = wl.reps
    wl.launch(0)  # eager first call: sizes the context workspace before capture
    ctx.flush()
    ctx.capture_begin()
    for r in range(launches):
        wl.launch(r)
    g = ctx.capture_end()
    for _ in range(max(1, warmup)):
        g.launch()
    ctx.flush()
    e0, e1 = ctx.event(), ctx.event()
    reps = max(1, steps)
    e0.record()
    for _ in range(reps):
        g.launch()
    e1.record()
    ms = e0.elapsed_ms(e1)
    us = ms * 1e3 / (reps * launches)
    b = wl.algorithmic_bytes()
    gbs = b / (us * 1e-6) / 1e9
    return {"name": wl.name, "fmt": wl.fmt, "kind": wl.kind, "n": wl.n, "k": wl.k, "m": wl.m,
            "bytes": b, "us": round(us, 3), "gbs": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "launches": reps * launches,
            "tflops": round(wl.flops() / (us * 1e-6) / 1e12, 3)}


def cpu_baseline(model, token: int, pos: int, gpu_token: int, seconds: float = 16.0) -> dict:
    """The reference CPU path on the config-2 step itself: the oracle's f32
    restatement of the reference's CPU helpers composed into one greedy decode
    step (dequantise row → sequential f32 dot of cpu_gemv, dispatch.rs:
    1705-1709; cpu_rms_norm, RoPE, attention over kv_len 512, SiLU, LM head,
    argmax) on a host model rebuilt from the GPU model's seeds, byte-identical
    to the weights and KV cache the GPU step reads.  Timed as whole steps:
    single-thread (the reference's CPU code is single-threaded) for about
    3/4 of `seconds`, then with GEMV rows split over every host core."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import oracle_lib as ora  # noqa: E402  (test infrastructure: baseline only)
    t0 = time.perf_counter()
    host = ora.HostStepModel.from_recipe(model)
    t_build = time.perf_counter() - t0
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    res = {}
    for threads, budget in ((1, 0.75 * seconds), (cores, 0.25 * seconds)):
        n, t0 = 0, time.perf_counter()
        while True:
            tok, _ = host.step(token, pos, threads)
            n += 1
            if time.perf_counter() - t0 >= budget:
                break
        res[threads] = ((time.perf_counter() - t0) / n, n, tok)
    (t1, n1, tok1), (tn, nn, _) = res[1], res[cores]
    return {"value": round(1.0 / t1, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "ms_per_token": round(t1 * 1e3, 1), "token": tok1, "gpu_token": gpu_token,
            "token_match": tok1 == gpu_token,
            "all_cores": {"value": round(1.0 / tn, 3), "unit": "tok/s", "cores": cores,
                          "ms_per_token": round(tn * 1e3, 1), "steps": nn},
            "sample": (f"{n1} whole config-2 decode steps single-thread (token {token} at pos "
                       f"{pos}, kv_len {pos + 1}, 24 layers + LM head + argmax) on the GPU "
                       f"model's seeded weights and KV cache rebuilt on the host "
                       f"({t_build:.1f} s to rebuild), then {nn} steps with GEMV rows over "
                       f"{cores} threads")}


def _bench_prefill(ctx, m, cfg, P: int, steps: int) -> float:
    """Milliseconds of one captured prefill of a P-token prompt."""
    m._verify_arena(P, logits=False)
    toks = np.arange(P, dtype=np.uint32) % cfg.vocab
    ctx._check(d.load_library().rt_upload(ctx.handle, m._vbufs["tok"], toks.ctypes.data,
                                          toks.nbytes))
    m.verify_pass(P, 0, last_only=True)
    ctx.flush()
    ctx.capture_begin()
    m.verify_pass(P, 0, last_only=True)
    g = ctx.capture_end()
    g.launch()
    ctx.flush()
    e0, e1 = ctx.event(), ctx.event()
    reps = max(3, steps // 10)
    e0.record()
    for _ in range(reps):
        g.launch()
    e1.record()
    del g
    return e0.elapsed_ms(e1) / reps


def bench_verify_eager(ctx, steps: int, q4k_7b: bool = False) -> dict:
    """The batched verify passes (M = 4, 8, 16 on the multi-row GEMVs; 16, 32
    on the GEMMs) and a 512-token prefill of the 0.5B model — or, with
    q4k_7b, of the 7B Q4_K_M-mix model on the GEMMs at M = 8, 16, 32 —
    launched eagerly (no graph), for kernel traces of their kernels:
    rocprofv3 --kernel-trace ends in a host-side fault when it traces the
    replay of their graphs."""
    from runit_mac_amd.decode import Q4K_M, DecodeConfig, DecodeModel
    if q4k_7b:
        cfg = DecodeConfig(layers=28, hidden=3584, heads=28, kv_heads=4, head_dim=128, ff=18944,
                           vocab=152064, max_seq=1024)
        m = DecodeModel(ctx, cfg, seed=9, quant=Q4K_M)
        forms = ((8, "gemm"), (16, "gemm"), (32, "gemm"))
    else:
        cfg = DecodeConfig()
        m = DecodeModel(ctx, cfg, seed=7)
        forms = ((4, "rows"), (8, "rows"), (16, "rows"), (16, "gemm"), (32, "gemm"))
    pos, out = 511, {}
    for M, form in forms:
        m.verify_forward([1] * M, pos, form)  # uploads the ids, sizes the buffers
        ctx.flush()
        e0, e1 = ctx.event(), ctx.event()
        e0.record()
        for _ in range(steps):
            m.verify_pass(M, pos, form)
        e1.record()
        out[f"{form}_m{M}"] = e0.elapsed_ms(e1) * 1e3 / steps
        log(f"verify pass ({form}, eager launches), {M} tokens: {out[f'{form}_m{M}']:.1f} us")
    P = 512
    m._verify_arena(P, logits=False)
    toks = np.arange(P, dtype=np.uint32) % cfg.vocab
    ctx._check(d.load_library().rt_upload(ctx.handle, m._vbufs["tok"], toks.ctypes.data,
                                          toks.nbytes))
    m.verify_pass(P, 0, last_only=True)
    ctx.flush()
    e0, e1 = ctx.event(), ctx.event()
    reps = max(3, steps // 10)
    e0.record()
    for _ in range(reps):
        m.verify_pass(P, 0, last_only=True)
    e1.record()
    out["prefill_512"] = e0.elapsed_ms(e1) * 1e3 / reps
    log(f"prefill of {P} tokens (eager launches): {out['prefill_512'] / 1e3:.2f} ms")
    m.free()
    return out


def bench_decode(ctx, steps: int, warmup: int, verify_forms: bool = True) -> dict:
    """Config 2: one greedy decode step of the 0.5B Q8_0 shape at kv_len 512,
    captured as one HIP graph and replayed (one replay = one token)."""
    from runit_mac_amd.decode import DecodeConfig, DecodeModel
    cfg = DecodeConfig()
    m = DecodeModel(ctx, cfg, seed=7)
    pos = 511  # decoding position 511 → kv_len 512
    # one eager step from token 1: the greedy token the CPU baseline must match
    m.set_token(1)
    m.step_fused(pos)
    ctx.flush()
    gpu_token = m.get_token()
    m.set_token(1)
    res = {}
    # the persistent step: one launch for the embedding and every layer, then
    # the LM head and the argmax
    step = m.plan_persistent(pos)
    step.run()
    step.check()
    ctx.capture_begin()
    step.run()
    g = ctx.capture_end()
    for _ in range(max(1, warmup)):
        g.launch()
    ctx.flush()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    for _ in range(steps):
        g.launch()
    e1.record()
    res["persistent"] = e0.elapsed_ms(e1) / steps
    step.check()
    del g
    for name, fused in (("fused", True), ("reference_sequence", False)):
        g = m.capture(pos, fused=fused)
        for _ in range(max(1, warmup)):
            g.launch()
        ctx.flush()
        e0, e1 = ctx.event(), ctx.event()
        e0.record()
        for _ in range(steps):
            g.launch()
        e1.record()
        res[name] = e0.elapsed_ms(e1) / steps
        del g
    # the batched verify pass (verify_draft: M tokens through every layer on
    # the batched GEMMs, causal attention over the cache + the M new rows),
    # captured as one graph; the cache is restored between replays
    verify = {}
    for M, form in ((4, "rows"), (8, "rows"), (16, "rows"), (8, "gemm"), (16, "gemm"), (32, "gemm")) if verify_forms else ():
        m.verify_forward([1] * M, pos, form)  # uploads the ids, sizes the buffers
        ctx.flush()
        ctx.capture_begin()
        m.verify_pass(M, pos, form)
        g = ctx.capture_end()
        for _ in range(max(1, warmup)):
            g.launch()
        ctx.flush()
        e0, e1 = ctx.event(), ctx.event()
        e0.record()
        for _ in range(steps):
            g.launch()
        e1.record()
        verify[(M, form)] = e0.elapsed_ms(e1) / steps
        del g
    # prefill of a 512-token prompt (prefill.rs): one batched pass from
    # position 0 on the batched GEMMs, the LM head on the last row
    P = 512
    prefill_ms = float("nan")
    if verify_forms:
        prefill_ms = _bench_prefill(ctx, m, cfg, P, steps)
    # the step's single-kernel launches, each timed live over the model's own
    # 24 layers (a graph of 24 launches on the library stream, HIP events
    # around its replays): norm-fused Q/K/V + bias, norm-fused gate+up+SiLU,
    # down + residual.  The roofline reports the one with the most time per
    # token.
    h, ff, kvd = cfg.hidden, cfg.ff, cfg.kv_dim

    def live_us(launch) -> float:
        launch(m.layers[0])  # eager: names the kernel the library chose
        ctx.flush()
        names.append(d.last_launch_name(ctx))
        ctx.capture_begin()
        for L in m.layers:
            launch(L)
        g = ctx.capture_end()
        for _ in range(max(1, warmup)):
            g.launch()
        ctx.flush()
        e0, e1 = ctx.event(), ctx.event()
        reps = max(20, steps)
        e0.record()
        for _ in range(reps):
            g.launch()
        e1.record()
        us = e0.elapsed_ms(e1) * 1e3 / (reps * cfg.layers)
        del g
        return us

    wq = d.weight_bytes("q8_0", cfg.q_dim + 2 * kvd, h)
    names = []
    kernels = {
        "ffn": {
            "role": "rms_norm + gate/up 2x4864x896 + SiLU",
            "us": live_us(lambda L: d.rms_norm_fused_ffn_q8_0_f32(
                ctx, L["wg"], L["wu"], m.x, L["ffn_norm"], cfg.eps, m.act, ff, h)),
            # weights + x + gamma + act
            "bytes": 2 * d.weight_bytes("q8_0", ff, h) + 4 * h * 2 + 4 * ff,
            "pmc": "ffn_q8_0_0p5b_pmc_traffic.md"},
        "down": {
            "role": "down 896x4864 + residual",
            "us": live_us(lambda L: d.gemv_q8_0_add_f32_f32in(ctx, L["wd"], m.act, m.x, m.x, h, ff)),
            # weights + act + residual read + output write
            "bytes": d.weight_bytes("q8_0", h, ff) + 4 * ff + 4 * h + 4 * h,
            "pmc": "down_q8_0_0p5b_pmc_traffic.md"},
        "qkv": {
            "role": "rms_norm + Q/K/V 1152x896 + bias",
            "us": live_us(lambda L: d.rms_norm_fused_qkv_bias_q8_0_f32(
                ctx, L["wq"], L["wk"], L["wv"], m.x, L["attn_norm"], cfg.eps, m.q, m.k, m.v,
                L["bq"], L["bk"], L["bv"], cfg.q_dim, kvd, h)),
            # weights + x + gamma + f16 biases + outputs
            "bytes": wq + 4 * h * 2 + 2 * (cfg.q_dim + 2 * kvd) + 4 * (cfg.q_dim + 2 * kvd),
            "pmc": "qkv_q8_0_0p5b_pmc_traffic.md"},
    }
    # keyed by the kernel the library launched for each
    kernels = {nm: dict(kk, launch=key) for nm, (key, kk) in zip(names, kernels.items())}
    for kk in kernels.values():
        kk["us_per_token"] = kk["us"] * cfg.layers
    return {"cfg": cfg, "model": m, "pos": pos, "gpu_token": gpu_token, "step": step,
            "ms_persistent": res["persistent"], "ms_fused": res["fused"], "ms_reference": res["reference_sequence"],
            "step_bytes": cfg.step_bytes(pos + 1), "kernels": kernels,
            "launches_fused": m.launches_fused(),
            "launches_reference": 1 + 10 * cfg.layers + 3, "verify_ms": verify,
            "prefill_ms": prefill_ms, "prefill_tokens": P}


def bench_q4km_decode(ctx, steps: int, warmup: int) -> dict:
    """Config 4 as a whole greedy decode step: Qwen2.5-7B shapes (28 layers,
    hidden 3584, 28/4 heads × 128, ff 18944, vocab 152064) with the Q4_K_M
    mix (Q/K/O/gate/up Q4_K; V, down and LM head Q6_K; Q8_0 embedding rows),
    RMSNorm, RoPE, KV-cache write and attention at kv_len 512, one graph
    replay per token; random-init weights of that shape."""
    from runit_mac_amd.decode import Q4K_M, DecodeConfig, DecodeModel
    cfg = DecodeConfig(layers=28, hidden=3584, heads=28, kv_heads=4, head_dim=128, ff=18944,
                       vocab=152064, max_seq=1024)
    m = DecodeModel(ctx, cfg, seed=9, quant=Q4K_M)
    pos = 511
    m.set_token(1)
    g = m.capture(pos, fused=True)
    for _ in range(max(1, warmup)):
        g.launch()
    ctx.flush()
    e0, e1 = ctx.event(), ctx.event()
    reps = max(5, steps // 2)
    e0.record()
    for _ in range(reps):
        g.launch()
    e1.record()
    ms = e0.elapsed_ms(e1) / reps
    del g
    launches = m.launches_fused()
    # the batched verify pass at these shapes (M draft tokens through all 28
    # layers on the Q4_K / Q6_K GEMMs, the form verify_draft takes at this
    # hidden size), one graph per M, replayed over the same cache positions
    verify = {}
    for M, form in ((4, "gemm"), (8, "gemm"), (16, "gemm"), (32, "gemm")):
        m.verify_forward([1] * M, pos, form)
        ctx.flush()
        ctx.capture_begin()
        m.verify_pass(M, pos, form)
        gv = ctx.capture_end()
        gv.launch()
        ctx.flush()
        e0.record()
        for _ in range(reps):
            gv.launch()
        e1.record()
        verify[(M, form)] = e0.elapsed_ms(e1) / reps
        del gv
    prefill_ms = _bench_prefill(ctx, m, cfg, 512, steps)
    m.free()
    return {"ms": ms, "step_bytes": cfg.step_bytes(pos + 1, Q4K_M), "launches": launches,
            "verify_ms": verify, "prefill_ms": prefill_ms, "prefill_tokens": 512}


def bench_q4km_step(ctx, steps: int, warmup: int) -> dict:
    """Config 4: every GEMV of one Qwen2.5-7B-shape token in a Q4_K_M-style
    mix — 28 layers of Q, K, O, gate+up (Q4_K) and V, down (Q6_K), the
    output and down projections adding into the residual — plus the
    152064×3584 Q6_K LM head, captured as one graph and replayed; random-init
    weights of that shape, one activation vector.  Q, K and V (+ their f16
    biases, as Qwen2.5 has them) run as one mixed-format launch (113 launches
    per token); the same step with three separate bias-free GEMVs instead
    (169 launches) is timed beside it."""
    h, ff, kv, vocab, layers = 3584, 18944, 512, 152064, 28
    sizes = {"q": d.weight_bytes("q4k", h, h), "k": d.weight_bytes("q4k", kv, h),
             "v": d.weight_bytes("q6k", kv, h), "o": d.weight_bytes("q4k", h, h),
             "g": d.weight_bytes("q4k", ff, h), "u": d.weight_bytes("q4k", ff, h),
             "d": d.weight_bytes("q6k", h, ff)}
    fmts = {"q": "q4k", "k": "q4k", "v": "q6k", "o": "q4k", "g": "q4k", "u": "q4k", "d": "q6k"}
    shapes = {"q": (h, h), "k": (kv, h), "v": (kv, h), "o": (h, h), "g": (ff, h), "u": (ff, h),
              "d": (h, ff)}
    lm_bytes = d.weight_bytes("q6k", vocab, h)
    total_w = layers * sum(sizes.values()) + lm_bytes
    arena = Arena(ctx, total_w + 4096 * (layers * len(sizes) + 1))
    L = []
    for i in range(layers):
        mats = {}
        for key, nb in sizes.items():
            b = arena.take(nb)
            n, k = shapes[key]
            el, _ = d.BLOCK[fmts[key]]
            d.synth_weights(ctx, fmts[key], b, n * k // el, 4000 + 16 * i + len(mats))
            mats[key] = b
        L.append(mats)
    bias_bytes = 2 * (h + 2 * kv)
    biases = []
    for i in range(layers):
        bq, bk, bv = ctx.new_buffer(2 * h), ctx.new_buffer(2 * kv), ctx.new_buffer(2 * kv)
        for j, (bb, n) in enumerate(((bq, h), (bk, kv), (bv, kv))):
            d.synth_normal_f16(ctx, bb, n, 5000 + 3 * i + j, 0.0, 0.02)
        biases.append((bq, bk, bv))
    lm = arena.take(lm_bytes)
    d.synth_weights(ctx, "q6k", lm, vocab * h // 256, 4999)
    x = ctx.new_buffer(4 * ff)
    d.synth_normal_f32(ctx, x, ff, 77)
    q, kb, vb = ctx.new_buffer(4 * h), ctx.new_buffer(4 * kv), ctx.new_buffer(4 * kv)
    hres, act, logits = ctx.new_buffer(4 * h), ctx.new_buffer(4 * ff), ctx.new_buffer(4 * vocab)
    d.synth_normal_f32(ctx, hres, h, 78)
    ctx.flush()

    def sequence(fused_qkv: bool):
        for m, (bq, bk, bv) in zip(L, biases):
            if fused_qkv:
                d.fused_qkv_bias_q4k_q6k_f32(ctx, m["q"], m["k"], m["v"], x, q, kb, vb,
                                             bq, bk, bv, h, kv, h)
            else:
                d.gemv_q4k_f32in_f32out(ctx, m["q"], x, q, h, h)
                d.gemv_q4k_f32in_f32out(ctx, m["k"], x, kb, kv, h)
                d.gemv_q6k_f32in_f32out(ctx, m["v"], x, vb, kv, h)
            d.gemv_q4k_add_f32_f32in(ctx, m["o"], x, hres, hres, h, h)
            d.fused_ffn_q4k_f32(ctx, m["g"], m["u"], x, act, ff, h)
            d.gemv_q6k_add_f32_f32in(ctx, m["d"], x, hres, hres, h, ff)
        d.gemv_q6k_f32in_f32out(ctx, lm, x, logits, vocab, h)

    def timed(fused_qkv: bool) -> float:
        sequence(fused_qkv)  # eager first pass: sizes the context workspace before capture
        ctx.flush()
        ctx.capture_begin()
        sequence(fused_qkv)
        g = ctx.capture_end()
        for _ in range(max(1, warmup)):
            g.launch()
        ctx.flush()
        e0, e1 = ctx.event(), ctx.event()
        reps = max(5, steps // 5)
        e0.record()
        for _ in range(reps):
            g.launch()
        e1.record()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        del g
        return us

    us = timed(True)
    us_sep = timed(False)
    # algorithmic bytes: every weight once, plus the activation reads, the
    # biases and output writes (residual read and write for O and down)
    act_bytes = layers * (4 * h * 5 + 4 * ff + 4 * (h + kv + kv + 2 * h + ff + 2 * h)
                          + bias_bytes) + 4 * h + 4 * vocab
    step_bytes = total_w + act_bytes
    for b in (x, q, kb, vb, hres, act, logits, *[bb for t in biases for bb in t]):
        b.free()
    arena.free()
    return {"us": us, "us_separate_qkv": us_sep, "bytes": step_bytes, "weight_bytes": total_w,
            "launches": 4 * layers + 1, "launches_separate_qkv": 6 * layers + 1}


def measured_traffic(summary: str):
    """HBM bytes per launch of a kernel, from its committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE, each scaled by a copy kernel's
    reading); None when the summary is absent."""
    import re
    path = os.path.join(REPO, "profiles", summary)
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", open(path).read())
    return int(m.group(1)) if m else None


def profile_pass(ctx, launches: int = 24) -> None:
    """Eager (not graph-captured) launches for hardware-counter runs
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE): the dominant kernel of the
    decode step — the norm-fused gate+up+SiLU GEMV at the 0.5B shape — over
    `launches` distinct weight replicas, the 7B Q4_K gate+up+SiLU over 8,
    the 7B Q6_K down projection over 8, then a plain copy kernel of known
    size whose counters calibrate the byte counts."""
    from runit_mac_amd.decode import DecodeConfig
    cfg = DecodeConfig()
    h, ff = cfg.hidden, cfg.ff
    wb = d.weight_bytes("q8_0", ff, h)
    arena = _arena_for(ctx, [wb, wb], launches)
    mats = []
    for r in range(launches):
        g, u = arena.take(wb), arena.take(wb)
        d.synth_weights(ctx, "q8_0", g, ff * h // 32, 100 + 2 * r)
        d.synth_weights(ctx, "q8_0", u, ff * h // 32, 101 + 2 * r)
        mats.append((g, u))
    x = ctx.new_buffer(4 * h)
    gamma = ctx.new_buffer(4 * h)
    act = ctx.new_buffer(4 * ff)
    d.synth_normal_f32(ctx, x, h, 5)
    d.synth_normal_f32(ctx, gamma, h, 6, 1.0, 0.02)
    ctx.flush()
    for g, u in mats:
        d.rms_norm_fused_ffn_q8_0_f32(ctx, g, u, x, gamma, cfg.eps, act, ff, h)
    ctx.flush()
    # the 0.5B down projection + residual (896x4864, workgroup-local K split)
    # over the same number of replicas
    wd5 = d.weight_bytes("q8_0", h, ff)
    arena_d5 = _arena_for(ctx, [wd5], launches)
    downs5 = []
    for r in range(launches):
        w = arena_d5.take(wd5)
        d.synth_weights(ctx, "q8_0", w, h * ff // 32, 200 + r)
        downs5.append(w)
    y5 = ctx.new_buffer(4 * h)
    d.synth_normal_f32(ctx, y5, h, 9)
    ctx.flush()
    for w in downs5:
        d.gemv_q8_0_add_f32_f32in(ctx, w, act, y5, y5, h, ff)
    ctx.flush()
    # the 0.5B norm-fused Q/K/V + biases (1152x896) over the same number of
    # replicas
    qd, kvd = cfg.q_dim, cfg.kv_dim
    wqb, wkb = d.weight_bytes("q8_0", qd, h), d.weight_bytes("q8_0", kvd, h)
    arena_q = _arena_for(ctx, [wqb, wkb, wkb], launches)
    qkvs = []
    for r in range(launches):
        wq_, wk_, wv_ = arena_q.take(wqb), arena_q.take(wkb), arena_q.take(wkb)
        d.synth_weights(ctx, "q8_0", wq_, qd * h // 32, 500 + 3 * r)
        d.synth_weights(ctx, "q8_0", wk_, kvd * h // 32, 501 + 3 * r)
        d.synth_weights(ctx, "q8_0", wv_, kvd * h // 32, 502 + 3 * r)
        qkvs.append((wq_, wk_, wv_))
    bq, bk, bv = (ctx.new_buffer(2 * n + 4) for n in (qd, kvd, kvd))
    for b_, n in ((bq, qd), (bk, kvd), (bv, kvd)):
        d.synth_normal_f16(ctx, b_, n, 11 + n, 0.0, 0.02)
    oq, ok_, ov = ctx.new_buffer(4 * qd), ctx.new_buffer(4 * kvd), ctx.new_buffer(4 * kvd)
    ctx.flush()
    for wq_, wk_, wv_ in qkvs:
        d.rms_norm_fused_qkv_bias_q8_0_f32(ctx, wq_, wk_, wv_, x, gamma, cfg.eps, oq, ok_, ov,
                                           bq, bk, bv, qd, kvd, h)
    ctx.flush()
    # the 7B Q4_K gate+up+SiLU (LDS-streamed body) over 8 replicas of 76 MB
    ff7, h7 = 18944, 3584
    wb7 = d.weight_bytes("q4k", ff7, h7)
    arena7 = _arena_for(ctx, [wb7, wb7], 8)
    mats7 = []
    for r in range(8):
        g, u = arena7.take(wb7), arena7.take(wb7)
        d.synth_weights(ctx, "q4k", g, ff7 * h7 // 256, 300 + 2 * r)
        d.synth_weights(ctx, "q4k", u, ff7 * h7 // 256, 301 + 2 * r)
        mats7.append((g, u))
    x7, act7 = ctx.new_buffer(4 * h7), ctx.new_buffer(4 * ff7)
    d.synth_normal_f32(ctx, x7, h7, 7)
    ctx.flush()
    for g, u in mats7:
        d.fused_ffn_q4k_f32(ctx, g, u, x7, act7, ff7, h7)
    ctx.flush()
    # the 7B Q6_K down projection + residual (workgroup-local K split) over 8
    # replicas of 56 MB
    wd7 = d.weight_bytes("q6k", h7, ff7)
    arena_d = _arena_for(ctx, [wd7], 8)
    downs = []
    for r in range(8):
        w = arena_d.take(wd7)
        d.synth_weights(ctx, "q6k", w, h7 * ff7 // 256, 400 + r)
        downs.append(w)
    y7 = ctx.new_buffer(4 * h7)
    d.synth_normal_f32(ctx, y7, h7, 8)
    ctx.flush()
    for w in downs:
        d.gemv_q6k_add_f32_f32in(ctx, w, act7, y7, y7, h7, ff7)
    ctx.flush()
    copy_bytes = 256 << 20
    src, dst = ctx.new_buffer(copy_bytes), ctx.new_buffer(copy_bytes)
    for _ in range(3):
        d.stream_copy(ctx, dst, src, copy_bytes)
    ctx.flush()
    log(f"profile pass: {launches} x k_ffn_q8_0 ({2 * wb} weight bytes each), "
        f"{launches} x k_gemv_q8_0_f32_f32add ({wd5} weight bytes each), "
        f"{launches} x k_qkv_bias_q8_0 ({wqb + 2 * wkb} weight bytes each), "
        f"8 x k_ffn_q4k ({2 * wb7} weight bytes each), "
        f"3 x k_stream_copy ({copy_bytes} bytes each)")
    for b in (src, dst, x, gamma, act, x7, act7, y5, bq, bk, bv, oq, ok_, ov):
        b.free()
    arena_q.free()
    arena_d5.free()
    arena.free()
    arena7.free()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--suite", default="all",
                    choices=["all", "gemv", "quick", "decode", "step", "q4decode", "verify", "verify7b"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-verify", action="store_true",
                    help="skip the verify / prefill graphs (rocprofv3 --kernel-trace runs)")
    ap.add_argument("--only", default=None, help="run only GEMV workloads whose label contains this")
    ap.add_argument("--profile-pass", action="store_true",
                    help="eager launches of the dominant kernel + a calibration copy, for "
                         "rocprofv3 --pmc runs; prints no JSON")
    args = ap.parse_args()
    if args.gpus != 1:
        sys.exit("bench.py measures one GPU only: this build has no multi-GPU path "
                 "(how the path would shard is a design note, not code); run with --gpus 1")

    ctx = d.HipContext()
    if args.profile_pass:
        profile_pass(ctx)
        return
    if args.suite in ("verify", "verify7b"):
        # eager verify / prefill passes for kernel traces; prints no JSON
        bench_verify_eager(ctx, args.steps, q4k_7b=args.suite == "verify7b")
        ctx.close()
        return
    line = {
        "metric": "quant GEMV HBM GB/s (% of peak) + decode tok/s, 0.5B Q8_0 & 7B Q4_K",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "data": "synthetic (seeded N(0,0.02) weights quantised per block, N(0,1) activations "
                "and KV cache)",
    }
    dec = None
    if args.suite in ("all", "decode") and not args.only:
        dec = bench_decode(ctx, args.steps, args.warmup, verify_forms=not args.no_verify)
        cfg = dec["cfg"]
        ms = dec["ms_fused"]
        tok_s = 1e3 / ms
        # the roofline kernel: the step's single-kernel launch with the most
        # time per token (all three are 24 launches per token)
        kname = max(dec["kernels"], key=lambda k: dec["kernels"][k]["us_per_token"])
        kern = dec["kernels"][kname]
        kern_gbs = kern["bytes"] / (kern["us"] * 1e-6) / 1e9
        log(f"decode step (fused graph, {dec['launches_fused']} launches): {ms * 1e3:.1f} us "
            f"= {tok_s:.1f} tok/s; reference sequence ({dec['launches_reference']} launches): "
            f"{dec['ms_reference'] * 1e3:.1f} us; step bytes {dec['step_bytes'] / 1e6:.1f} MB "
            f"→ {dec['step_bytes'] / (ms * 1e-3) / 1e9:.0f} GB/s effective")
        log(f"persistent step (1 launch for embedding + 24 layers, then LM head + argmax): "
            f"{dec['ms_persistent'] * 1e3:.1f} us = {1e3 / dec['ms_persistent']:.1f} tok/s")
        for (M, form), vms in dec["verify_ms"].items():
            log(f"verify pass ({form}), {M} tokens at kv 512..{512 + M - 1}: {vms * 1e3:.1f} us "
                f"({vms * 1e3 / M:.1f} us per token; {M} fused decode steps: {M * ms * 1e3:.1f} us)")
        if dec["verify_ms"]:
            log(f"prefill of {dec['prefill_tokens']} tokens: {dec['prefill_ms']:.2f} ms = "
                f"{dec['prefill_tokens'] / dec['prefill_ms'] * 1e3:.0f} tok/s")
        for kn, kk in dec["kernels"].items():
            log(f"live kernel {kn} ({kk['role']}): {kk['us']:.2f} us x {cfg.layers} per token, "
                f"{kk['bytes'] / (kk['us'] * 1e-6) / 1e9:.0f} GB/s"
                + ("  <- roofline kernel" if kn == kname else ""))
        line.update({
            "value": round(tok_s, 2), "unit": "tok/s", "ms_per_step": round(ms, 5),
            "dtype": "q8_0 x f32 (int8 matrix-core dots, f32 scales/accumulate)",
            "config": {"workload": "config 2: Qwen2.5-0.5B-shape greedy decode step, Q8_0, "
                                   "batch 1, kv_len 512 (24 layers, hidden 896, 14/2 heads x 64, "
                                   "ff 4864, vocab 151936), one HIP-graph replay per token",
                       "global_batch": 1, "kv_len": 512},
            "roofline": {"bound": "hbm", "kernel": f"{kname} ({kern['role']})",
                         "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
                         "traffic": measured_traffic(kern["pmc"]) if kern["pmc"] else None,
                         "bytes_per_launch": kern["bytes"],
                         "avg_launch_us": round(kern["us"], 3),
                         "us_per_token": round(kern["us_per_token"], 1),
                         "others": {kn: {"us": round(kk["us"], 3), "bytes_per_launch": kk["bytes"],
                                         "frac": round(kk["bytes"] / (kk["us"] * 1e-6) / 1e9
                                                       / HBM_PEAK_GBS, 4),
                                         "traffic": (measured_traffic(kk["pmc"]) if kk["pmc"]
                                                     else None)}
                                    for kn, kk in dec["kernels"].items() if kn != kname}},
            "decode": {"tok_s": round(tok_s, 2), "us_per_token": round(ms * 1e3, 1),
                       "reference_sequence_us_per_token": round(dec["ms_reference"] * 1e3, 1),
                       "launches_per_token": dec["launches_fused"],
                       "step_bytes": dec["step_bytes"],
                       "effective_gbs": round(dec["step_bytes"] / (ms * 1e-3) / 1e9, 1),
                       "roofline_tok_s_at_peak": round(HBM_PEAK_GBS * 1e9 / dec["step_bytes"], 0)},
            "prefill": ({"tokens": dec["prefill_tokens"], "ms": round(dec["prefill_ms"], 3),
                         "tok_s": round(dec["prefill_tokens"] / dec["prefill_ms"] * 1e3, 1)}
                        if dec["verify_ms"] else None),
            "verify": {f"{form}_m{M}": {"us": round(v * 1e3, 1), "us_per_token": round(v * 1e3 / M, 1)}
                       for (M, form), v in dec["verify_ms"].items()},
        })

    if args.suite in ("all", "gemv", "step", "q4decode") and not args.only:
        q4d = bench_q4km_decode(ctx, args.steps, args.warmup)
        dgbs = q4d["step_bytes"] / (q4d["ms"] * 1e-3) / 1e9
        log(f"config 4 as a decode step (7B Q4_K_M mix, kv_len 512, {q4d['launches']} launches): "
            f"{q4d['ms'] * 1e3:.1f} us = {1e3 / q4d['ms']:.1f} tok/s; step bytes "
            f"{q4d['step_bytes'] / 1e9:.3f} GB → {dgbs:.0f} GB/s ({100 * dgbs / HBM_PEAK_GBS:.1f}% HBM)")
        line["q4k_m_7b_decode"] = {
            "tok_s": round(1e3 / q4d["ms"], 2), "us_per_token": round(q4d["ms"] * 1e3, 1),
            "step_bytes": q4d["step_bytes"], "gbs": round(dgbs, 1),
            "frac": round(dgbs / HBM_PEAK_GBS, 4), "launches_per_token": q4d["launches"],
            "kv_len": 512,
            "verify": {f"{form}_m{M}": {"us": round(v * 1e3, 1), "us_per_token": round(v * 1e3 / M, 1)}
                       for (M, form), v in q4d["verify_ms"].items()}}
        line["q4k_m_7b_decode"]["prefill"] = {
            "tokens": q4d["prefill_tokens"], "ms": round(q4d["prefill_ms"], 3),
            "tok_s": round(q4d["prefill_tokens"] / (q4d["prefill_ms"] * 1e-3), 1)}
        for (M, form), v in q4d["verify_ms"].items():
            log(f"config 4 verify pass, {M} tokens ({form}): {v * 1e3:.1f} us = "
                f"{v * 1e3 / M:.1f} us per token")
        log(f"config 4 prefill of {q4d['prefill_tokens']} tokens: {q4d['prefill_ms']:.2f} ms")
    if args.suite in ("all", "gemv", "step") and not args.only:
        q4 = bench_q4km_step(ctx, args.steps, args.warmup)
        gbs = q4["bytes"] / (q4["us"] * 1e-6) / 1e9
        log(f"config 4 (7B Q4_K_M mix, all 28 layers' GEMVs + Q6_K LM head, {q4['launches']} "
            f"launches): {q4['us']:.1f} us per token = {1e6 / q4['us']:.1f} tok/s of GEMVs; "
            f"{q4['bytes'] / 1e9:.3f} GB → {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% HBM); "
            f"with separate bias-free Q/K/V GEMVs ({q4['launches_separate_qkv']} launches): "
            f"{q4['us_separate_qkv']:.1f} us")
        line["q4k_m_7b_gemv_step"] = {
            "us_per_token": round(q4["us"], 1), "tok_s_gemv_only": round(1e6 / q4["us"], 1),
            "bytes": q4["bytes"], "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "launches": q4["launches"],
            "us_per_token_separate_qkv": round(q4["us_separate_qkv"], 1)}
    specs = [] if args.suite in ("decode", "step", "q4decode") else gemv_specs(ctx, args.suite)
    if args.only:
        specs = [sp for sp in specs if args.only in sp[0]]
    results = []
    for label, mk in specs:
        wl = mk()
        r = time_workload(ctx, wl, max(3, args.steps // 10), min(args.warmup, 2))
        r["label"] = label
        log(f"{label:34s} {r['us']:9.2f} us  {r['gbs']:8.1f} GB/s  {100 * r['frac_hbm']:5.1f}% HBM"
            f"  ({r['launches']} launches, {wl.reps} replicas)")
        results.append(r)
        wl.free()
    if results:
        line["gemv"] = {r["label"]: {"us": r["us"], "gbs": r["gbs"], "frac": r["frac_hbm"],
                                     "tflops": r["tflops"]} for r in results}
    if dec is None and results:
        r0 = results[0]
        line.update({"value": r0["gbs"], "unit": "GB/s", "ms_per_step": round(r0["us"] * 1e-3, 5),
                     "dtype": "quant x f32", "config": {"workload": r0["label"]},
                     "roofline": {"bound": "hbm", "achieved": r0["gbs"], "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": r0["frac_hbm"], "traffic": None}})
    if dec is not None:
        if not args.no_cpu:
            cb = cpu_baseline(dec["model"], 1, dec["pos"], dec["gpu_token"])
            log(f"cpu baseline: {cb['ms_per_token']} ms/token single-thread, "
                f"{cb['all_cores']['ms_per_token']} ms/token on {cb['all_cores']['cores']} "
                f"threads; token {cb['token']} (GPU {cb['gpu_token']})")
            line["cpu_baseline"] = cb
        dec["model"].free()
    ctx.close()
    print(json.dumps(line), flush=True)


def gemv_specs(ctx, suite):
    specs = [
        ("c1_q8_0_ffn_up_4864x896", lambda: Workload(ctx, "c1", "q8_0", "gemv", 4864, 896, seed=1)),
        ("c3_q4_0_ffn_2x18944x3584", lambda: Workload(ctx, "c3_ffn", "q4_0", "ffn", 18944, 3584, seed=2)),
        ("c3_q4_0_down_3584x18944", lambda: Workload(ctx, "c3_down", "q4_0", "add", 3584, 18944, seed=3)),
        ("c3_q4_0_qkv_4608x3584", lambda: QKVWorkload(ctx, "c3_qkv", "q4_0", 3584, 512, 3584, seed=4)),
        ("c4_q4k_q_3584x3584", lambda: Workload(ctx, "c4_q", "q4k", "gemv", 3584, 3584, seed=5)),
        ("c4_q4k_k_512x3584", lambda: Workload(ctx, "c4_k", "q4k", "gemv", 512, 3584, seed=21)),
        ("c4_q6k_v_512x3584", lambda: Workload(ctx, "c4_v", "q6k", "gemv", 512, 3584, seed=22)),
        ("c4_qkv_bias_q4k_q6k_4608x3584", lambda: QKVWorkload(ctx, "c4_qkv", "q4k", 3584, 512, 3584,
                                                             seed=24, fmt_v="q6k")),
        ("c4_q4k_o_add_3584x3584", lambda: Workload(ctx, "c4_o", "q4k", "add", 3584, 3584, seed=23)),
        ("c4_q4k_ffn_2x18944x3584", lambda: Workload(ctx, "c4_ffn", "q4k", "ffn", 18944, 3584, seed=6)),
        ("c4_q6k_down_3584x18944", lambda: Workload(ctx, "c4_down", "q6k", "add", 3584, 18944, seed=7)),
        ("c4_q6k_lmhead_152064x3584", lambda: Workload(ctx, "c4_lm", "q6k", "gemv", 152064, 3584, seed=8)),
        ("c2_q8_0_lmhead_151936x896", lambda: Workload(ctx, "c2_lm", "q8_0", "gemv", 151936, 896, seed=9)),
        ("c2_q8_0_ffn_2x4864x896", lambda: Workload(ctx, "c2_ffn", "q8_0", "ffn", 4864, 896, seed=10)),
    ]
    if suite in ("all", "gemv"):
        # 5-bit formats (Q5_K_M / Q5_0 files) at the 7B shapes
        specs += [
            ("c6_q5k_ffn_2x18944x3584", lambda: Workload(ctx, "c6_ffn", "q5k", "ffn", 18944, 3584, seed=13)),
            ("c6_q5k_down_3584x18944", lambda: Workload(ctx, "c6_down", "q5k", "add", 3584, 18944, seed=14)),
            ("c6_q5_0_ffn_2x18944x3584", lambda: Workload(ctx, "c6_ffn0", "q5_0", "ffn", 18944, 3584, seed=15)),
            # ggml layouts of the config-4 mix (upstream Q4_K_M files)
            ("c4g_q4kg_ffn_2x18944x3584", lambda: Workload(ctx, "c4g_ffn", "q4kg", "ffn", 18944, 3584, seed=16)),
            ("c4g_q6kg_down_3584x18944", lambda: Workload(ctx, "c4g_down", "q6kg", "add", 3584, 18944, seed=17)),
            ("c4g_q6kg_lmhead_152064x3584", lambda: Workload(ctx, "c4g_lm", "q6kg", "gemv", 152064, 3584, seed=18)),
            ("c3g_q4_0g_ffn_2x18944x3584", lambda: Workload(ctx, "c3g_ffn", "q4_0g", "ffn", 18944, 3584, seed=19)),
        ]
        for fmt in ("q4_0", "q4k"):  # verify / prefill GEMM of the 4-bit 7B formats
            for m in (4, 16, 32):
                specs.append((f"c5q_gemm_{fmt}_m{m}_18944x3584",
                              (lambda m=m, fmt=fmt: Workload(ctx, "c5q", fmt, "gemm", 18944, 3584,
                                                             m=m, seed=20))))
        for m in (4, 16, 32):  # the Q4_K_M mix's Q6_K down projection, batched
            specs.append((f"c5q_gemm_q6k_m{m}_3584x18944",
                          (lambda m=m: Workload(ctx, "c5q", "q6k", "gemm", 3584, 18944, m=m, seed=21))))
        for m in (1, 4, 8, 16, 32):
            specs.append((f"c5_gemm_q8_0_m{m}_18944x3584",
                          (lambda m=m: Workload(ctx, "c5", "q8_0", "gemm", 18944, 3584, m=m, seed=11))))
            specs.append((f"c5_gemm_q8_0_m{m}_3584x18944",
                          (lambda m=m: Workload(ctx, "c5", "q8_0", "gemm", 3584, 18944, m=m, seed=12))))
    return specs


if __name__ == "__main__":
    main()
