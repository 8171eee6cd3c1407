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
                d.synth_weights(ctx, fmt, b, n * k // el, seed * 1000 + r * 2 + j)
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
            d.gemm_q8_0_f32(ctx, w[0], self.x, self.y, self.m, n, k)
        else:
            raise ValueError(self.kind)

    def free(self):
        self.arena.free()
        self.w = []


class QKVWorkload(Workload):
    def __init__(self, ctx, name, fmt, q_dim, kv_dim, k, seed=1):
        self.q_dim, self.kv_dim = q_dim, kv_dim
        self.ctx, self.name, self.fmt, self.kind, self.k, self.m = ctx, name, fmt, "qkv", k, 1
        self.n = q_dim + 2 * kv_dim
        el, _ = d.BLOCK[fmt]
        dims = (q_dim, kv_dim, kv_dim)
        self.wbytes_per_launch = sum(d.weight_bytes(fmt, n, k) for n in dims)
        self.reps = max(2, min(512, -(-WORKSET_BYTES // self.wbytes_per_launch)))
        self.arena = _arena_for(ctx, [d.weight_bytes(fmt, n, k) for n in dims], self.reps)
        self.w = []
        for r in range(self.reps):
            mats = []
            for j, n in enumerate(dims):
                b = self.arena.take(d.weight_bytes(fmt, n, k))
                d.synth_weights(ctx, fmt, b, n * k // el, seed * 1000 + r * 3 + j)
                mats.append(b)
            self.w.append(mats)
        self.x = ctx.new_buffer(4 * k)
        d.synth_normal_f32(ctx, self.x, k, seed + 7)
        self.outs = [ctx.new_buffer(4 * n) for n in dims]
        self.bias = [ctx.new_buffer(2 * n) for n in dims]
        for i, (b, n) in enumerate(zip(self.bias, dims)):
            d.synth_normal_f16(ctx, b, n, seed + 20 + i, 0.0, 0.02)
        ctx.flush()

    def launch(self, r: int):
        w = self.w[r % self.reps]
        getattr(d, f"fused_qkv_bias_{self.fmt}_f32")(
            self.ctx, w[0], w[1], w[2], self.x, *self.outs, *self.bias,
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


def cpu_baseline(seconds: float = 10.0) -> dict:
    """Reference CPU path (oracle restatement) on config 1: Q8_0 4864×896."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import oracle_lib as ora  # noqa: E402  (test infrastructure, baseline only)
    n, k = 4864, 896
    w = ora.synth_weights("q8_0", n, k, seed=1) if False else None
    # host weights: random bytes with valid f16 scales (values do not affect timing)
    rng = np.random.default_rng(1)
    raw = rng.integers(-127, 128, size=(n * k // 32, 34), dtype=np.int16).astype(np.uint8)
    scale = np.float16(0.0005).view(np.uint16)
    raw[:, 0] = scale & 255
    raw[:, 1] = scale >> 8
    raw = raw.ravel()
    x = rng.standard_normal(k).astype(np.float32)
    out = {}
    for threads in (1, os.cpu_count() or 1):
        t0 = time.perf_counter()
        it = 0
        while True:
            ora.gemv_ref_f32("q8_0", raw, x, n, k, threads)
            it += 1
            el = time.perf_counter() - t0
            if el > seconds / 2:
                break
        out[threads] = el / it
    del w
    b = n * (k // 32) * 34 + 4 * k + 4 * n
    t1 = out[1]
    tn = out[max(out)]
    return {"value": round(b / t1 / 1e9, 3), "unit": "GB/s",
            "cores": 1, "kind": "port",
            "sample": f"config 1 Q8_0 4864x896 GEMV, dequant+sequential f32 dot, "
                      f"{1e3 * t1:.2f} ms/GEMV single-thread; {max(out)}-thread OpenMP "
                      f"{1e3 * tn:.3f} ms/GEMV ({b / tn / 1e9:.2f} GB/s)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--suite", default="all", choices=["all", "gemv", "quick"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None, help="run only workloads whose label contains this")
    args = ap.parse_args()
    if args.gpus != 1:
        sys.exit("bench.py measures one GPU only: this build has no multi-GPU path "
                 "(see DESIGN.md on how the path would shard); run with --gpus 1")

    ctx = d.HipContext()
    specs = [
        ("c1_q8_0_ffn_up_4864x896", lambda: Workload(ctx, "c1", "q8_0", "gemv", 4864, 896, seed=1)),
        ("c3_q4_0_ffn_2x18944x3584", lambda: Workload(ctx, "c3_ffn", "q4_0", "ffn", 18944, 3584, seed=2)),
        ("c3_q4_0_down_3584x18944", lambda: Workload(ctx, "c3_down", "q4_0", "add", 3584, 18944, seed=3)),
        ("c3_q4_0_qkv_4608x3584", lambda: QKVWorkload(ctx, "c3_qkv", "q4_0", 3584, 512, 3584, seed=4)),
        ("x_q4_0_plain_4608x3584", lambda: Workload(ctx, "xq4", "q4_0", "gemv", 4608, 3584, seed=12)),
        ("x_q8_0_plain_4608x3584", lambda: Workload(ctx, "xq8", "q8_0", "gemv", 4608, 3584, seed=13)),
        ("c4_q4k_q_3584x3584", lambda: Workload(ctx, "c4_q", "q4k", "gemv", 3584, 3584, seed=5)),
        ("c4_q4k_ffn_2x18944x3584", lambda: Workload(ctx, "c4_ffn", "q4k", "ffn", 18944, 3584, seed=6)),
        ("c4_q6k_down_3584x18944", lambda: Workload(ctx, "c4_down", "q6k", "add", 3584, 18944, seed=7)),
        ("c4_q6k_lmhead_152064x3584", lambda: Workload(ctx, "c4_lm", "q6k", "gemv", 152064, 3584, seed=8)),
        ("c2_q8_0_lmhead_151936x896", lambda: Workload(ctx, "c2_lm", "q8_0", "gemv", 151936, 896, seed=9)),
        ("c2_q8_0_ffn_2x4864x896", lambda: Workload(ctx, "c2_ffn", "q8_0", "ffn", 4864, 896, seed=10)),
    ]
    if args.suite != "quick":
        for m in (1, 4, 8, 16, 32):
            specs.append((f"c5_gemm_q8_0_m{m}_18944x3584",
                          (lambda m=m: Workload(ctx, "c5", "q8_0", "gemm", 18944, 3584, m=m, seed=11))))
    if args.only:
        specs = [sp for sp in specs if args.only in sp[0]]
    results = []
    for label, mk in specs:
        wl = mk()
        r = time_workload(ctx, wl, args.steps, args.warmup)
        r["label"] = label
        log(f"{label:34s} {r['us']:9.2f} us  {r['gbs']:8.1f} GB/s  {100 * r['frac_hbm']:5.1f}% HBM"
            f"  ({r['launches']} launches, {wl.reps} replicas)")
        results.append(r)
        wl.free()

    # headline until the decode step lands: the 7B Q4_0 fused FFN GEMV
    main_r = next((r for r in results if r["label"] == "c3_q4_0_ffn_2x18944x3584"), results[0])
    line = {
        "metric": "quant GEMV HBM GB/s (% of peak) + decode tok/s, 0.5B Q8_0 & 7B Q4_K",
        "value": main_r["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(main_r["us"] * 1e-3, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "q4_0xf32",
        "data": "synthetic (seeded N(0,0.02) weights quantised per block, N(0,1) activations)",
        "config": {"workload": "config 3: Q4_0 fused gate+up+SiLU 2x18944x3584, M=1"},
        "roofline": {"bound": "hbm", "achieved": main_r["gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": main_r["frac_hbm"], "traffic": None},
        "gemv": {r["label"]: {"us": r["us"], "gbs": r["gbs"], "frac": r["frac_hbm"],
                              "tflops": r["tflops"]} for r in results},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
