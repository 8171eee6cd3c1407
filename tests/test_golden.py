"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the oracle reproduces the fixtures exactly and meets the closed forms.
GPU: the HIP path (through the C ABI) matches the fixtures — dequantisation
bit-exact, GEMV / fused outputs within 1e-4·Σ|w·x| per row, argmax equal.
"""
import os

import numpy as np
import pytest

import oracle_lib as ora
from gpu_helpers import check_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FMTS = ["q8_0", "q4_0", "q4k", "q6k"]


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def gemv_cases(fmt):
    f = load(f"gemv_{fmt}.npz")
    i = 0
    while f"w{i}" in f:
        n, k = (int(v) for v in f[f"shape{i}"])
        yield n, k, f[f"w{i}"], f[f"x{i}"], f[f"y{i}"], f[f"sabs{i}"], f[f"deq{i}"]
        i += 1


# ───────────────────────────── CPU ─────────────────────────────

@pytest.mark.parametrize("fmt", FMTS)
def test_oracle_reproduces_gemv_fixtures(fmt):
    for n, k, w, x, y, s, deq in gemv_cases(fmt):
        assert np.array_equal(ora.dequant(fmt, w).view(np.uint32), deq.view(np.uint32))
        y2, s2 = ora.gemv(fmt, w, x, n, k)
        assert np.allclose(y2, y, rtol=0, atol=1e-12) and np.allclose(s2, s, rtol=0, atol=1e-12)


def test_oracle_closed_forms():
    c = load("closed_forms.npz")
    for fmt in ("q8_0", "q4_0"):
        y, _ = ora.gemv(fmt, c[f"ones_{fmt}"], c["ones_x"], 4, 64)
        assert np.array_equal(y, c["ones_y"])
    y, _ = ora.gemv("q8_0", c["eye_q8_0"], c["ones_x"], 4, 64)
    assert np.array_equal(y, c["eye_y"])
    for key in ("q8_0", "q8_0h", "q4_0", "q4k", "q4kz"):
        fmt = key.rstrip("hz") if key != "q8_0h" else "q8_0"
        got = ora.dequant(fmt, c[f"deq_{key}_in"])
        assert np.array_equal(got, c[f"deq_{key}_out"]), key


def test_oracle_reproduces_fused_fixtures():
    f = load("fused.npz")
    qd, kd, k = (int(v) for v in f["qkv_shape"])
    for name, n in (("q", qd), ("k", kd), ("v", kd)):
        y, _ = ora.gemv("q8_0", f[f"qkv_w{name}"], f["qkv_x"], n, k)
        bias = f[f"qkv_b{name}"].view(np.float16).astype(np.float64)
        assert np.allclose(y + bias, f[f"qkv_y{name}"], rtol=0, atol=1e-12)
    i = 0
    while f"argmax_v{i}" in f:
        assert ora.argmax(f[f"argmax_v{i}"]) == int(f[f"argmax_r{i}"])
        i += 1


# ───────────────────────────── GPU ─────────────────────────────

@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FMTS)
def test_device_gemv_and_dequant_match_fixtures(ctx, fmt):
    from runit_mac_amd import dispatch as d
    gemv = getattr(d, f"gemv_{fmt}_f32in_f32out")
    for n, k, w, x, y, s, deq in gemv_cases(fmt):
        wb = ctx.buffer_from(w)
        out = ctx.new_buffer(4 * n)
        dq = ctx.new_buffer(4 * deq.size)
        gemv(ctx, wb, ctx.buffer_from(x), out, n, k)
        d.dequant_f32(ctx, fmt, wb, dq, w.size // d.BLOCK[fmt][1])
        ctx.flush()
        check_close(out.read(np.float32, n), y, s, f"{fmt} {n}x{k}")
        assert np.array_equal(dq.read(np.uint32, deq.size), deq.view(np.uint32)), fmt


@pytest.mark.gpu
def test_device_closed_forms(ctx):
    from runit_mac_amd import dispatch as d
    c = load("closed_forms.npz")
    x = ctx.buffer_from(c["ones_x"])
    for key, fn in (("ones_q8_0", d.gemv_q8_0_f32in_f32out), ("ones_q4_0", d.gemv_q4_0_f32in_f32out),
                    ("eye_q8_0", d.gemv_q8_0_f32in_f32out)):
        out = ctx.new_buffer(16)
        fn(ctx, ctx.buffer_from(c[key]), x, out, 4, 64)
        ctx.flush()
        want = c["eye_y"] if key.startswith("eye") else c["ones_y"]
        assert np.array_equal(out.read(np.float32, 4).astype(np.float64), want), key
    for key, fmt in (("q8_0", "q8_0"), ("q8_0h", "q8_0"), ("q4_0", "q4_0"), ("q4k", "q4k"),
                     ("q4kz", "q4k")):
        src = c[f"deq_{key}_in"]
        ref = c[f"deq_{key}_out"]
        out = ctx.new_buffer(4 * ref.size)
        d.dequant_f32(ctx, fmt, ctx.buffer_from(src), out, src.size // d.BLOCK[fmt][1])
        ctx.flush()
        assert np.array_equal(out.read(np.float32, ref.size), ref), key


@pytest.mark.gpu
def test_device_fused_match_fixtures(ctx):
    from runit_mac_amd import dispatch as d
    f = load("fused.npz")
    qd, kd, k = (int(v) for v in f["qkv_shape"])
    outs = [ctx.new_buffer(4 * n) for n in (qd, kd, kd)]
    d.fused_qkv_bias_q8_0_f32(ctx, *[ctx.buffer_from(f[f"qkv_w{c}"]) for c in "qkv"],
                              ctx.buffer_from(f["qkv_x"]), *outs,
                              *[ctx.buffer_from(f[f"qkv_b{c}"]) for c in "qkv"], qd, kd, k)
    ctx.flush()
    for c, n, o in zip("qkv", (qd, kd, kd), outs):
        check_close(o.read(np.float32, n), f[f"qkv_y{c}"], f[f"qkv_s{c}"], f"qkv {c}")
    ff, k = (int(v) for v in f["ffn_shape"])
    for fmt, fn in (("q8_0", d.fused_ffn_q8_0_f32), ("q4_0", d.fused_ffn_q4_0_f32)):
        act = ctx.new_buffer(4 * ff)
        fn(ctx, ctx.buffer_from(f[f"ffn_{fmt}_wg"]), ctx.buffer_from(f[f"ffn_{fmt}_wu"]),
           ctx.buffer_from(f[f"ffn_{fmt}_x"]), act, ff, k)
        ctx.flush()
        g, u = f[f"ffn_{fmt}_g"], f[f"ffn_{fmt}_u"]
        gs, us = f[f"ffn_{fmt}_gs"], f[f"ffn_{fmt}_us"]
        # |silu'| ≤ 1.1: act error ≤ 1.1·|u|·eg + |silu(g)|·eu (+ f32 rounding)
        sg = np.abs(g) / (1 + np.exp(-g))
        tol = 1.1 * np.abs(u) * 1e-4 * gs + sg * 1e-4 * us + 4 * 2.0 ** -24 * np.abs(
            f[f"ffn_{fmt}_act"])
        got = act.read(np.float32, ff).astype(np.float64)
        assert np.all(np.abs(got - f[f"ffn_{fmt}_act"]) <= tol), fmt
    i = 0
    res = ctx.new_buffer(4)
    while f"argmax_v{i}" in f:
        d.argmax_f32(ctx, ctx.buffer_from(f[f"argmax_v{i}"]), res, f[f"argmax_v{i}"].size)
        ctx.flush()
        assert int(res.read(np.uint32, 1)[0]) == int(f[f"argmax_r{i}"]), i
        i += 1
