"""The BASELINE.json configurations at full size, on the GPU, against the
oracle (f64) on identical seeded inputs (weights generated on the device,
downloaded, and checked on the host)."""
import numpy as np
import pytest

import oracle_lib as ora
from gpu_helpers import check_close, device_normal, device_weights
from test_gpu_fused import ffn_check
from runit_mac_amd import dispatch as d

pytestmark = pytest.mark.gpu


def _gemv(ctx, fmt, n, k, seed, fn):
    wbuf, raw = device_weights(ctx, fmt, n, k, seed)
    xb, x = device_normal(ctx, k, seed + 1)
    y = ctx.new_buffer(4 * n)
    fn(ctx, wbuf, xb, y, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(y.read(np.float32, n), yref, sabs, f"{fmt} {n}x{k}")
    return y.read(np.float32, n), yref


def test_config1_q8_0_ffn_up_0p5b(ctx):
    # W 4864×896 Q8_0 from N(0, 0.02), x ~ N(0, 1)
    _gemv(ctx, "q8_0", 4864, 896, 2024, d.gemv_q8_0_f32in_f32out)


def test_config2_lm_head_argmax_0p5b(ctx):
    # LM head 151936×896 Q8_0 followed by argmax: identical to the oracle's
    # argmax whenever the top-2 gap exceeds the tolerance of both entries.
    n, k = 151936, 896
    wbuf, raw = device_weights(ctx, "q8_0", n, k, 31)
    xb, x = device_normal(ctx, k, 32)
    y = ctx.new_buffer(4 * n)
    d.gemv_q8_0_f32in_f32out_mr(ctx, wbuf, xb, y, n, k)
    res = ctx.new_buffer(4)
    d.argmax_f32(ctx, y, res, n)
    ctx.flush()
    got = y.read(np.float32, n)
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    check_close(got, yref, sabs, "lm head")
    top = np.argsort(yref)[-2:]
    gap = yref[top[1]] - yref[top[0]]
    assert gap > 1e-4 * (sabs[top[0]] + sabs[top[1]]), "seed gives an ambiguous argmax"
    assert int(res.read(np.uint32, 1)[0]) == ora.argmax(yref.astype(np.float32)) == int(top[1])


def test_config3_q4_0_7b_shapes(ctx):
    ff, h = 18944, 3584
    wg, rg = device_weights(ctx, "q4_0", ff, h, 41)
    wu, ru = device_weights(ctx, "q4_0", ff, h, 42)
    xb, x = device_normal(ctx, h, 43)
    act = ctx.new_buffer(4 * ff)
    d.fused_ffn_q4_0_f32(ctx, wg, wu, xb, act, ff, h)
    ctx.flush()
    g, gs = ora.gemv("q4_0", rg, x, ff, h)
    u, us = ora.gemv("q4_0", ru, x, ff, h)
    ffn_check(act.read(np.float32, ff), g, gs, u, us, "7B q4_0 ffn")
    del wg, wu
    _gemv(ctx, "q4_0", h, ff, 44, d.gemv_q4_0_f32in_f32out)  # down 3584×18944


def test_config4_q4k_q6k_7b_shapes(ctx):
    _gemv(ctx, "q4k", 3584, 3584, 51, d.gemv_q4k_f32in_f32out)    # Q / O
    _gemv(ctx, "q4k", 18944, 3584, 52, d.gemv_q4k_f32in_f32out)   # gate / up
    _gemv(ctx, "q6k", 512, 3584, 53, d.gemv_q6k_f32in_f32out)     # V
    _gemv(ctx, "q6k", 3584, 18944, 54, d.gemv_q6k_f32in_f32out)   # down


def test_config4_q6k_lm_head_argmax(ctx):
    n, k = 152064, 3584
    wbuf, raw = device_weights(ctx, "q6k", n, k, 61)
    xb, x = device_normal(ctx, k, 62)
    y = ctx.new_buffer(4 * n)
    d.gemv_q6k_f32in_f32out(ctx, wbuf, xb, y, n, k)
    res = ctx.new_buffer(4)
    d.argmax_f32(ctx, y, res, n)
    ctx.flush()
    yref, sabs = ora.gemv("q6k", raw, x, n, k)
    check_close(y.read(np.float32, n), yref, sabs, "q6k lm head")
    assert int(res.read(np.uint32, 1)[0]) == ora.argmax(yref.astype(np.float32))


@pytest.mark.parametrize("m", [1, 4, 8, 16, 32])
def test_config5_gemm_q8_0_7b(ctx, m):
    for n, k, s in ((18944, 3584, 71), (3584, 18944, 72)):
        wbuf, raw = device_weights(ctx, "q8_0", n, k, s + m)
        x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
        y = ctx.new_buffer(4 * m * n)
        d.gemm_q8_0_f32(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
        ctx.flush()
        yref, sabs = ora.gemv("q8_0", raw, x, n, k)
        check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm {m}x{n}x{k}")


@pytest.mark.parametrize("fmt,n,k,m", [("q6k", 3584, 18944, 2), ("q6k", 3584, 18944, 8),
                                       ("q6k", 3584, 18944, 32), ("q6kg", 3584, 18944, 32),
                                       ("q4k", 18944, 3584, 4), ("q4k", 18944, 3584, 32),
                                       ("q4_0", 18944, 3584, 32)])
def test_config5_gemm_4bit_q6k_7b(ctx, fmt, n, k, m):
    # the bench's batched 4-bit / Q6_K lines at full size: Q6_K on 128-row
    # tiles with the planner's K splits filling the CUs (28 tiles × 8
    # splits), Q4_K on 256-row tiles at 32 rows, the int8 form at 4
    wbuf, raw = device_weights(ctx, fmt, n, k, 170 + m)
    x = np.random.default_rng(m + 1).standard_normal((m, k)).astype(np.float32)
    y = ctx.new_buffer(4 * m * n)
    getattr(d, f"gemm_{fmt}_f32")(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm {fmt} {m}x{n}x{k}")


@pytest.mark.parametrize("fmt", ["q4kg", "q5k", "q5_0"])
def test_7b_ffn_other_formats(ctx, fmt):
    # the 7B gate+up+SiLU in the ggml Q4_K layout (upstream Q4_K_M files) and
    # the Q5 formats (Q5_K_M / Q5_0 files): the LDS-streamed body at full size
    ff, h = 18944, 3584
    wg, rg = device_weights(ctx, fmt, ff, h, 81)
    wu, ru = device_weights(ctx, fmt, ff, h, 82)
    xb, x = device_normal(ctx, h, 83)
    act = ctx.new_buffer(4 * ff)
    getattr(d, f"fused_ffn_{fmt}_f32")(ctx, wg, wu, xb, act, ff, h)
    ctx.flush()
    g, gs = ora.gemv(fmt, rg, x, ff, h)
    u, us = ora.gemv(fmt, ru, x, ff, h)
    ffn_check(act.read(np.float32, ff), g, gs, u, us, f"7B {fmt} ffn")


@pytest.mark.parametrize("fmt", ["q6kg", "q5k", "q4kg"])
def test_7b_down_other_formats(ctx, fmt):
    # down 3584×18944 (+ residual, aliased as in forward.rs:1702): K split
    # into chunks whose partial sums meet through memory
    n, k = 3584, 18944
    wbuf, raw = device_weights(ctx, fmt, n, k, 91)
    xb, x = device_normal(ctx, k, 92)
    res = np.random.default_rng(93).standard_normal(n).astype(np.float32)
    yr = ctx.buffer_from(res)
    getattr(d, f"gemv_{fmt}_add_f32_f32in")(ctx, wbuf, xb, yr, yr, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(yr.read(np.float32, n), yref + res, sabs, f"7B {fmt} down")
