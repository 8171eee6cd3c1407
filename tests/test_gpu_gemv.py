"""GPU parity of the quantized GEMV family against the CPU oracle.

Every call goes through the C ABI (librunit_hip.so) via the dispatch mirror.
Tolerance (BASELINE): |y − y_ref| ≤ 1e-4·Σ|w_i·x_i| per row, y_ref in f64;
f16 outputs additionally get one binary16 rounding (gpu_helpers.f16_extra);
dequantisation is compared bit for bit.
"""
import numpy as np
import pytest

import oracle_lib as ora
from gpu_helpers import (F32_EPS, check_close, device_normal, device_weights, f16_extra,
                         f16_to_f64)
from runit_mac_amd import dispatch as d

pytestmark = pytest.mark.gpu

FMTS = ["q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg", "q5kg", "q6kg"]

VARIANTS = {
    "q8_0": ["f32in_f32out", "add_f32_f32in", "f32in", "f16", "add_f16", "add_f32res_f16",
             "f32in_f32out_mr", "add_f32_f32in_mr"],
    "q4_0": ["f32in_f32out", "add_f32_f32in", "f32in", "f16", "add_f16"],
    "q4k": ["f32in_f32out", "add_f32_f32in", "f16", "add_f16", "add_f32res_f16"],
    "q6k": ["f32in_f32out", "add_f32_f32in", "f32in"],
    "q5_0": ["f32in_f32out", "add_f32_f32in", "f32in"],
    "q5k": ["f32in_f32out", "add_f32_f32in", "f32in"],
    **{g: ["f32in_f32out", "add_f32_f32in", "f32in"] for g in ("q4_0g", "q4kg", "q5kg", "q6kg")},
}


def run_variant(ctx, fmt, var, wbuf, wraw, n, k, seed):
    """Runs dispatch.gemv_<fmt>_<var> on seeded inputs and checks it."""
    rng = np.random.default_rng(seed)
    x_f16_in = var in ("f16", "add_f16", "add_f32res_f16")
    x32 = rng.standard_normal(k).astype(np.float32)
    if x_f16_in:
        x16 = x32.astype(np.float16)
        x32 = x16.astype(np.float32)
        xbuf = ctx.buffer_from(x16)
    else:
        xbuf = ctx.buffer_from(x32)
    yref, sabs = ora.gemv(fmt, wraw, x32, n, k)
    fn = getattr(d, f"gemv_{fmt}_{var}")
    out_f16 = var in ("f32in", "f16", "add_f16")
    ybuf = ctx.new_buffer(n * (2 if out_f16 else 4))
    if var.startswith("add"):
        res32 = rng.standard_normal(n).astype(np.float32)
        if var == "add_f16":
            res16 = res32.astype(np.float16)
            res32 = res16.astype(np.float32)
            rbuf = ctx.buffer_from(res16)
        else:
            rbuf = ctx.buffer_from(res32)
        fn(ctx, wbuf, xbuf, ybuf, rbuf, n, k)
        ref = yref + res32.astype(np.float64)
    else:
        fn(ctx, wbuf, xbuf, ybuf, n, k)
        ref = yref
    ctx.flush()
    if out_f16:
        got = f16_to_f64(ybuf.read(np.uint16, n))
        check_close(got, ref, sabs, f"{fmt}/{var} {n}x{k}", f16_extra(ref, sabs))
    else:
        got = ybuf.read(np.float32, n)
        check_close(got, ref, sabs, f"{fmt}/{var} {n}x{k}", F32_EPS * np.abs(ref))


# ───────────────────────── dequantisation: bit-exact ─────────────────────────

def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan]) and
                np.array_equal(np.isnan(a), np.isnan(b)))


@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_bit_exact_synth(ctx, fmt):
    el, by = d.BLOCK[fmt]
    n, k = 48, 1024
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=101)
    nblk = n * k // el
    out = ctx.new_buffer(4 * n * k)
    d.dequant_f32(ctx, fmt, wbuf, out, nblk)
    ctx.flush()
    assert _bits_equal(out.read(np.float32, n * k), ora.dequant(fmt, raw))


@pytest.mark.parametrize("fmt", FMTS)
def test_dequant_bit_exact_random_bytes(ctx, fmt):
    # arbitrary bit patterns: subnormal / Inf / NaN scales, every code value
    el, by = d.BLOCK[fmt]
    nblk = 333
    raw = np.random.default_rng(7).integers(0, 256, nblk * by, dtype=np.uint8)
    out = ctx.new_buffer(4 * nblk * el)
    d.dequant_f32(ctx, fmt, ctx.buffer_from(raw), out, nblk)
    ctx.flush()
    assert _bits_equal(out.read(np.float32, nblk * el), ora.dequant(fmt, raw))


def test_dequant_q4k_f16_bit_exact(ctx):
    nblk = 257
    raw = np.random.default_rng(8).integers(0, 256, nblk * 144, dtype=np.uint8)
    out = ctx.new_buffer(2 * nblk * 256)
    d.dequant_q4k_f16(ctx, ctx.buffer_from(raw), out, nblk)
    ctx.flush()
    got = out.read(np.uint16, nblk * 256)
    ref = ora.dequant_q4k_f16(raw)
    gn = np.isnan(got.view(np.float16))
    rn = np.isnan(ref.view(np.float16))
    assert np.array_equal(gn, rn) and np.array_equal(got[~gn], ref[~rn])


# ───────────────────────── GEMV variants ─────────────────────────

SHAPES = [(64, 256), (37, 512), (300, 768), (1, 2048), (129, 1536)]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("n,k", SHAPES)
def test_gemv_variants(ctx, fmt, n, k):
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=1000 + n + k)
    for i, var in enumerate(VARIANTS[fmt]):
        run_variant(ctx, fmt, var, wbuf, raw, n, k, seed=17 * i + n)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q5_0", "q4_0g"])
@pytest.mark.parametrize("k", [32, 64, 96, 160])
def test_gemv_small_and_odd_block_counts(ctx, fmt, k):
    n = 77
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=5 + k)
    run_variant(ctx, fmt, "f32in_f32out", wbuf, raw, n, k, seed=k)


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_long_k_staged_in_chunks(ctx, fmt):
    # K = 32768 → 1024 activation records = 112 KiB > the per-pass LDS budget,
    # so the kernel restages the activations in several passes.
    n, k = 96, 32768
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=77)
    run_variant(ctx, fmt, "f32in_f32out", wbuf, raw, n, k, seed=3)
    run_variant(ctx, fmt, "add_f32_f32in", wbuf, raw, n, k, seed=4)


@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_output_aliases_residual(ctx, fmt):
    # forward.rs:1619,1702 pass the same buffer as output and residual
    n, k = 513, 1024
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=9)
    x = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    res = np.random.default_rng(2).standard_normal(n).astype(np.float32)
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    buf = ctx.buffer_from(res)
    getattr(d, f"gemv_{fmt}_add_f32_f32in")(ctx, wbuf, ctx.buffer_from(x), buf, buf, n, k)
    ctx.flush()
    ref = yref + res
    check_close(buf.read(np.float32, n), ref, sabs, f"{fmt} aliased", F32_EPS * np.abs(ref))


def test_gemv_heavy_tailed_activations(ctx):
    # activations with 100× outliers inside blocks (post-norm LLM activations
    # have such channels): the limb form keeps 22 bits below the block max
    n, k = 256, 4096
    wbuf, raw = device_weights(ctx, "q8_0", n, k, seed=12)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(k).astype(np.float32)
    x[rng.integers(0, k, 40)] *= 100.0
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    y = ctx.new_buffer(4 * n)
    d.gemv_q8_0_f32in_f32out(ctx, wbuf, ctx.buffer_from(x), y, n, k)
    ctx.flush()
    check_close(y.read(np.float32, n), yref, sabs, "heavy-tailed x")


def test_gemv_zero_and_tiny_activations(ctx):
    n, k = 64, 512
    wbuf, raw = device_weights(ctx, "q4k", n, k, seed=13)
    x = np.zeros(k, np.float32)
    x[100:132] = np.float32(1e-40)  # subnormal block
    x[300] = np.float32(3.0e-30)
    yref, sabs = ora.gemv("q4k", raw, x, n, k)
    y = ctx.new_buffer(4 * n)
    d.gemv_q4k_f32in_f32out(ctx, wbuf, ctx.buffer_from(x), y, n, k)
    ctx.flush()
    check_close(y.read(np.float32, n), yref, sabs, "tiny x", 1e-44)


def test_gemv_rejects_bad_k(ctx):
    w = ctx.new_buffer(1024)
    x = ctx.new_buffer(1024)
    y = ctx.new_buffer(1024)
    with pytest.raises(d.Dispatch):
        d.gemv_q8_0_f32in_f32out(ctx, w, x, y, 4, 48)
    with pytest.raises(d.Dispatch):
        d.gemv_q4k_f32in_f32out(ctx, w, x, y, 4, 128)
    with pytest.raises(d.Dispatch):  # misaligned activation pointer
        d.gemv_q8_0_f32in_f32out(ctx, w, x.ptr + 4, y, 4, 64)
    # m = 0 is a no-op, like a zero-width Metal dispatch
    d.gemv_q8_0_f32in_f32out(ctx, w, x, y, 0, 64)
    ctx.flush()


def test_pipeline_lookup(ctx):
    ctx.has_kernel("k_gemv_q8_0_f32_f32_r1")
    with pytest.raises(d.PipelineNotFound):
        ctx.has_kernel("no_such_kernel")


# ───────────── K split over workgroups (K > 8192, matrix-core path) ─────────────

@pytest.mark.parametrize("fmt", FMTS)
def test_gemv_k_split_all_variants_twice(ctx, fmt):
    """K = 18944 (the 7B down projection's K) with few rows: the launch splits
    K into 4096-element chunks whose partial sums meet in the workspace.  Each
    variant runs twice (the arrival counters must be reset by the first)."""
    n, k = 200, 18944
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=91)
    for var in VARIANTS[fmt]:
        for rep in range(2):
            run_variant(ctx, fmt, var, wbuf, raw, n, k, seed=5 + rep)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0"])
def test_gemv_k_split_output_aliases_residual(ctx, fmt):
    n, k = 300, 12288
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=92)
    rng = np.random.default_rng(8)
    x = rng.standard_normal(k).astype(np.float32)
    y0 = rng.standard_normal(n).astype(np.float32)
    yb = ctx.buffer_from(y0)
    getattr(d, f"gemv_{fmt}_add_f32_f32in")(ctx, wbuf, ctx.buffer_from(x), yb, yb, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(yb.read(np.float32, n), yref + y0, sabs, f"{fmt} split aliased")


def test_fused_k_split_ffn_and_qkv(ctx):
    from test_gpu_fused import ffn_check
    ff, k = 150, 18944
    wg, rg = device_weights(ctx, "q4_0", ff, k, seed=93)
    wu, ru = device_weights(ctx, "q4_0", ff, k, seed=94)
    x = np.random.default_rng(9).standard_normal(k).astype(np.float32)
    act = ctx.new_buffer(4 * ff)
    d.fused_ffn_q4_0_f32(ctx, wg, wu, ctx.buffer_from(x), act, ff, k)
    ctx.flush()
    gr, gs = ora.gemv("q4_0", rg, x, ff, k)
    ur, us = ora.gemv("q4_0", ru, x, ff, k)
    ffn_check(act.read(np.float32, ff), gr, gs, ur, us, "split ffn q4_0")
    qd, kd = 64, 32
    ws = [device_weights(ctx, "q8_0", n, k, seed=95 + i) for i, n in enumerate((qd, kd, kd))]
    bias = [np.random.default_rng(10 + i).standard_normal(n).astype(np.float16) for i, n in
            enumerate((qd, kd, kd))]
    outs = [ctx.new_buffer(4 * n) for n in (qd, kd, kd)]
    d.fused_qkv_bias_q8_0_f32(ctx, ws[0][0], ws[1][0], ws[2][0], ctx.buffer_from(x), *outs,
                              *[ctx.buffer_from(b) for b in bias], qd, kd, k)
    ctx.flush()
    for i, n in enumerate((qd, kd, kd)):
        y, s = ora.gemv("q8_0", ws[i][1], x, n, k)
        check_close(outs[i].read(np.float32, n), y + bias[i].astype(np.float64), s, f"split qkv {i}")


def test_norm_then_gemv_long_k(ctx):
    """RMSNorm into the workspace, then a K-split GEMV (partials kept apart)."""
    n, k = 120, 16384
    rng = np.random.default_rng(11)
    x = (2 * rng.standard_normal(k)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(k)).astype(np.float32)
    xn = ora.rms_norm(x, g, 1e-6).astype(np.float32)
    wbuf, raw = device_weights(ctx, "q8_0", n, k, seed=96)
    y = ctx.new_buffer(4 * n)
    d.rms_norm_gemv_q8_0_f32in_f32out(ctx, wbuf, ctx.buffer_from(x), ctx.buffer_from(g), 1e-6, y,
                                      n, k)
    ctx.flush()
    yref, sabs = ora.gemv("q8_0", raw, xn, n, k)
    check_close(y.read(np.float32, n), yref, sabs, "norm then split gemv", F32_EPS * np.abs(yref))


def test_long_k_prepass_path_without_split():
    """The pre-pass + whole-K path (RUNIT_GEMV_KSPLIT=0) stays correct."""
    import os
    os.environ["RUNIT_GEMV_KSPLIT"] = "0"
    try:
        c2 = d.HipContext()
    finally:
        del os.environ["RUNIT_GEMV_KSPLIT"]
    try:
        for fmt in FMTS:
            wbuf, raw = device_weights(c2, fmt, 96, 18944, seed=97)
            run_variant(c2, fmt, "f32in_f32out", wbuf, raw, 96, 18944, seed=12)
    finally:
        c2.close()


def limb_error_bound(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Worst-case error per row of the activation limb form: every element
    of a 32-element block is held to 2^(E−22), E the block maximum's frexp
    exponent (max|x_b| < 2^E), so |x_i − x̂_i| ≤ 2^(E−23) and
        |Σ w_i x_i − Σ w_i x̂_i| ≤ Σ_b 2^(E_b−23)·Σ_{i∈b} |w_i|."""
    xb = np.abs(x.astype(np.float64)).reshape(-1, 32).max(axis=1)
    E = np.frexp(xb)[1]                      # xb = m·2^E, 0.5 ≤ m < 1
    step = np.where(xb > 0, np.ldexp(1.0, E - 23), 0.0)
    return (np.abs(W).reshape(W.shape[0], -1, 32).sum(axis=2) * step).sum(axis=1)


@pytest.mark.parametrize("n", [4608, 18944])
def test_gemv_limb_range_outliers_on_zero_codes(ctx, n):
    """The activation limb form at a large in-block dynamic range: every
    32-element block of x holds a ±2^12 outlier on a column whose Q4_0 code
    is 8 (weight exactly 0) in every row, the rest N(0, 1), at K = 3584 (the
    7B Q/K/V launch shape, matrix-core body, and the 7B gate/up row count,
    LDS-streamed body).  The reference multiplies full f32 per element
    (gemv_q4_0.metal:26-49); here the other 31 elements of each block are
    held to 2^(13−22) = 2^-9, so the worst-case limb error per row is
    ~1.2e-3·Σ|w·x| — past the range where 1e-4·Σ|w·x| is guaranteed (the
    ratio Σ_b 2^(E_b−23)·Σ_b|w| / Σ|w·x| ≤ 1e-4 − 64·2^-24).  The errors are
    roundings to nearest, centred and independent, so the row error is
    ~√K·rms(w)·2^-10/√3 ≈ 7e-4 (rms), and the largest of 18,944 rows reaches
    ~0.6 of the 1e-4·Σ|w·x| bound (host simulation of the rounding).  Checked: the BASELINE
    tolerance on every row, and the deterministic limb bound (plus f32
    combination) on every row."""
    k = 3584
    wbuf, raw = device_weights(ctx, "q4_0", n, k, seed=31)
    blk = raw.reshape(n, k // 32, 18).copy()
    blk[:, :, 2] = (blk[:, :, 2] & 0xF0) | 0x08  # element 0 of every block: code 8 → w = 0
    raw = blk.reshape(-1)
    wbuf.write(raw)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(k).astype(np.float32)
    x[0::32] = np.where(rng.random(k // 32) < 0.5, -4096.0, 4096.0).astype(np.float32)
    yref, sabs = ora.gemv("q4_0", raw, x, n, k)
    y = ctx.new_buffer(4 * n)
    d.gemv_q4_0_f32in_f32out(ctx, wbuf, ctx.buffer_from(x), y, n, k)
    ctx.flush()
    got = y.read(np.float32, n)
    W = ora.dequant("q4_0", raw).reshape(n, k).astype(np.float64)
    assert np.all(W[:, 0::32] == 0.0)
    lb = limb_error_bound(W, x)
    assert np.all(lb > 1e-4 * sabs)  # the case is outside the guaranteed range
    err = np.abs(got.astype(np.float64) - yref)
    assert np.all(err <= lb + 64 * F32_EPS * sabs), (err / lb).max()
    check_close(got, yref, sabs, "x outliers 2^12 on zero codes")


def test_gemv_limb_range_standard_inputs_guaranteed(ctx):
    """For the BASELINE inputs (N(0, 0.02) weights, N(0, 1) activations) the
    worst-case limb error of every row is far inside 1e-4·Σ|w·x| (at most
    1/180 of it for this seed): the tolerance is guaranteed there, not only observed."""
    n, k = 4864, 896
    wbuf, raw = device_weights(ctx, "q8_0", n, k, seed=21)
    x = np.random.default_rng(6).standard_normal(k).astype(np.float32)
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    W = ora.dequant("q8_0", raw).reshape(n, k).astype(np.float64)
    lb = limb_error_bound(W, x)
    assert np.all(lb + 64 * F32_EPS * sabs <= 1e-4 * sabs)
    y = ctx.new_buffer(4 * n)
    d.gemv_q8_0_f32in_f32out(ctx, wbuf, ctx.buffer_from(x), y, n, k)
    ctx.flush()
    err = np.abs(y.read(np.float32, n).astype(np.float64) - yref)
    assert np.all(err <= lb + 64 * F32_EPS * sabs)
