"""GPU parity of fused QKV(+bias), fused gate+up+SiLU, argmax and the batched
Q8_0 GEMM, against the CPU oracle, through the C ABI."""
import numpy as np
import pytest

import oracle_lib as ora
from gpu_helpers import F32_EPS, REL, check_close, device_weights
from runit_mac_amd import dispatch as d

pytestmark = pytest.mark.gpu


def _qkv_case(ctx, fmt, q_dim, kv_dim, k, bias, seed):
    rng = np.random.default_rng(seed)
    ws = [device_weights(ctx, fmt, n, k, seed=seed + i) for i, n in
          enumerate((q_dim, kv_dim, kv_dim))]
    x = rng.standard_normal(k).astype(np.float32)
    xb = ctx.buffer_from(x)
    outs = [ctx.new_buffer(4 * n) for n in (q_dim, kv_dim, kv_dim)]
    biases = [(0.02 * rng.standard_normal(n)).astype(np.float16) for n in (q_dim, kv_dim, kv_dim)]
    if bias:
        fn = getattr(d, f"fused_qkv_bias_{fmt}_f32")
        fn(ctx, ws[0][0], ws[1][0], ws[2][0], xb, *outs, *[ctx.buffer_from(b) for b in biases],
           q_dim, kv_dim, k)
    else:
        d.fused_qkv_q8_0_f32(ctx, ws[0][0], ws[1][0], ws[2][0], xb, *outs, q_dim, kv_dim, k)
    ctx.flush()
    for i, n in enumerate((q_dim, kv_dim, kv_dim)):
        yref, sabs = ora.gemv(fmt, ws[i][1], x, n, k)
        if bias:
            yref = yref + biases[i].astype(np.float64)  # fused_qkv.metal:68
        check_close(outs[i].read(np.float32, n), yref, sabs, f"qkv[{i}] {fmt}",
                    F32_EPS * np.abs(yref))


@pytest.mark.parametrize("q_dim,kv_dim,k", [(896, 128, 896), (256, 64, 512), (100, 20, 256)])
def test_fused_qkv_bias_q8_0(ctx, q_dim, kv_dim, k):
    _qkv_case(ctx, "q8_0", q_dim, kv_dim, k, True, seed=q_dim)


def test_fused_qkv_no_bias_q8_0(ctx):
    _qkv_case(ctx, "q8_0", 896, 128, 896, False, seed=3)


@pytest.mark.parametrize("q_dim,kv_dim,k", [(3584, 512, 3584), (256, 64, 512)])
def test_fused_qkv_bias_q4_0(ctx, q_dim, kv_dim, k):
    _qkv_case(ctx, "q4_0", q_dim, kv_dim, k, True, seed=q_dim + 1)


@pytest.mark.parametrize("fmt,q_dim,kv_dim,k", [("q5_0", 3584, 512, 3584), ("q5_0", 100, 20, 96),
                                              ("q5k", 896, 128, 1024), ("q5k", 256, 64, 512)])
def test_fused_qkv_bias_q5(ctx, fmt, q_dim, kv_dim, k):
    _qkv_case(ctx, fmt, q_dim, kv_dim, k, True, seed=q_dim + 7)


def _qkv_mixed_case(ctx, fq, fv, q_dim, kv_dim, k, bias, seed):
    """Q and K in format fq, V in fv, one launch; biases all given or all None."""
    rng = np.random.default_rng(seed)
    fmts = (fq, fq, fv)
    ws = [device_weights(ctx, f, n, k, seed=seed + i) for i, (f, n) in
          enumerate(zip(fmts, (q_dim, kv_dim, kv_dim)))]
    x = rng.standard_normal(k).astype(np.float32)
    outs = [ctx.new_buffer(4 * n) for n in (q_dim, kv_dim, kv_dim)]
    biases = [(0.02 * rng.standard_normal(n)).astype(np.float16) for n in (q_dim, kv_dim, kv_dim)]
    bb = [ctx.buffer_from(b) for b in biases] if bias else [None] * 3
    name = f"fused_qkv_bias_{fq}_f32" if fq == fv else f"fused_qkv_bias_{fq}_{fv}_f32"
    getattr(d, name)(ctx, ws[0][0], ws[1][0], ws[2][0], ctx.buffer_from(x), *outs, *bb,
                     q_dim, kv_dim, k)
    ctx.flush()
    for i, n in enumerate((q_dim, kv_dim, kv_dim)):
        yref, sabs = ora.gemv(fmts[i], ws[i][1], x, n, k)
        if bias:
            yref = yref + biases[i].astype(np.float64)  # add_f16_into_f32 after each GEMV
        check_close(outs[i].read(np.float32, n), yref, sabs, f"qkv[{i}] {fmts[i]}",
                    F32_EPS * np.abs(yref))


@pytest.mark.parametrize("fq,fv,q_dim,kv_dim,k,bias", [
    ("q4k", "q6k", 3584, 512, 3584, True),    # config 4 (7B Q4_K_M mix)
    ("q4k", "q6k", 3584, 512, 3584, False),
    ("q4k", "q6k", 896, 128, 1024, True),
    ("q4k", "q6k", 100, 20, 256, True),       # ragged: tiles past the last row
    ("q4k", "q6k", 256, 64, 9216, True),      # K past one staging pass: x converted once
    ("q4k", "q6k", 4, 4, 256, True),          # one row quad per part
    ("q4kg", "q6kg", 3584, 512, 3584, True),
    ("q4kg", "q6kg", 256, 64, 512, False),
    ("q4k", "q4k", 3584, 512, 3584, True),
    ("q4k", "q4k", 256, 64, 512, False),
    ("q4kg", "q4kg", 896, 128, 1024, True),
])
def test_fused_qkv_q4k_mix(ctx, fq, fv, q_dim, kv_dim, k, bias):
    _qkv_mixed_case(ctx, fq, fv, q_dim, kv_dim, k, bias, seed=q_dim + kv_dim + k)


def test_fused_qkv_q4k_mix_partial_bias_rejected(ctx):
    ws = [device_weights(ctx, f, n, 256, seed=i)[0] for i, (f, n) in
          enumerate((("q4k", 32), ("q4k", 16), ("q6k", 16)))]
    x = ctx.buffer_from(np.ones(256, np.float32))
    outs = [ctx.new_buffer(4 * n) for n in (32, 16, 16)]
    b = ctx.buffer_from(np.zeros(32, np.float16))
    with pytest.raises(Exception, match="biases"):
        d.fused_qkv_bias_q4k_q6k_f32(ctx, *ws, x, *outs, b, None, None, 32, 16, 256)


def ffn_check(got, gate_ref, gate_s, up_ref, up_s, what):
    """act = silu(g)·u with |g−g_ref| ≤ eg, |u−u_ref| ≤ eu: |silu'| ≤ 1.1 gives
    |Δact| ≤ 1.1·eg·(|u|+eu) + (|silu(g)|+1.1·eg)·eu, plus f32 epilogue rounding."""
    eg, eu = REL * gate_s, REL * up_s
    sil = np.array([ora.silu(g) for g in gate_ref])
    ref = sil * up_ref
    tol = 1.1 * eg * (np.abs(up_ref) + eu) + (np.abs(sil) + 1.1 * eg) * eu + 4 * F32_EPS * np.abs(ref)
    err = np.abs(got.astype(np.float64) - ref)
    bad = ~(err <= tol)
    assert not bad.any(), f"{what}: {int(bad.sum())} outside; worst {err[bad].max():.3e}"


@pytest.mark.parametrize("fmt,ff,k", [("q8_0", 4864, 896), ("q8_0", 300, 512),
                                      ("q4_0", 1000, 3584), ("q4_0", 77, 256),
                                      ("q4k", 1000, 3584), ("q4k", 33, 512),
                                      ("q5_0", 1000, 3584), ("q5_0", 45, 160),
                                      ("q5k", 1000, 3584), ("q5k", 33, 512),
                                      ("q4_0g", 1000, 3584), ("q4_0g", 45, 160),
                                      ("q4kg", 1000, 3584), ("q5kg", 300, 1024)])
def test_fused_ffn(ctx, fmt, ff, k):
    wg, rg = device_weights(ctx, fmt, ff, k, seed=ff + 1)
    wu, ru = device_weights(ctx, fmt, ff, k, seed=ff + 2)
    x = np.random.default_rng(ff).standard_normal(k).astype(np.float32)
    act = ctx.new_buffer(4 * ff)
    getattr(d, f"fused_ffn_{fmt}_f32")(ctx, wg, wu, ctx.buffer_from(x), act, ff, k)
    ctx.flush()
    g, gs = ora.gemv(fmt, rg, x, ff, k)
    u, us = ora.gemv(fmt, ru, x, ff, k)
    ffn_check(act.read(np.float32, ff), g, gs, u, us, f"ffn {fmt} {ff}x{k}")


# ───────────────────────── argmax ─────────────────────────

@pytest.mark.parametrize("n", [1, 5, 1000, 1024, 1025, 151936, 152064])
def test_argmax_random(ctx, n):
    v = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    res = ctx.new_buffer(4)
    d.argmax_f32(ctx, ctx.buffer_from(v), res, n)
    ctx.flush()
    assert int(res.read(np.uint32, 1)[0]) == ora.argmax(v)


def test_argmax_ties_and_nan_follow_rust_max_by(ctx):
    nan = np.float32("nan")
    rng = np.random.default_rng(0)
    cases = [np.zeros(5000, np.float32), np.full(3000, -np.inf, np.float32)]
    v = rng.standard_normal(70000).astype(np.float32)
    v[[10, 5000, 69000]] = 9.0
    cases.append(v)
    for pos in (0, 17, 40000, 69999):
        w = rng.standard_normal(70000).astype(np.float32)
        w[pos] = nan
        cases.append(w)
    w = rng.standard_normal(50000).astype(np.float32)
    w[[5, 30000]] = nan
    w[20000] = 50.0
    w[45000] = 7.0
    cases.append(w)
    res = ctx.new_buffer(4)
    for c in cases:
        d.argmax_f32(ctx, ctx.buffer_from(c), res, c.size)
        ctx.flush()
        assert int(res.read(np.uint32, 1)[0]) == ora.argmax(c)


def test_argmax_nan_ranges_at_vocab_size(ctx):
    """NaNs in several workgroup ranges, the maximum before, inside and after
    the range holding the last NaN, and ties across ranges (later wins)."""
    rng = np.random.default_rng(11)
    n = 151936
    res = ctx.new_buffer(4)
    for case in range(24):
        v = rng.standard_normal(n).astype(np.float32)
        k = int(rng.integers(0, 4))
        if k:
            v[rng.integers(0, n, size=k)] = np.float32("nan")
        for pos in rng.integers(0, n, size=int(rng.integers(1, 4))):
            v[pos] = 6.0  # equal maxima, possibly on both sides of a NaN
        if case == 0:
            v[-1] = np.float32("nan")
        d.argmax_f32(ctx, ctx.buffer_from(v), res, n)
        ctx.flush()
        assert int(res.read(np.uint32, 1)[0]) == ora.argmax(v), case


def test_argmax_f16(ctx):
    v = np.random.default_rng(9).standard_normal(151936).astype(np.float16)
    res = ctx.new_buffer(4)
    d.argmax_f16(ctx, ctx.buffer_from(v), res, v.size)
    ctx.flush()
    assert int(res.read(np.uint32, 1)[0]) == ora.argmax(v.astype(np.float32))


# ───────────────────────── batched Q8_0 GEMM ─────────────────────────

@pytest.mark.parametrize("m", [1, 2, 4, 5, 8, 13, 16, 32, 37])
@pytest.mark.parametrize("n,k", [(512, 1024), (130, 3584), (33, 96), (1100, 32), (70, 8192)])
def test_gemm_q8_0(ctx, m, n, k):
    wbuf, raw = device_weights(ctx, "q8_0", n, k, seed=m + n)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    y = ctx.new_buffer(4 * m * n)
    d.gemm_q8_0_f32(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm m={m}")
    # a second call reuses the workspace; a smaller batch must not read stale rows
    if m > 2:
        y2 = ctx.new_buffer(4 * 2 * n)
        d.gemm_q8_0_f32(ctx, wbuf, ctx.buffer_from(x[:2]), y2, 2, n, k)
        ctx.flush()
        check_close(y2.read(np.float32, 2 * n), yref[:2].ravel(), sabs[:2].ravel(), "gemm m=2")


@pytest.mark.parametrize("m", [12, 32])
def test_gemm_f16_form_long_rows(ctx, m):
    """Rows longer than 20,480 elements: the f16 form's activations are
    prepared by the multi-workgroup pass (record ranges, every workgroup
    reducing its row's maximum), the K range split over workgroups and the
    splits summed by their own launch."""
    n, k = 96, 24576
    wbuf, raw = device_weights(ctx, "q8_0", n, k, seed=m + 91)
    x = np.random.default_rng(m + 92).standard_normal((m, k)).astype(np.float32)
    x[:, ::997] *= 50.0  # a wider range inside each row
    y = ctx.new_buffer(4 * m * n)
    d.gemm_q8_0_f32(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm long rows m={m}")


@pytest.mark.parametrize("fmt", ["q4_0", "q4k"])
@pytest.mark.parametrize("m", [2, 4, 7, 16, 32, 37])
@pytest.mark.parametrize("n,k", [(512, 1024), (130, 3584), (70, 8192)])
def test_gemm_4bit(ctx, fmt, m, n, k):
    """Batched GEMM on reference-layout Q4_0 / Q4_K weights: every output row
    within the GEMV bound of the per-row oracle."""
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=m + n + 5)
    x = np.random.default_rng(m + 1).standard_normal((m, k)).astype(np.float32)
    y = ctx.new_buffer(4 * m * n)
    getattr(d, f"gemm_{fmt}_f32")(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm {fmt} m={m}")


@pytest.mark.parametrize("m", [3, 9])
def test_gemm_q4_0_unaligned_rows_fall_back_to_gemvs(ctx, m):
    # k = 96: 3 blocks per row (54 bytes) — not a whole stage, so one GEMV per row
    n, k = 77, 96
    wbuf, raw = device_weights(ctx, "q4_0", n, k, seed=m)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    y = ctx.new_buffer(4 * m * n)
    d.gemm_q4_0_f32(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv("q4_0", raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm fallback m={m}")


def test_gemm_q4k_rejects_k_not_multiple_of_256(ctx):
    w = ctx.new_buffer(4096)
    with pytest.raises(d.Dispatch):
        d.gemm_q4k_f32(ctx, w, ctx.new_buffer(4096), ctx.new_buffer(4096), 2, 4, 128)


def test_gemm_q8_0_direct_kernel_matches_staged(ctx):
    """The unstaged kernel (any K) on a shape the staged kernel also takes."""
    import os
    n, k, m = 300, 2048, 12
    wbuf, raw = device_weights(ctx, "q8_0", n, k, seed=5)
    x = np.random.default_rng(9).standard_normal((m, k)).astype(np.float32)
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    os.environ["RUNIT_GEMM_DIRECT"] = "1"
    try:
        c2 = d.HipContext()
    finally:
        del os.environ["RUNIT_GEMM_DIRECT"]
    try:
        w2 = c2.buffer_from(raw)
        y = c2.new_buffer(4 * m * n)
        d.gemm_q8_0_f32(c2, w2, c2.buffer_from(x), y, m, n, k)
        c2.flush()
        check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), "gemm direct")
    finally:
        c2.close()


@pytest.mark.parametrize("fmt", ["q8_0", "q4k", "q6kg"])
@pytest.mark.parametrize("m", [16, 32])
def test_gemm_int8_form_matches_oracle(fmt, m):
    """The int8 limb form of the staged GEMM, which batches above 8 rows take
    only with RUNIT_GEMM_F16=0 (they take the f16 form by default)."""
    import os
    n, k = 130, 3584
    os.environ["RUNIT_GEMM_F16"] = "0"
    try:
        c2 = d.HipContext()
    finally:
        del os.environ["RUNIT_GEMM_F16"]
    try:
        wbuf, raw = device_weights(c2, fmt, n, k, seed=m + 40)
        x = np.random.default_rng(m + 41).standard_normal((m, k)).astype(np.float32)
        y = c2.new_buffer(4 * m * n)
        getattr(d, f"gemm_{fmt}_f32")(c2, wbuf, c2.buffer_from(x), y, m, n, k)
        c2.flush()
        yref, sabs = ora.gemv(fmt, raw, x, n, k)
        check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm int8 {fmt} m={m}")
    finally:
        c2.close()


@pytest.mark.parametrize("fmt", ["q8_0", "q4k", "q4_0", "q6k", "q6kg"])
def test_gemm_f16_form_wide_range(ctx, fmt):
    """f16 forms: each activation row is scaled into f16's range on its own
    (hi/lo pairs carry ~22 bits of every element down to 2^-24 of the row's
    scale), so rows of 1e-6-sized activations, rows of 1e4-sized ones and rows
    of 1e-3-sized values with an outlier of 3e3 in every record (a range of
    ~1e7 inside the row) all stay within the bound."""
    n, k, m = 200, 1024, 24
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=77)
    rng = np.random.default_rng(78)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0:8] *= 1e-6
    x[8:16] *= 1e4
    x[16:24] *= 1e-3
    x[16:24, ::32] = 3e3  # one outlier per record
    y = ctx.new_buffer(4 * m * n)
    getattr(d, f"gemm_{fmt}_f32")(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm f16 range {fmt}")


GEMM_MORE = ["q5_0", "q5k", "q6k", "q4_0g", "q4kg", "q5kg", "q6kg"]


@pytest.mark.parametrize("fmt", GEMM_MORE)
@pytest.mark.parametrize("m", [2, 5, 16, 32, 37])
@pytest.mark.parametrize("n,k", [(512, 1024), (130, 3584), (70, 8192)])
def test_gemm_more_formats(ctx, fmt, m, n, k):
    """Batched GEMM on the Q5_0 / Q5_K / Q6_K and ggml-layout weights: every
    output row within the GEMV bound of the per-row oracle; a second, smaller
    batch reuses the workspace."""
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=m + n + 11)
    x = np.random.default_rng(m + 3).standard_normal((m, k)).astype(np.float32)
    y = ctx.new_buffer(4 * m * n)
    getattr(d, f"gemm_{fmt}_f32")(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm {fmt} m={m}")
    if m > 2:
        y2 = ctx.new_buffer(4 * 2 * n)
        getattr(d, f"gemm_{fmt}_f32")(ctx, wbuf, ctx.buffer_from(x[:2]), y2, 2, n, k)
        ctx.flush()
        check_close(y2.read(np.float32, 2 * n), yref[:2].ravel(), sabs[:2].ravel(),
                    f"gemm {fmt} m=2 after m={m}")


@pytest.mark.parametrize("fmt", ["q8_0", "q4k", "q5k"])
@pytest.mark.parametrize("m", [32, 27])
def test_gemm_256_row_tiles_partial_last_tile(ctx, fmt, m):
    # n = 16500 rows: enough 256-row tiles (≥ a quarter of the CUs) for the
    # 16-wave form at 32 rows, the last tile 116 rows short; m = 27 pads the
    # activation rows of the last 8-row group
    n, k = 16500, 512
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=m + 31)
    x = np.random.default_rng(m + 32).standard_normal((m, k)).astype(np.float32)
    y = ctx.new_buffer(4 * m * n)
    getattr(d, f"gemm_{fmt}_f32")(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm {fmt} {m}x{n}x{k}")


@pytest.mark.parametrize("fmt", ["q6k", "q6kg"])
def test_gemm_q6k_odd_block_count_falls_back_to_gemvs(ctx, fmt):
    # k = 3840: 15 super-blocks per row, not a whole number of two-block stages
    n, k, m = 66, 3840, 6
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=21)
    x = np.random.default_rng(22).standard_normal((m, k)).astype(np.float32)
    y = ctx.new_buffer(4 * m * n)
    getattr(d, f"gemm_{fmt}_f32")(ctx, wbuf, ctx.buffer_from(x), y, m, n, k)
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm {fmt} fallback")
