"""GPU parity of the LDS-streamed GEMV body (rt_gemv_ls.h) against the CPU
oracle, through the C ABI.

The library takes that body only for launches with at least 16 items (row
quads × K chunks) per CU; a second context created with RUNIT_GEMV_LS_MIN=0
takes it for every shape it can serve, so the cases below cover its edges at small sizes: row counts that are
not a multiple of 4, a weight base that is not 16-byte aligned, an output that
aliases the residual, fused QKV (+bias) and gate+up+SiLU row mappings, a
K split into chunks (rows longer than 3 KB), and a launch with more items per
wave than one result group.  Tolerance as in gpu_helpers (BASELINE's
|y − y_ref| ≤ 1e-4·Σ|w_i·x_i|).
"""
import os

import numpy as np
import pytest

import oracle_lib as ora
from gpu_helpers import F32_EPS, check_close, device_weights, f16_extra, f16_to_f64
from runit_mac_amd import dispatch as d
from test_gpu_fused import ffn_check

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lsctx():
    old = os.environ.get("RUNIT_GEMV_LS_MIN")
    os.environ["RUNIT_GEMV_LS_MIN"] = "0"
    try:
        c = d.HipContext()
    finally:
        if old is None:
            del os.environ["RUNIT_GEMV_LS_MIN"]
        else:
            os.environ["RUNIT_GEMV_LS_MIN"] = old
    yield c
    c.close()


def _weights_at(ctx, fmt, n, k, seed, offset):
    """Weights generated on the device, then placed `offset` bytes into a
    fresh buffer (offset 0: the generated buffer itself)."""
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=seed)
    if offset == 0:
        return wbuf.ptr, raw, [wbuf]
    buf = ctx.new_buffer(raw.nbytes + 64)
    buf.write(raw, offset)
    return buf.ptr + offset, raw, [wbuf, buf]


LS_FMTS = ["q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg", "q5kg", "q6kg"]
KQUANTS = ("q4k", "q6k", "q5k", "q4kg", "q5kg", "q6kg")


@pytest.mark.parametrize("fmt", LS_FMTS)
@pytest.mark.parametrize("n,k,offset", [(37, 512, 0), (300, 3584, 2), (1027, 896, 0),
                                        (5, 1024, 4), (2053, 256, 8)])
def test_ls_gemv_plain_and_residual(lsctx, fmt, n, k, offset):
    if fmt in KQUANTS and k % 256:
        pytest.skip("K-quants need K % 256 == 0")
    if fmt in ("q8_0", "q4_0", "q5_0", "q4_0g") and (k // 32) % 2:
        pytest.skip("odd block count: single-block kernels")
    w, raw, keep = _weights_at(lsctx, fmt, n, k, seed=n + k, offset=offset)
    rng = np.random.default_rng(n * 7 + k)
    x = rng.standard_normal(k).astype(np.float32)
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    xb = lsctx.buffer_from(x)
    y = lsctx.new_buffer(4 * n)
    getattr(d, f"gemv_{fmt}_f32in_f32out")(lsctx, w, xb, y, n, k)
    # residual aliasing the output (forward.rs:1619,1702)
    res = rng.standard_normal(n).astype(np.float32)
    yr = lsctx.buffer_from(res)
    getattr(d, f"gemv_{fmt}_add_f32_f32in")(lsctx, w, xb, yr, yr, n, k)
    lsctx.flush()
    check_close(y.read(np.float32, n), yref, sabs, f"ls {fmt} {n}x{k}+{offset}",
                F32_EPS * np.abs(yref))
    ref = yref + res
    check_close(yr.read(np.float32, n), ref, sabs, f"ls add {fmt} {n}x{k}+{offset}",
                F32_EPS * np.abs(ref))
    del keep


def test_ls_gemv_f16_out_q8_0(lsctx):
    n, k = 4099, 896
    w, raw, keep = _weights_at(lsctx, "q8_0", n, k, seed=3, offset=2)
    x = np.random.default_rng(3).standard_normal(k).astype(np.float32)
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    y = lsctx.new_buffer(2 * n)
    d.gemv_q8_0_f32in(lsctx, w, lsctx.buffer_from(x), y, n, k)
    lsctx.flush()
    check_close(f16_to_f64(y.read(np.uint16, n)), yref, sabs, "ls q8_0 f16 out",
                f16_extra(yref, sabs))
    del keep


def test_ls_gemv_q6kg(lsctx):
    n, k = 999, 3584
    wbuf, raw = device_weights(lsctx, "q6kg", n, k, seed=21)
    x = np.random.default_rng(21).standard_normal(k).astype(np.float32)
    yref, sabs = ora.gemv("q6kg", raw, x, n, k)
    y = lsctx.new_buffer(4 * n)
    d.gemv_q6kg_f32in_f32out(lsctx, wbuf, lsctx.buffer_from(x), y, n, k)
    lsctx.flush()
    check_close(y.read(np.float32, n), yref, sabs, "ls q6kg", F32_EPS * np.abs(yref))


@pytest.mark.parametrize("fmt,n,k", [("q4_0", 96, 18944), ("q6k", 70, 18944),
                                     ("q8_0", 130, 8192), ("q4k", 33, 16384),
                                     ("q5k", 41, 18944), ("q5_0", 37, 9216),
                                     ("q4kg", 29, 18944), ("q6kg", 22, 18944),
                                     ("q4_0g", 31, 18944), ("q5kg", 19, 18944)])
def test_ls_gemv_k_split(lsctx, fmt, n, k):
    # rows longer than 3 KB: K chunks whose partial sums meet in the workspace
    wbuf, raw = device_weights(lsctx, fmt, n, k, seed=n)
    rng = np.random.default_rng(n)
    x = rng.standard_normal(k).astype(np.float32)
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    xb = lsctx.buffer_from(x)
    res = rng.standard_normal(n).astype(np.float32)
    for rep in range(2):  # twice: the arrival counters must be reset by the first call
        y = lsctx.new_buffer(4 * n)
        getattr(d, f"gemv_{fmt}_f32in_f32out")(lsctx, wbuf, xb, y, n, k)
        yr = lsctx.buffer_from(res)
        getattr(d, f"gemv_{fmt}_add_f32_f32in")(lsctx, wbuf, xb, yr, yr, n, k)
        lsctx.flush()
        check_close(y.read(np.float32, n), yref, sabs, f"ls split {fmt} rep {rep}",
                    F32_EPS * np.abs(yref))
        ref = yref + res
        check_close(yr.read(np.float32, n), ref, sabs, f"ls split add {fmt} rep {rep}",
                    F32_EPS * np.abs(ref))


@pytest.mark.parametrize("fmt,ff,k", [("q8_0", 4864, 896), ("q8_0", 301, 512),
                                      ("q4_0", 1000, 3584), ("q4k", 77, 512),
                                      ("q4_0", 129, 18944), ("q5_0", 1000, 3584),
                                      ("q5k", 333, 3584), ("q4_0g", 257, 3584),
                                      ("q4kg", 1000, 3584), ("q5kg", 65, 1024)])
def test_ls_fused_ffn(lsctx, fmt, ff, k):
    wg, rg = device_weights(lsctx, fmt, ff, k, seed=ff + 1)
    wu, ru = device_weights(lsctx, fmt, ff, k, seed=ff + 2)
    x = np.random.default_rng(ff).standard_normal(k).astype(np.float32)
    act = lsctx.new_buffer(4 * ff)
    getattr(d, f"fused_ffn_{fmt}_f32")(lsctx, wg, wu, lsctx.buffer_from(x), act, ff, k)
    lsctx.flush()
    g, gs = ora.gemv(fmt, rg, x, ff, k)
    u, us = ora.gemv(fmt, ru, x, ff, k)
    ffn_check(act.read(np.float32, ff), g, gs, u, us, f"ls ffn {fmt} {ff}x{k}")


@pytest.mark.parametrize("fmt,q_dim,kv_dim,k", [("q8_0", 896, 128, 896), ("q8_0", 102, 22, 256),
                                              ("q4_0", 3584, 512, 3584)])
def test_ls_fused_qkv_bias(lsctx, fmt, q_dim, kv_dim, k):
    rng = np.random.default_rng(q_dim)
    dims = (q_dim, kv_dim, kv_dim)
    ws = [device_weights(lsctx, fmt, n, k, seed=q_dim + i) for i, n in enumerate(dims)]
    x = rng.standard_normal(k).astype(np.float32)
    outs = [lsctx.new_buffer(4 * n) for n in dims]
    biases = [(0.02 * rng.standard_normal(n)).astype(np.float16) for n in dims]
    getattr(d, f"fused_qkv_bias_{fmt}_f32")(lsctx, ws[0][0], ws[1][0], ws[2][0],
                                            lsctx.buffer_from(x), *outs,
                                            *[lsctx.buffer_from(b) for b in biases],
                                            q_dim, kv_dim, k)
    lsctx.flush()
    for i, n in enumerate(dims):
        yref, sabs = ora.gemv(fmt, ws[i][1], x, n, k)
        yref = yref + biases[i].astype(np.float64)
        check_close(outs[i].read(np.float32, n), yref, sabs, f"ls qkv[{i}] {fmt}",
                    F32_EPS * np.abs(yref))


def test_ls_default_context_vocab_sized(ctx):
    # the default context takes the body at vocabulary-sized N
    n, k = 65537, 1024
    wbuf, raw = device_weights(ctx, "q8_0", n, k, seed=99)
    x = np.random.default_rng(99).standard_normal(k).astype(np.float32)
    yref, sabs = ora.gemv("q8_0", raw, x, n, k)
    y = ctx.new_buffer(4 * n)
    d.gemv_q8_0_f32in_f32out(ctx, wbuf, ctx.buffer_from(x), y, n, k)
    ctx.flush()
    check_close(y.read(np.float32, n), yref, sabs, "vocab-sized q8_0", F32_EPS * np.abs(yref))


@pytest.mark.parametrize("fmt,n,k", [("q8_0", 896, 4864), ("q8_0", 37, 6144), ("q4_0", 301, 4864),
                                     ("q4k", 130, 4608), ("q5k", 77, 8192), ("q4kg", 66, 4608),
                                     ("q5kg", 9, 5120), ("q4_0g", 129, 4864), ("q5_0", 64, 4864)])
def test_lsk_workgroup_k_split(ctx, fmt, n, k):
    # rows longer than the LDS slot with the whole K's records ≤ 32 KB (the
    # 0.5B down projection's shape): every K chunk of a row quad in one
    # workgroup, partial sums added in LDS in chunk order
    w, raw, keep = _weights_at(ctx, fmt, n, k, seed=n + 5, offset=2 if fmt == "q8_0" else 0)
    rng = np.random.default_rng(n + k)
    x = rng.standard_normal(k).astype(np.float32)
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    xb = ctx.buffer_from(x)
    res = rng.standard_normal(n).astype(np.float32)
    for rep in range(2):
        y = ctx.new_buffer(4 * n)
        getattr(d, f"gemv_{fmt}_f32in_f32out")(ctx, w, xb, y, n, k)
        yr = ctx.buffer_from(res)
        getattr(d, f"gemv_{fmt}_add_f32_f32in")(ctx, w, xb, yr, yr, n, k)
        ctx.flush()
        check_close(y.read(np.float32, n), yref, sabs, f"lsk {fmt} {n}x{k} rep {rep}",
                    F32_EPS * np.abs(yref))
        ref = yref + res
        check_close(yr.read(np.float32, n), ref, sabs, f"lsk add {fmt} {n}x{k} rep {rep}",
                    F32_EPS * np.abs(ref))
    del keep


def test_lsk_fused_ffn_q4_0(ctx):
    ff, k = 257, 5120
    wg, rg = device_weights(ctx, "q4_0", ff, k, seed=71)
    wu, ru = device_weights(ctx, "q4_0", ff, k, seed=72)
    x = np.random.default_rng(73).standard_normal(k).astype(np.float32)
    act = ctx.new_buffer(4 * ff)
    d.fused_ffn_q4_0_f32(ctx, wg, wu, ctx.buffer_from(x), act, ff, k)
    ctx.flush()
    g, gs = ora.gemv("q4_0", rg, x, ff, k)
    u, us = ora.gemv("q4_0", ru, x, ff, k)
    ffn_check(act.read(np.float32, ff), g, gs, u, us, "lsk ffn q4_0")


@pytest.fixture(scope="module")
def valuctx():
    old = os.environ.get("RUNIT_GEMV_VALU")
    os.environ["RUNIT_GEMV_VALU"] = "1"
    try:
        c = d.HipContext()
    finally:
        if old is None:
            del os.environ["RUNIT_GEMV_VALU"]
        else:
            os.environ["RUNIT_GEMV_VALU"] = old
    yield c
    c.close()


@pytest.mark.parametrize("what", ["q4k_ffn_7b", "q6k_lm_head_7b"])
def test_valu_dot_twin_equals_matrix_core_form(ctx, valuctx, what):
    """The VALU-dot twins (v_dot4 over the three limbs) of the 7B Q4_K FFN
    and the Q6_K LM head compute the same integer sums and the same f32
    combination as the matrix-core form: equal bit for bit, and on the
    oracle."""
    outs = []
    if what == "q4k_ffn_7b":
        ff, k = 18944, 3584
        for c in (ctx, valuctx):
            wg, rg = device_weights(c, "q4k", ff, k, seed=31)
            wu, ru = device_weights(c, "q4k", ff, k, seed=32)
            xb = c.new_buffer(4 * k)
            d.synth_normal_f32(c, xb, k, 33)
            c.flush()
            x = xb.read(np.float32, k)
            ob = c.new_buffer(4 * ff)
            d.fused_ffn_q4k_f32(c, wg, wu, xb, ob, ff, k)
            c.flush()
            outs.append(ob.read(np.float32, ff))
        g_ref, g_s = ora.gemv("q4k", rg, x, ff, k)
        u_ref, u_s = ora.gemv("q4k", ru, x, ff, k)
        ffn_check(outs[1], g_ref, g_s, u_ref, u_s, "q4k valu ffn")
    else:
        n, k = 152064, 3584
        for c in (ctx, valuctx):
            wb, raw = device_weights(c, "q6k", n, k, seed=41)
            xb = c.new_buffer(4 * k)
            d.synth_normal_f32(c, xb, k, 42)
            c.flush()
            x = xb.read(np.float32, k)
            ob = c.new_buffer(4 * n)
            d.gemv_q6k_f32in_f32out(c, wb, xb, ob, n, k)
            c.flush()
            outs.append(ob.read(np.float32, n))
        rows = slice(0, 4096)  # oracle on a slice of the rows (CPU time)
        ref, sabs = ora.gemv("q6k", raw[:4096 * (k // 256) * 210], x, 4096, k)
        check_close(outs[1][rows], ref, sabs, "q6k valu lm head")
    assert np.array_equal(outs[0], outs[1])
