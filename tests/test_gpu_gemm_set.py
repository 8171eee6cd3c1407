"""rt_gemm_set_f32: the batched GEMMs of one activation matrix with the
RMSNorm in the activation preparation and the bias / residual / SiLU in the
K-split sums (verify_draft's projections, forward.rs:2186-2271), against the
oracle: the normalised rows against ora.rms_norm, each projection against the
per-row f64 GEMV of the same packed blocks over the rows the GPU normalised.
Row counts cover the shared f16 form (8, 27, 32 rows; 27 leaves padded rows
in the last group) and its fallbacks (1 row: GEMVs; 4 rows: the int8 form of
the 4-bit formats, separate launches)."""
import numpy as np
import pytest

import oracle_lib as ora
from runit_mac_amd import dispatch as d
from gpu_helpers import check_close, device_weights
from test_gpu_fused import ffn_check

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _x(m, k, seed):
    return np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)


def _norm_checked(ctx, xn, x, gamma, m, h):
    got = xn.read(np.float32, m * h).reshape(m, h)
    ref = ora.rms_norm(x, gamma, EPS).reshape(m, h)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.abs(ref).max(), "rms_norm rows"
    return got


@pytest.mark.parametrize("fmts", [("q4k", "q4k", "q6k"), ("q8_0", "q8_0", "q8_0")])
@pytest.mark.parametrize("m", [1, 4, 8, 27, 32])
def test_gemm_set_qkv_norm_bias(ctx, fmts, m):
    h, ns = 1024, [1024, 256, 256]
    W = [device_weights(ctx, f, n, h, 300 + i) for i, (f, n) in enumerate(zip(fmts, ns))]
    rng = np.random.default_rng(m)
    x = _x(m, h, m + 10)
    gamma = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    biases = [(0.1 * rng.standard_normal(n)).astype(np.float16) for n in ns]
    ys = [ctx.new_buffer(4 * m * n) for n in ns]
    xn = ctx.new_buffer(4 * m * h)
    d.gemm_set_f32(ctx, list(fmts), [w for w, _ in W], ys, ns, ctx.buffer_from(x), m, h,
                   biases=[ctx.buffer_from(b.view(np.uint16)) for b in biases],
                   gamma=ctx.buffer_from(gamma), eps=EPS, xn=xn)
    ctx.flush()
    xr = _norm_checked(ctx, xn, x, gamma, m, h)
    for i, (f, n) in enumerate(zip(fmts, ns)):
        yref, sabs = ora.gemv(f, W[i][1], xr, n, h)
        yref = yref + biases[i].astype(np.float64)[None, :]
        check_close(ys[i].read(np.float32, m * n), yref.ravel(), sabs.ravel(),
                    f"gemm_set {f} m={m} matrix {i}", extra=1e-6 * np.abs(yref.ravel()))


@pytest.mark.parametrize("fmt", ["q4k", "q8_0"])
@pytest.mark.parametrize("m", [1, 4, 8, 32])
def test_gemm_set_silu_pair(ctx, fmt, m):
    h, ff = 1024, 2048
    (wg, rg), (wu, ru) = device_weights(ctx, fmt, ff, h, 311), device_weights(ctx, fmt, ff, h, 312)
    x = _x(m, h, 40 + m)
    gamma = np.linspace(0.5, 1.5, h, dtype=np.float32)
    g, u, xn = ctx.new_buffer(4 * m * ff), ctx.new_buffer(4 * m * ff), ctx.new_buffer(4 * m * h)
    d.gemm_set_f32(ctx, [fmt, fmt], [wg, wu], [g, u], [ff, ff], ctx.buffer_from(x), m, h,
                   gamma=ctx.buffer_from(gamma), eps=EPS, xn=xn, silu_pair=True)
    ctx.flush()
    xr = _norm_checked(ctx, xn, x, gamma, m, h)
    gr, gs = ora.gemv(fmt, rg, xr, ff, h)
    ur, us = ora.gemv(fmt, ru, xr, ff, h)
    ffn_check(g.read(np.float32, m * ff), gr.ravel(), gs.ravel(), ur.ravel(), us.ravel(),
              f"gemm_set silu {fmt} m={m}")


@pytest.mark.parametrize("fmt,n,k", [("q6k", 1024, 2048), ("q4k", 1024, 3072), ("q8_0", 896, 4864),
                                     ("q8_0", 4864, 896), ("q4_0", 1000, 896)])
@pytest.mark.parametrize("m", [1, 4, 8, 32])
def test_gemm_set_residual(ctx, fmt, n, k, m):
    w, raw = device_weights(ctx, fmt, n, k, 320)
    x = _x(m, k, 50 + m)
    res = _x(m, n, 60 + m)
    y = ctx.new_buffer(4 * m * n)
    d.gemm_set_f32(ctx, [fmt], [w], [y], [n], ctx.buffer_from(x), m, k, res=ctx.buffer_from(res))
    ctx.flush()
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    yref = yref + res.astype(np.float64)
    check_close(y.read(np.float32, m * n), yref.ravel(), sabs.ravel(), f"gemm_set res {fmt} m={m}",
                extra=1e-6 * np.abs(yref.ravel()))


def test_gemm_set_rejects_bad_sets(ctx):
    w, _ = device_weights(ctx, "q8_0", 64, 256, 330)
    x, y, y2 = ctx.new_buffer(4 * 8 * 256), ctx.new_buffer(4 * 8 * 64), ctx.new_buffer(4 * 8 * 64)
    with pytest.raises(d.KernelError, match="residual"):
        d.gemm_set_f32(ctx, ["q8_0"], [w], [y], [64], x, 8, 256, res=y)  # res aliases y[0]
    with pytest.raises(d.KernelError, match="SiLU pair"):
        d.gemm_set_f32(ctx, ["q8_0"], [w], [y], [64], x, 8, 256, silu_pair=True)
    with pytest.raises(d.KernelError, match="format"):
        d.gemm_set_f32(ctx, ["q9"], [w], [y], [64], x, 8, 256)
    with pytest.raises(d.KernelError, match="gamma without xn"):
        d.gemm_set_f32(ctx, ["q8_0", "q8_0"], [w, w], [y, y2], [64, 64], x, 8, 256, gamma=x)


@pytest.mark.parametrize("fmts", [("q4k", "q4k", "q4k", "q6k"), ("q8_0", "q8_0", "q8_0", "q8_0")])
@pytest.mark.parametrize("m", [1, 4, 8, 27, 32, 70])
def test_gemm_ffn_block_equals_the_three_sets(ctx, fmts, m):
    """rt_gemm_ffn_block_f32 against the same layer part as three GEMM sets
    (each pinned to the oracle above): the folded sums add the same terms in
    the same order, so x_mid and x are bit-identical.  70 rows: the SiLU sum
    folded into the down projection's preparation as well (64 rows on)."""
    h, qd, ff = 1024, 1024, 2048
    fo, fg, fu, fd = fmts
    wo, _ = device_weights(ctx, fo, h, qd, 340)
    wg, _ = device_weights(ctx, fg, ff, h, 341)
    wu, _ = device_weights(ctx, fu, ff, h, 342)
    wd, _ = device_weights(ctx, fd, h, ff, 343)
    att = ctx.buffer_from(_x(m, qd, 70 + m))
    x0 = _x(m, h, 80 + m)
    gamma = ctx.buffer_from(np.linspace(0.5, 1.5, h, dtype=np.float32))
    outs = []
    for block in (True, False):
        x, xm = ctx.buffer_from(x0), ctx.new_buffer(4 * m * h)
        g, u, xn = ctx.new_buffer(4 * m * ff), ctx.new_buffer(4 * m * ff), ctx.new_buffer(4 * m * h)
        if block:
            d.gemm_ffn_block_f32(ctx, fmts, wo, wg, wu, wd, att, x, xm, gamma, EPS, g, u, xn,
                                 m, h, qd, ff)
        else:
            d.gemm_set_f32(ctx, [fo], [wo], [xm], [h], att, m, qd, res=x)
            d.gemm_set_f32(ctx, [fg, fu], [wg, wu], [g, u], [ff, ff], xm, m, h, gamma=gamma,
                           eps=EPS, xn=xn, silu_pair=True)
            d.gemm_set_f32(ctx, [fd], [wd], [x], [h], g, m, ff, res=xm)
        ctx.flush()
        outs.append((xm.read(np.float32, m * h), x.read(np.float32, m * h)))
    assert np.array_equal(outs[0][0], outs[1][0]), "x_mid"
    assert np.array_equal(outs[0][1], outs[1][1]), "x"
    assert np.all(np.isfinite(outs[0][1]))


@pytest.mark.parametrize("fmts,hd,heads,kvh", [(("q4k", "q4k", "q6k"), 128, 8, 2),
                                               (("q8_0", "q8_0", "q8_0"), 64, 14, 2)])
@pytest.mark.parametrize("m", [1, 4, 8, 27, 32])
def test_gemm_qkv_rope_equals_set_then_rope(ctx, fmts, hd, heads, kvh, m):
    """rt_gemm_qkv_rope_f32 against the Q/K/V set followed by
    rt_rope_kv_write_batch_f32 (each pinned to the oracle elsewhere): the
    same sums and angles; the rotation's r·c − i·s may contract to a fused
    multiply-add differently in the two kernels, so the rotated q and keys
    agree to 2e-6 of their range and the values exactly; the cache outside
    rows start_pos .. start_pos + m stays untouched."""
    h, qd, kvd, S, start = 1024, heads * hd, kvh * hd, 64, 20
    W = [device_weights(ctx, f, n, h, 350 + i) for i, (f, n) in enumerate(zip(fmts, (qd, kvd, kvd)))]
    rng = np.random.default_rng(90 + m)
    x = ctx.buffer_from(_x(m, h, 91 + m))
    gamma = ctx.buffer_from((1 + 0.1 * rng.standard_normal(h)).astype(np.float32))
    biases = [ctx.buffer_from((0.1 * rng.standard_normal(n)).astype(np.float16).view(np.uint16))
              for n in (qd, kvd, kvd)]
    cache0 = rng.standard_normal(kvh * S * hd).astype(np.float32)
    outs = []
    for fused in (True, False):
        q, k, v = (ctx.new_buffer(4 * m * n) for n in (qd, kvd, kvd))
        xn = ctx.new_buffer(4 * m * h)
        kc, vc = ctx.buffer_from(cache0), ctx.buffer_from(cache0)
        if fused:
            d.gemm_qkv_rope_f32(ctx, fmts, W[0][0], W[1][0], W[2][0], *biases, x, gamma, EPS, xn,
                                q, k, v, kc, vc, m, h, qd, kvd, hd, start, 10000.0, S)
        else:
            d.gemm_set_f32(ctx, list(fmts), [w for w, _ in W], [q, k, v], [qd, kvd, kvd], x, m, h,
                           biases=biases, gamma=gamma, eps=EPS, xn=xn)
            d.rope_kv_write_batch_f32(ctx, q, k, v, kc, vc, hd, heads, kvh, start, 10000.0, m, S)
        ctx.flush()
        outs.append([b.read(np.float32, n) for b, n in ((q, m * qd), (kc, cache0.size),
                                                        (vc, cache0.size))])
    for a, b, what in zip(outs[0][:2], outs[1][:2], ("q", "k cache")):
        assert np.max(np.abs(a - b)) <= 2e-6 * np.abs(b).max(), what
    assert np.array_equal(outs[0][2], outs[1][2]), "v cache"
    kc = outs[0][1].reshape(kvh, S, hd)
    keep = np.ones(S, bool)
    keep[start:start + m] = False
    assert np.array_equal(kc[:, keep], cache0.reshape(kvh, S, hd)[:, keep]), "rows outside"


def test_gemm_set_unaligned_operands_take_the_separate_launches(ctx):
    """A γ that is not 16-byte aligned (the shared form loads it in 16-byte
    units) makes the set run as the separate launches; the result matches
    the aligned call to rounding."""
    m, h, n = 8, 1024, 512
    w, _ = device_weights(ctx, "q4k", n, h, 360)
    x = ctx.buffer_from(_x(m, h, 361))
    gamma = np.linspace(0.5, 1.5, h, dtype=np.float32)
    ga = ctx.buffer_from(gamma)
    gu = ctx.new_buffer(4 * (h + 1))
    gu.write(gamma, offset=4)
    outs = []
    for gptr in (ga, gu.ptr + 4):
        y, xn = ctx.new_buffer(4 * m * n), ctx.new_buffer(4 * m * h)
        d.gemm_set_f32(ctx, ["q4k"], [w], [y], [n], x, m, h, gamma=gptr, eps=EPS, xn=xn)
        ctx.flush()
        outs.append(y.read(np.float32, m * n))
    assert np.max(np.abs(outs[0] - outs[1])) <= 1e-5 * np.abs(outs[1]).max()


@pytest.mark.parametrize("fmts", [("q4k", "q4k", "q4k", "q6k"), ("q8_0", "q8_0", "q8_0", "q8_0")])
@pytest.mark.parametrize("hd,heads,kvh", [(128, 8, 2), (64, 16, 2)])
@pytest.mark.parametrize("m,start", [(4, 300), (8, 40), (8, 300), (27, 200), (32, 0), (70, 200)])
def test_gemm_attn_ffn_block_equals_attention_then_block(ctx, fmts, hd, heads, kvh, m, start):
    """rt_gemm_attn_ffn_block_f32 against rt_flash_attention_f32 then
    rt_gemm_ffn_block_f32 (both pinned above and in the attention tests).
    8 rows after 300 cached positions and 27 / 70 rows after 200 take the
    folded form (the attention's key-range partials merged in the O
    preparation, 3-8 ranges); 8 rows after 40 and 32 rows from position 0
    (one key range) and 4 rows (int8 form of Q4_K) the two calls.  The merge adds the
    same terms as the attention's last workgroup, up to the rounding of the
    division: x within 1e-5 of its largest magnitude."""
    h, qd, ff, max_seq = 1024, heads * hd, 2048, 512
    fo, fg, fu, fd = fmts
    wo, _ = device_weights(ctx, fo, h, qd, 350)
    wg, _ = device_weights(ctx, fg, ff, h, 351)
    wu, _ = device_weights(ctx, fu, ff, h, 352)
    wd, _ = device_weights(ctx, fd, h, ff, 353)
    rng = np.random.default_rng(90 + m)
    q = ctx.buffer_from(rng.standard_normal((m, qd)).astype(np.float32))
    kc = ctx.buffer_from(rng.standard_normal((kvh, max_seq, hd)).astype(np.float32))
    vc = ctx.buffer_from(rng.standard_normal((kvh, max_seq, hd)).astype(np.float32))
    x0 = _x(m, h, 95 + m)
    gamma = ctx.buffer_from(np.linspace(0.5, 1.5, h, dtype=np.float32))
    outs = []
    for fused in (True, False):
        att = ctx.new_buffer(4 * m * qd)
        x, xm = ctx.buffer_from(x0), ctx.new_buffer(4 * m * h)
        g, u, xn = ctx.new_buffer(4 * m * ff), ctx.new_buffer(4 * m * ff), ctx.new_buffer(4 * m * h)
        if fused:
            d.gemm_attn_ffn_block_f32(ctx, q, kc, vc, start + m, heads, kvh, hd, max_seq, start,
                                      att, fmts, wo, wg, wu, wd, x, xm, gamma, EPS, g, u, xn,
                                      m, h, ff)
        else:
            d.flash_attention_f32(ctx, q, kc, vc, att, 1, m, start + m, heads, kvh, hd, max_seq,
                                  q_start=start)
            d.gemm_ffn_block_f32(ctx, fmts, wo, wg, wu, wd, att, x, xm, gamma, EPS, g, u, xn,
                                 m, h, qd, ff)
        ctx.flush()
        outs.append((xm.read(np.float32, m * h), x.read(np.float32, m * h)))
    for i, name in enumerate(("x_mid", "x")):
        a, b = outs[0][i], outs[1][i]
        assert np.all(np.isfinite(a)), name
        assert np.max(np.abs(a - b)) <= 1e-5 * np.abs(b).max(), name
