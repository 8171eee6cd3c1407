"""GPU parity of the decode-step glue (RMSNorm, RoPE, KV scatter, decode
attention, fused variants, embedding) against the CPU oracle."""
import numpy as np
import pytest

import oracle_lib as ora
from gpu_helpers import F32_EPS, check_close, device_weights
from runit_mac_amd import dispatch as d

pytestmark = pytest.mark.gpu


def test_rms_norm(ctx):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 896)).astype(np.float32) * 3
    g = (1 + 0.02 * rng.standard_normal(896)).astype(np.float32)
    y = ctx.new_buffer(x.nbytes)
    d.rms_norm_f32_f32_f32g(ctx, ctx.buffer_from(x), y, ctx.buffer_from(g), 1e-6, 896, 3)
    ctx.flush()
    ref = ora.rms_norm(x, g, 1e-6).ravel()
    got = y.read(np.float32, x.size)
    # f32 Σx² over 896 terms and one rsqrt: a few ulps relative
    assert np.all(np.abs(got - ref) <= 4e-6 * np.abs(ref) + 1e-7)
    # in place (y aliases x), as the reference's QK-norm calls do
    xb = ctx.buffer_from(x)
    d.rms_norm_f32_f32_f32g(ctx, xb, xb, ctx.buffer_from(g), 1e-6, 896, 3)
    ctx.flush()
    assert np.all(np.abs(xb.read(np.float32, x.size) - ref) <= 4e-6 * np.abs(ref) + 1e-7)


@pytest.mark.parametrize("hidden", [3584, 8192, 8196, 90, 12])
def test_rms_norm_row_sizes(ctx, hidden):
    """Rows the one-round-trip form takes (multiples of 4 up to 8192) and
    rows it leaves to the element loop (8196, 90), in place and not."""
    rng = np.random.default_rng(hidden)
    x = rng.standard_normal((2, hidden)).astype(np.float32) * 2
    g = (1 + 0.02 * rng.standard_normal(hidden)).astype(np.float32)
    ref = ora.rms_norm(x, g, 1e-6).ravel()
    y = ctx.new_buffer(x.nbytes)
    d.rms_norm_f32_f32_f32g(ctx, ctx.buffer_from(x), y, ctx.buffer_from(g), 1e-6, hidden, 2)
    xb = ctx.buffer_from(x)
    d.rms_norm_f32_f32_f32g(ctx, xb, xb, ctx.buffer_from(g), 1e-6, hidden, 2)
    ctx.flush()
    tol = 2e-5 * np.abs(ref) + 1e-7  # f32 Σx² over up to 8196 terms, one rsqrt
    assert np.all(np.abs(y.read(np.float32, x.size) - ref) <= tol)
    assert np.all(np.abs(xb.read(np.float32, x.size) - ref) <= tol)


@pytest.mark.parametrize("pos", [0, 1, 511, 4095])
def test_fused_rope(ctx, pos):
    rng = np.random.default_rng(pos)
    hd, qh, kvh, theta = 64, 14, 2, 1e6
    q = rng.standard_normal(qh * hd).astype(np.float32)
    k = rng.standard_normal(kvh * hd).astype(np.float32)
    qb, kb = ctx.buffer_from(q), ctx.buffer_from(k)
    d.fused_rope_qk_f32(ctx, qb, kb, hd, qh, kvh, pos, theta)
    ctx.flush()
    for buf, v, h in ((qb, q, qh), (kb, k, kvh)):
        ref = ora.rope(v, h, hd, pos, theta)
        got = buf.read(np.float32, v.size).astype(np.float64)
        vv = v.reshape(h, hd).astype(np.float64)
        mag = np.abs(np.concatenate([vv[:, :hd // 2], vv[:, :hd // 2]], axis=1)) + \
            np.abs(np.concatenate([vv[:, hd // 2:], vv[:, hd // 2:]], axis=1))
        # powf / sincosf of an f32 angle up to ~4e3 rad: ≤ ~1e-4 relative
        assert np.all(np.abs(got - ref) <= 2e-4 * mag.ravel() + 1e-6)


def test_kv_copy(ctx):
    hd, kvh, max_seq, pos = 64, 2, 40, 17
    src = np.random.default_rng(1).standard_normal(kvh * hd).astype(np.float32)
    cache = np.zeros((kvh, max_seq, hd), np.float32)
    cb = ctx.buffer_from(cache)
    d.kv_copy_to_cache_f32(ctx, ctx.buffer_from(src), cb, pos, max_seq, hd, kvh)
    ctx.flush()
    cache[:, pos] = src.reshape(kvh, hd)
    assert np.array_equal(cb.read(np.float32, cache.size), cache.ravel())


@pytest.mark.parametrize("kv_len", [0, 1, 7, 512, 5000])
def test_decode_attention(ctx, kv_len):
    rng = np.random.default_rng(kv_len)
    H, KVH, hd, S = 14, 2, 64, max(kv_len, 1) + 3
    q = rng.standard_normal(H * hd).astype(np.float32)
    k = rng.standard_normal((KVH, S, hd)).astype(np.float32)
    v = rng.standard_normal((KVH, S, hd)).astype(np.float32)
    out = ctx.new_buffer(4 * H * hd)
    d.decode_attention_f32(ctx, ctx.buffer_from(q), ctx.buffer_from(k), ctx.buffer_from(v), out,
                           1, kv_len, H, KVH, hd, S)
    ctx.flush()
    ref = ora.attention(q, k, v, H, KVH, hd, kv_len, S)
    got = out.read(np.float32, H * hd).astype(np.float64)
    vmax = np.abs(v).max()
    # f32 scores / exp / weighted sums over ≤ 5000 positions
    assert np.all(np.abs(got - ref) <= 2e-5 * vmax + 1e-6), np.abs(got - ref).max()


@pytest.mark.parametrize("batch,H,KVH,hd,kv_len", [
    (2, 14, 2, 64, 300),     # batch rows share no state
    (1, 32, 2, 128, 1500),   # 16 query heads per kv head: two head blocks
    (1, 40, 8, 128, 4097),   # 5 per kv head, a ragged last split
    (1, 8, 8, 256, 65),      # MHA, head_dim 256
    (1, 4, 1, 64, 20000),    # many splits, each longer than 64 positions
])
def test_decode_attention_shapes(ctx, batch, H, KVH, hd, kv_len):
    rng = np.random.default_rng(H * kv_len + hd)
    S = kv_len + 5
    q = rng.standard_normal((batch, H * hd)).astype(np.float32)
    k = rng.standard_normal((batch, KVH, S, hd)).astype(np.float32)
    v = rng.standard_normal((batch, KVH, S, hd)).astype(np.float32)
    out = ctx.new_buffer(4 * batch * H * hd)
    qb, kb, vb = ctx.buffer_from(q), ctx.buffer_from(k), ctx.buffer_from(v)
    for _ in range(2):  # the second call reuses the arrival counters
        d.decode_attention_f32(ctx, qb, kb, vb, out, batch, kv_len, H, KVH, hd, S)
        ctx.flush()
        got = out.read(np.float32, batch * H * hd).reshape(batch, -1).astype(np.float64)
        for bi in range(batch):
            ref = ora.attention(q[bi], k[bi], v[bi], H, KVH, hd, kv_len, S)
            assert np.all(np.abs(got[bi] - ref) <= 2e-5 * np.abs(v[bi]).max() + 1e-6), \
                (bi, np.abs(got[bi] - ref).max())


@pytest.mark.parametrize("pos", [0, 511, 4200])
def test_decode_attention_rope_fused(ctx, pos):
    rng = np.random.default_rng(pos + 1)
    H, KVH, hd, max_seq, theta = 14, 2, 64, 4300, 1e6
    q = rng.standard_normal(H * hd).astype(np.float32)
    k_new = rng.standard_normal(KVH * hd).astype(np.float32)
    v_new = rng.standard_normal(KVH * hd).astype(np.float32)
    kc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    kcb, vcb = ctx.buffer_from(kc), ctx.buffer_from(vc)
    out = ctx.new_buffer(4 * H * hd)
    d.decode_attention_rope_f32(ctx, ctx.buffer_from(q), ctx.buffer_from(k_new),
                                ctx.buffer_from(v_new), kcb, vcb, out, pos, max_seq, H, KVH, hd,
                                theta)
    ctx.flush()
    q_r = ora.rope(q, H, hd, pos, theta)
    k_r = ora.rope(k_new, KVH, hd, pos, theta)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, pos] = k_r.reshape(KVH, hd).astype(np.float32)
    vc2[:, pos] = v_new.reshape(KVH, hd)
    got_k = kcb.read(np.float32, kc.size).reshape(kc.shape)
    got_v = vcb.read(np.float32, vc.size).reshape(vc.shape)
    # cache: untouched except position pos (v exact, rotated k to RoPE tolerance)
    mask = np.ones(max_seq, bool)
    mask[pos] = False
    assert np.array_equal(got_k[:, mask], kc[:, mask]) and np.array_equal(got_v, vc2)
    assert np.all(np.abs(got_k[:, pos] - kc2[:, pos]) <= 2e-4 * 2 * np.abs(k_new).max() + 1e-6)
    ref = ora.attention(q_r, kc2, vc2, H, KVH, hd, pos + 1, max_seq)
    got = out.read(np.float32, H * hd).astype(np.float64)
    # RoPE angle error (≤ ~1e-4 relative on q, k) moves the scores by ≲ 1e-3
    # relative; the output stays within 2e-3·max|v|
    assert np.all(np.abs(got - ref) <= 2e-3 * np.abs(vc2).max() + 1e-6), np.abs(got - ref).max()


@pytest.mark.parametrize("fmt,H,KVH,hd,hidden,pos", [
    ("q8_0", 14, 2, 64, 896, 0), ("q8_0", 14, 2, 64, 896, 63), ("q8_0", 14, 2, 64, 896, 511),
    ("q8_0", 14, 2, 64, 896, 4200), ("q8_0", 8, 8, 128, 512, 300), ("q8_0", 28, 4, 128, 3584, 511),
    # Q4_K projections (q_dim a multiple of 256): merged at 2..8 KV splits
    # (pos 63..511), the two kernels at one split (pos 0) and past 8 (pos 1000)
    ("q4k", 28, 4, 128, 3584, 0), ("q4k", 28, 4, 128, 3584, 63), ("q4k", 28, 4, 128, 3584, 511),
    ("q4k", 28, 4, 128, 3584, 1000), ("q4k", 8, 8, 128, 512, 300), ("q4k", 16, 2, 64, 1024, 200),
    ("q4kg", 28, 4, 128, 3584, 511), ("q4kg", 8, 8, 128, 512, 300)])
def test_attention_oproj_matches_the_two_call_sequence(ctx, fmt, H, KVH, hd, hidden, pos):
    """decode_attention_rope_oproj_<fmt>_f32 (split merge inside the
    projection's staging when the attention splits the KV range in 2..8,
    else the two kernels) against decode_attention_rope_f32 followed by
    gemv_<fmt>_add_f32_f32in on copies of the same inputs."""
    rng = np.random.default_rng(pos + hd)
    max_seq, theta, q_dim = 4300, 1e6, H * hd
    q = rng.standard_normal(q_dim).astype(np.float32)
    k_new = rng.standard_normal(KVH * hd).astype(np.float32)
    v_new = rng.standard_normal(KVH * hd).astype(np.float32)
    kc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    x0 = rng.standard_normal(hidden).astype(np.float32)
    wo, raw = device_weights(ctx, fmt, hidden, q_dim, seed=pos + 3)
    qb, kb, vb = ctx.buffer_from(q), ctx.buffer_from(k_new), ctx.buffer_from(v_new)
    # the two-call sequence
    kc1, vc1, x1 = ctx.buffer_from(kc), ctx.buffer_from(vc), ctx.buffer_from(x0)
    att = ctx.new_buffer(4 * q_dim)
    d.decode_attention_rope_f32(ctx, qb, kb, vb, kc1, vc1, att, pos, max_seq, H, KVH, hd, theta)
    getattr(d, f"gemv_{fmt}_add_f32_f32in")(ctx, wo, att, x1, x1, hidden, q_dim)
    # the merged call
    kc2, vc2, x2 = ctx.buffer_from(kc), ctx.buffer_from(vc), ctx.buffer_from(x0)
    getattr(d, f"decode_attention_rope_oproj_{fmt}_f32")(ctx, qb, kb, vb, kc2, vc2, wo, x2, pos,
                                                         max_seq, H, KVH, hd, theta, hidden)
    ctx.flush()
    assert np.array_equal(kc1.read(np.float32, kc.size), kc2.read(np.float32, kc.size))
    assert np.array_equal(vc1.read(np.float32, vc.size), vc2.read(np.float32, vc.size))
    y1 = x1.read(np.float32, hidden).astype(np.float64)
    y2 = x2.read(np.float32, hidden).astype(np.float64)
    # same merge formula and order; the only freedom is the compiler's
    # contraction of the merge's multiply-adds, well inside the GEMV tolerance
    a = att.read(np.float32, q_dim).astype(np.float64)
    W = ora.dequant(fmt, raw).reshape(hidden, q_dim).astype(np.float64)
    sabs = np.abs(W) @ np.abs(a)
    assert np.all(np.abs(y1 - y2) <= 1e-5 * sabs + 1e-6), np.abs(y1 - y2).max()


def test_embed_q8_0(ctx):
    vocab, k = 1000, 896
    tb, raw = device_weights(ctx, "q8_0", vocab, k, 5)
    tok = ctx.buffer_from(np.array([777], np.uint32))
    out = ctx.new_buffer(4 * k)
    d.embed_q8_0_f32(ctx, tb, tok, out, k)
    ctx.flush()
    row = ora.dequant("q8_0", raw[777 * (k // 32) * 34:778 * (k // 32) * 34])
    assert np.array_equal(out.read(np.float32, k).view(np.uint32), row.view(np.uint32))


def test_rms_norm_fused_gemvs(ctx):
    rng = np.random.default_rng(3)
    h, q_dim, kv_dim, ff = 896, 896, 128, 4864
    x = (3 * rng.standard_normal(h)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(h)).astype(np.float32)
    xn = ora.rms_norm(x, g, 1e-6).astype(np.float32)  # oracle input of the GEMVs (f64→f32)
    xb, gb = ctx.buffer_from(x), ctx.buffer_from(g)
    ws = [device_weights(ctx, "q8_0", n, h, 10 + i) for i, n in enumerate((q_dim, kv_dim, kv_dim))]
    bias = [(0.02 * rng.standard_normal(n)).astype(np.float16) for n in (q_dim, kv_dim, kv_dim)]
    outs = [ctx.new_buffer(4 * n) for n in (q_dim, kv_dim, kv_dim)]
    d.rms_norm_fused_qkv_bias_q8_0_f32(ctx, ws[0][0], ws[1][0], ws[2][0], xb, gb, 1e-6, *outs,
                                       *[ctx.buffer_from(b) for b in bias], q_dim, kv_dim, h)
    wg, rg = device_weights(ctx, "q8_0", ff, h, 20)
    wu, ru = device_weights(ctx, "q8_0", ff, h, 21)
    act = ctx.new_buffer(4 * ff)
    d.rms_norm_fused_ffn_q8_0_f32(ctx, wg, wu, xb, gb, 1e-6, act, ff, h)
    wl, rl = device_weights(ctx, "q8_0", 5000, h, 22)
    yl = ctx.new_buffer(4 * 5000)
    d.rms_norm_gemv_q8_0_f32in_f32out(ctx, wl, xb, gb, 1e-6, yl, 5000, h)
    ctx.flush()
    # the f32-vs-f64 normalised input adds ≤ ~1e-6 relative per element,
    # inside the 1e-4·Σ|w·x| bound
    for i, n in enumerate((q_dim, kv_dim, kv_dim)):
        y, s = ora.gemv("q8_0", ws[i][1], xn, n, h)
        ref = y + bias[i].astype(np.float64)
        check_close(outs[i].read(np.float32, n), ref, s, f"norm+qkv[{i}]", F32_EPS * np.abs(ref))
    from test_gpu_fused import ffn_check
    gr, gs = ora.gemv("q8_0", rg, xn, ff, h)
    ur, us = ora.gemv("q8_0", ru, xn, ff, h)
    ffn_check(act.read(np.float32, ff), gr, gs, ur, us, "norm+ffn")
    y, s = ora.gemv("q8_0", rl, xn, 5000, h)
    check_close(yl.read(np.float32, 5000), y, s, "norm+lm head")


def test_rms_norm_fused_q4k_m_gemvs(ctx):
    """The Q4_K_M forms: norm + Q/K (Q4_K) + V (Q6_K) + biases, norm + Q4_K
    gate+up+SiLU, norm + Q6_K LM head, at 7B widths (hidden 3584; the FFN
    and LM head narrower than the model's, same code paths)."""
    rng = np.random.default_rng(4)
    h, q_dim, kv_dim, ff, vocab = 3584, 3584, 512, 4096, 20000
    x = (3 * rng.standard_normal(h)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(h)).astype(np.float32)
    xn = ora.rms_norm(x, g, 1e-6).astype(np.float32)
    xb, gb = ctx.buffer_from(x), ctx.buffer_from(g)
    fmts = ("q4k", "q4k", "q6k")
    ws = [device_weights(ctx, f, n, h, 30 + i) for i, (f, n) in
          enumerate(zip(fmts, (q_dim, kv_dim, kv_dim)))]
    bias = [(0.02 * rng.standard_normal(n)).astype(np.float16) for n in (q_dim, kv_dim, kv_dim)]
    outs = [ctx.new_buffer(4 * n) for n in (q_dim, kv_dim, kv_dim)]
    d.rms_norm_fused_qkv_bias_q4k_q6k_f32(ctx, ws[0][0], ws[1][0], ws[2][0], xb, gb, 1e-6, *outs,
                                          *[ctx.buffer_from(b) for b in bias], q_dim, kv_dim, h)
    wg, rg = device_weights(ctx, "q4k", ff, h, 40)
    wu, ru = device_weights(ctx, "q4k", ff, h, 41)
    act = ctx.new_buffer(4 * ff)
    d.rms_norm_fused_ffn_q4k_f32(ctx, wg, wu, xb, gb, 1e-6, act, ff, h)
    wl, rl = device_weights(ctx, "q6k", vocab, h, 42)
    yl = ctx.new_buffer(4 * vocab)
    d.rms_norm_gemv_q6k_f32in_f32out(ctx, wl, xb, gb, 1e-6, yl, vocab, h)
    ctx.flush()
    for i, n in enumerate((q_dim, kv_dim, kv_dim)):
        y, s = ora.gemv(fmts[i], ws[i][1], xn, n, h)
        ref = y + bias[i].astype(np.float64)
        check_close(outs[i].read(np.float32, n), ref, s, f"norm+qkv[{i}] {fmts[i]}",
                    F32_EPS * np.abs(ref))
    from test_gpu_fused import ffn_check
    gr, gs = ora.gemv("q4k", rg, xn, ff, h)
    ur, us = ora.gemv("q4k", ru, xn, ff, h)
    ffn_check(act.read(np.float32, ff), gr, gs, ur, us, "norm+ffn q4k")
    y, s = ora.gemv("q6k", rl, xn, vocab, h)
    check_close(yl.read(np.float32, vocab), y, s, "norm+lm head q6k")
    # k past the norm-fused staging limit is refused, not run unnormalised
    with pytest.raises(d.Dispatch):
        d.rms_norm_fused_qkv_bias_q4k_q6k_f32(ctx, ws[0][0], ws[1][0], ws[2][0], xb, gb, 1e-6,
                                              *outs, *[ctx.buffer_from(b) for b in bias], 4, 4,
                                              8448)


@pytest.mark.parametrize("fmt,H,KVH,hd,hidden,pos", [
    ("q4k", 28, 4, 128, 3584, 511), ("q4k", 28, 4, 128, 3584, 200),
    ("q4kg", 28, 4, 128, 3584, 511), ("q8_0", 14, 2, 64, 896, 511)])
def test_attention_oproj_matches_oracle(ctx, fmt, H, KVH, hd, hidden, pos):
    """decode_attention_rope_oproj_<fmt>_f32 at the 7B head count (28/4 heads
    of 128, hidden 3584: 8 KV splits merged in the O projection's staging at
    pos 511, 4 at pos 200) against the f64 oracle: RoPE, the cache write,
    attention over pos + 1 positions (attention.metal:248-308) and
    x + W_o·att (gemv_multirow.metal:205-243).

    theta = 1 makes every RoPE frequency exactly 1 (1/powf(1, ·) = 1), so
    every angle is the integer pos, exact in f32, and the device's f32
    rotation differs from the oracle's only by its sincosf rounding (~1e-7
    relative).  The tolerance is then the GEMV bound on the oracle's
    attention output plus the f32 attention error carried through |W_o|:
        |y − y_ref| ≤ 1e-4·Σ_j|w_ij·a_j| + Σ_j|w_ij|·ε_a,
        ε_a = 1e-5·max|v|  (f32 scores, exp and the ≤ 64-position partial
                             sums of each split, then an 8-way merge)."""
    rng = np.random.default_rng(pos + 7 * hd)
    max_seq, theta, q_dim = 1024, 1.0, H * hd
    q = rng.standard_normal(q_dim).astype(np.float32)
    k_new = rng.standard_normal(KVH * hd).astype(np.float32)
    v_new = rng.standard_normal(KVH * hd).astype(np.float32)
    kc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    x0 = rng.standard_normal(hidden).astype(np.float32)
    wo, raw = device_weights(ctx, fmt, hidden, q_dim, seed=pos + 11)
    qb, kb, vb = ctx.buffer_from(q), ctx.buffer_from(k_new), ctx.buffer_from(v_new)
    kcb, vcb, xb = ctx.buffer_from(kc), ctx.buffer_from(vc), ctx.buffer_from(x0)
    getattr(d, f"decode_attention_rope_oproj_{fmt}_f32")(ctx, qb, kb, vb, kcb, vcb, wo, xb, pos,
                                                         max_seq, H, KVH, hd, theta, hidden)
    ctx.flush()
    # oracle: rotate, write position pos, attend, project, add
    q_r = ora.rope(q.astype(np.float64), H, hd, pos, theta)
    k_r = ora.rope(k_new.astype(np.float64), KVH, hd, pos, theta)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, pos] = k_r.reshape(KVH, hd).astype(np.float32)
    vc2[:, pos] = v_new.reshape(KVH, hd)
    att = ora.attention(q_r, kc2, vc2, H, KVH, hd, pos + 1, max_seq)
    y, sabs = ora.gemv(fmt, raw, att.astype(np.float32), hidden, q_dim)
    ref = x0.astype(np.float64) + y
    W = np.abs(ora.dequant(fmt, raw).reshape(hidden, q_dim).astype(np.float64))
    eps_a = 1e-5 * np.abs(vc2[:, :pos + 1]).max()
    got = xb.read(np.float32, hidden)
    check_close(got, ref, sabs, f"attention+O {fmt} {H}/{KVH}x{hd} pos {pos}",
                W.sum(axis=1) * eps_a + F32_EPS * np.abs(ref))
    # the cache row the call wrote: v exact, k the rotated key
    assert np.array_equal(vcb.read(np.float32, vc.size).reshape(vc.shape)[:, pos], vc2[:, pos])
    got_k = kcb.read(np.float32, kc.size).reshape(kc.shape)[:, pos].astype(np.float64)
    assert np.all(np.abs(got_k - kc2[:, pos]) <= 1e-6 * np.abs(k_new).max())


@pytest.mark.parametrize("m,k", [(896, 4864), (4864, 896), (900, 896)])
def test_gemv_add_ssq_writes_quad_sums(ctx, m, k):
    """gemv_q8_0_add_f32_f32in_ssq: the same output as gemv_q8_0_add_f32_f32in
    (bit for bit) plus Σy² over every 4 output rows — written by the
    launch's own epilogue (896 rows: VALU small-launch body) or by a kernel
    of its own where the chosen body has no such epilogue (4864 rows)."""
    rng = np.random.default_rng(m + k)
    w, raw = device_weights(ctx, "q8_0", m, k, seed=m)
    x = rng.standard_normal(k).astype(np.float32)
    r = rng.standard_normal(m).astype(np.float32)
    y1, y2 = ctx.buffer_from(r), ctx.buffer_from(r)
    nq = (m + 3) // 4
    ssq = ctx.new_buffer(4 * nq)
    xb = ctx.buffer_from(x)
    d.gemv_q8_0_add_f32_f32in(ctx, w, xb, y1, y1, m, k)
    d.gemv_q8_0_add_f32_f32in_ssq(ctx, w, xb, y2, y2, m, k, ssq)
    ctx.flush()
    a, b = y1.read(np.float32, m), y2.read(np.float32, m)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    yy = np.zeros(4 * nq)
    yy[:m] = b.astype(np.float64) ** 2
    ref = yy.reshape(nq, 4).sum(axis=1)
    assert np.allclose(ssq.read(np.float32, nq), ref, rtol=4 * F32_EPS, atol=0)


def test_attention_oproj_and_norm_fused_ssq(ctx):
    """The 0.5B layer's hand-off: attention + O projection writing Σy² per
    quad (ssq), then norm-fused gate+up and Q/K/V reading them.  Producer:
    x bit-identical to the form without ssq; consumers: within 1e-6 relative
    of the forms that reduce x themselves (the only difference is the order
    of the f32 Σx²)."""
    rng = np.random.default_rng(9)
    H, KVH, hd, h, ff, pos, max_seq = 14, 2, 64, 896, 4864, 511, 1024
    q = rng.standard_normal(H * hd).astype(np.float32)
    kn = rng.standard_normal(KVH * hd).astype(np.float32)
    vn = rng.standard_normal(KVH * hd).astype(np.float32)
    kc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    vc = rng.standard_normal((KVH, max_seq, hd)).astype(np.float32)
    x0 = rng.standard_normal(h).astype(np.float32)
    wo, _ = device_weights(ctx, "q8_0", h, H * hd, seed=1)
    qb, kb, vb = ctx.buffer_from(q), ctx.buffer_from(kn), ctx.buffer_from(vn)
    outs = []
    ssq = ctx.new_buffer(4 * (h // 4))
    for with_ssq in (False, True):
        kcb, vcb, xb = ctx.buffer_from(kc), ctx.buffer_from(vc), ctx.buffer_from(x0)
        args = (ctx, qb, kb, vb, kcb, vcb, wo, xb, pos, max_seq, H, KVH, hd, 1e6, h)
        if with_ssq:
            d.decode_attention_rope_oproj_q8_0_f32_ssq(*args, ssq)
        else:
            d.decode_attention_rope_oproj_q8_0_f32(*args)
        ctx.flush()
        outs.append(xb)
    x1 = outs[0].read(np.float32, h)
    assert np.array_equal(x1.view(np.uint32), outs[1].read(np.float32, h).view(np.uint32))
    ref = (x1.astype(np.float64) ** 2).reshape(-1, 4).sum(axis=1)
    assert np.allclose(ssq.read(np.float32, h // 4), ref, rtol=4 * F32_EPS, atol=0)
    # consumers
    xb = outs[1]
    g = ctx.buffer_from((1 + 0.02 * rng.standard_normal(h)).astype(np.float32))
    wg, _ = device_weights(ctx, "q8_0", ff, h, seed=2)
    wu, _ = device_weights(ctx, "q8_0", ff, h, seed=3)
    a1, a2 = ctx.new_buffer(4 * ff), ctx.new_buffer(4 * ff)
    d.rms_norm_fused_ffn_q8_0_f32(ctx, wg, wu, xb, g, 1e-6, a1, ff, h)
    d.rms_norm_fused_ffn_q8_0_f32_ssq(ctx, wg, wu, xb, g, 1e-6, a2, ff, h, ssq, h // 4)
    qkv = [(d.weight_bytes("q8_0", n, h), n) for n in (896, 128, 128)]
    ws = [device_weights(ctx, "q8_0", n, h, seed=10 + i)[0] for i, (_, n) in enumerate(qkv)]
    bias = [ctx.buffer_from((0.02 * rng.standard_normal(n)).astype(np.float16)) for _, n in qkv]
    o1 = [ctx.new_buffer(4 * n) for _, n in qkv]
    o2 = [ctx.new_buffer(4 * n) for _, n in qkv]
    d.rms_norm_fused_qkv_bias_q8_0_f32(ctx, *ws, xb, g, 1e-6, *o1, *bias, 896, 128, h)
    d.rms_norm_fused_qkv_bias_q8_0_f32_ssq(ctx, *ws, xb, g, 1e-6, *o2, *bias, 896, 128, h, ssq,
                                           h // 4)
    ctx.flush()
    for u, v, n in [(a1, a2, ff)] + [(o1[i], o2[i], qkv[i][1]) for i in range(3)]:
        p1 = u.read(np.float32, n).astype(np.float64)
        p2 = v.read(np.float32, n).astype(np.float64)
        assert np.all(np.abs(p1 - p2) <= 1e-6 * np.abs(p1).max() + 1e-30), np.abs(p1 - p2).max()
