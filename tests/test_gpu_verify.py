"""The batched verify step (verify_draft, forward.rs:2118-2309) on the GPU:
its M-row kernels against the oracle, and the whole M-row pass against
sequential single-token steps of the CPU reference model (a causal batched
forward equals decoding its rows one after another)."""
import numpy as np
import pytest

import oracle_lib as ora
from runit_mac_amd import dispatch as d
from runit_mac_amd.decode import Q4K_M, DecodeConfig, DecodeModel

pytestmark = pytest.mark.gpu


def upload(ctx, arr):
    arr = np.ascontiguousarray(arr)
    buf = ctx.new_buffer(max(arr.nbytes, 16))
    buf.write(arr)
    return buf


def test_add_bias_silu_add_rows(ctx):
    rng = np.random.default_rng(1)
    seq, dim = 7, 1000
    x = rng.standard_normal(seq * dim).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float16)
    bx, bb = upload(ctx, x), upload(ctx, b)
    d.add_bias_broadcast_f32(ctx, bx, bb, seq, dim)
    ctx.flush()
    # one f32 addition of an exactly converted half: bit-exact
    assert np.array_equal(bx.read(np.float32, seq * dim),
                          (x.reshape(seq, dim) + b.astype(np.float32)).reshape(-1))
    g = rng.standard_normal(seq * dim).astype(np.float32) * 4
    u = rng.standard_normal(seq * dim).astype(np.float32)
    bg, bu, bo = upload(ctx, g), upload(ctx, u), ctx.new_buffer(4 * seq * dim)
    d.silu_mul_f32(ctx, bg, bu, bo, seq * dim)
    d.add_f32(ctx, bg, bu, bg, seq * dim)  # in place
    ctx.flush()
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(bo.read(np.float32, seq * dim), ref, rtol=1e-5, atol=1e-6)
    assert np.array_equal(bg.read(np.float32, seq * dim), g + u)


@pytest.mark.parametrize("hd,heads,start", [(64, 14, 0), (128, 4, 1000), (64, 2, 70000)])
def test_rope_batch_matches_oracle(ctx, hd, heads, start):
    rng = np.random.default_rng(hd + heads)
    seq = 9
    x = rng.standard_normal(seq * heads * hd).astype(np.float32)
    bx = upload(ctx, x)
    d.rope_batch_inplace_f32(ctx, bx, hd, heads, start, 1e6, seq)
    ctx.flush()
    ref = ora.rope_batch(x, seq, heads, hd, start, 1e6)
    # f32 angle (formed as the oracle forms it) and device sin/cos: a few ulp
    # of the angle, which is ≤ 7e4 rad here
    tol = 4e-7 * max(1.0, start + seq) * np.abs(x).max() + 1e-6
    assert np.max(np.abs(bx.read(np.float32, x.size) - ref)) <= tol


def test_kv_write_batch_places_rows(ctx):
    rng = np.random.default_rng(2)
    seq, kvh, hd, S, start = 5, 2, 64, 32, 27
    k = rng.standard_normal(seq * kvh * hd).astype(np.float32)
    v = rng.standard_normal(seq * kvh * hd).astype(np.float32)
    kc = rng.standard_normal(kvh * S * hd).astype(np.float32)
    vc = rng.standard_normal(kvh * S * hd).astype(np.float32)
    bk, bv, bkc, bvc = (upload(ctx, a) for a in (k, v, kc, vc))
    d.kv_write_batch_f32(ctx, bk, bv, bkc, bvc, start, seq, S, hd, kvh)
    ctx.flush()
    ek, ev = kc.reshape(kvh, S, hd).copy(), vc.reshape(kvh, S, hd).copy()
    ek[:, start:start + seq] = k.reshape(seq, kvh, hd).transpose(1, 0, 2)
    ev[:, start:start + seq] = v.reshape(seq, kvh, hd).transpose(1, 0, 2)
    assert np.array_equal(bkc.read(np.float32, kc.size), ek.reshape(-1))
    assert np.array_equal(bvc.read(np.float32, vc.size), ev.reshape(-1))
    with pytest.raises(d.Dispatch):
        d.kv_write_batch_f32(ctx, bk, bv, bkc, bvc, S - 2, seq, S, hd, kvh)


def test_argmax_rows_first(ctx):
    rng = np.random.default_rng(3)
    rows, n = 6, 151936
    m = rng.integers(-50, 50, size=(rows, n)).astype(np.float32)  # many ties
    m[1, :] = -np.inf
    m[2, ::3] = np.nan
    m[3, 100000] = 1e30
    m[3, 5] = 1e30
    bi, bo = upload(ctx, m), ctx.new_buffer(4 * rows)
    d.argmax_rows_first_f32(ctx, bi, bo, rows, n)
    ctx.flush()
    assert np.array_equal(bo.read(np.uint32, rows), ora.argmax_rows_first(m, rows))


@pytest.mark.parametrize("hd,H,KVH,M,kv_len,q_start", [
    (64, 14, 2, 8, 520, 512),     # verify with history: 0.5B heads, kv splits
    (64, 14, 2, 8, 8, 0),         # prefill from position 0
    (128, 28, 4, 5, 300, 0),      # the reference kernel's mask (q_start 0) with history
    (128, 28, 4, 16, 1040, 1024),
    (128, 28, 4, 200, 200, 0),    # prefill-length: many column groups, a few waves each
    (256, 8, 2, 6, 40, 34),       # head size 256 (4 column groups: the per-row kernel)
    (256, 8, 2, 40, 80, 40),      # head size 256 on the matrix cores
    (64, 12, 4, 7, 23, 16),       # 3 heads per KV head: column groups straddle rows
    (64, 12, 4, 11, 40, 29),      # the same on the matrix cores (12 column groups)
    (128, 28, 4, 1, 1, 0),        # one row, one position
])
def test_flash_attention_causal_matches_oracle(ctx, hd, H, KVH, M, kv_len, q_start):
    rng = np.random.default_rng(hd + M + kv_len)
    S = kv_len + 16
    q = rng.standard_normal(M * H * hd).astype(np.float32)
    kc = rng.standard_normal(KVH * S * hd).astype(np.float32)
    vc = rng.standard_normal(KVH * S * hd).astype(np.float32)
    bq, bk, bv = upload(ctx, q), upload(ctx, kc), upload(ctx, vc)
    bo = ctx.new_buffer(4 * M * H * hd)
    d.flash_attention_f32(ctx, bq, bk, bv, bo, 1, M, kv_len, H, KVH, hd, S, q_start)
    ctx.flush()
    got = bo.read(np.float32, M * H * hd).reshape(M, H * hd)
    ref = ora.causal_attention(q, kc, vc, M, H, KVH, hd, kv_len, S, q_start)
    # convex combination of values with f32 softmax: 1e-5 of the value range
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.abs(vc).max() * 8


@pytest.mark.parametrize("kv_len", [70, 300])
def test_flash_attention_batch_of_sequences(ctx, kv_len):
    """batch 2: each sequence reads its own cache [b][kvh][stride][hd] (at
    kv_len 300 the key range is split over workgroups and merged)."""
    rng = np.random.default_rng(9)
    hd, H, KVH, M, S = 64, 4, 2, 3, kv_len + 10
    q = rng.standard_normal(2 * M * H * hd).astype(np.float32)
    kc = rng.standard_normal(2 * KVH * S * hd).astype(np.float32)
    vc = rng.standard_normal(2 * KVH * S * hd).astype(np.float32)
    bq, bk, bv = upload(ctx, q), upload(ctx, kc), upload(ctx, vc)
    bo = ctx.new_buffer(4 * q.size)
    d.flash_attention_f32(ctx, bq, bk, bv, bo, 2, M, kv_len, H, KVH, hd, S, kv_len - M)
    ctx.flush()
    got = bo.read(np.float32, q.size).reshape(2, M, H * hd)
    per = KVH * S * hd
    for b in range(2):
        ref = ora.causal_attention(q.reshape(2, -1)[b], kc[b * per:(b + 1) * per],
                                   vc[b * per:(b + 1) * per], M, H, KVH, hd, kv_len, S, kv_len - M)
        assert np.max(np.abs(got[b] - ref)) <= 1e-4, b


def check_rows(got, ref, what):
    """Per row: logits within 1e-3 of the row's spread; the argmax equal to
    the reference's unless its top-2 gap is inside that tolerance."""
    for r in range(ref.shape[0]):
        tol = 1e-3 * (ref[r].max() - ref[r].min())
        err = np.max(np.abs(got[r] - ref[r]))
        assert err <= tol, (what, r, err, tol)


@pytest.mark.parametrize("form", ["rows", "gemm"])
@pytest.mark.parametrize("quant,cfg_kw,start", [
    (None, dict(layers=2, max_seq=600), 500),
    (Q4K_M, dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, ff=1024, vocab=1000,
                 max_seq=300), 130),
])
def test_verify_forward_equals_sequential_steps(ctx, quant, cfg_kw, start, form):
    """Each row of the batched pass equals the single-token step of the CPU
    reference model at its position (the host twin regenerated from the
    seeds, stepped once per row: its cache grows exactly as the batch's)."""
    cfg = DecodeConfig(**cfg_kw)
    m = DecodeModel(ctx, cfg, seed=21, quant=quant)
    host = ora.HostStepModel.from_recipe(m)
    toks = [11, 999 % cfg.vocab, 4242 % cfg.vocab, 7, 123 % cfg.vocab, 5]
    M = len(toks)
    B = m.verify_forward(toks, start, form)
    ctx.flush()
    got = m.read(B["logits"], M * cfg.vocab).reshape(M, cfg.vocab).astype(np.float64)
    idx = np.zeros(M, np.uint32)
    ctx._check(d.load_library().rt_download(ctx.handle, idx.ctypes.data, B["idx"], idx.nbytes))
    ref = np.stack([host.step(t, start + r, threads=8)[1] for r, t in enumerate(toks)])
    check_rows(got, ref.astype(np.float64), "verify rows")
    assert np.array_equal(idx, ora.argmax_rows_first(got.astype(np.float32), M))
    # the cache rows the pass wrote equal the ones the sequential steps wrote
    c = cfg
    for L, HL in zip(m.layers, host.layers):
        kc = m.read(L["kc"], c.kv_heads * c.max_seq * c.head_dim).reshape(c.kv_heads, c.max_seq, -1)
        hk = HL["kc"].reshape(c.kv_heads, c.max_seq, -1)
        seg, hseg = kc[:, start:start + M], hk[:, start:start + M]
        assert np.max(np.abs(seg - hseg)) <= 2e-3 * np.abs(hseg).max()
        assert np.array_equal(kc[:, :start], hk[:, :start])  # history untouched
    m.free()


def test_verify_draft_accepts_greedy_continuation(ctx):
    """Drafts equal to the greedy decode's own continuation are all
    accepted and the next token is the decode's next; a wrong draft stops
    acceptance there with the decode's token as the correction."""
    cfg = DecodeConfig(layers=2, max_seq=300)
    m = DecodeModel(ctx, cfg, seed=8)
    start, n = 200, 5
    snap = [(m.read(L["kc"], cfg.kv_heads * cfg.max_seq * cfg.head_dim),
             m.read(L["vc"], cfg.kv_heads * cfg.max_seq * cfg.head_dim)) for L in m.layers]

    def restore():
        for L, (kc, vc) in zip(m.layers, snap):
            for p, a in ((L["kc"], kc), (L["vc"], vc)):
                ctx._check(d.load_library().rt_upload(ctx.handle, p, a.ctypes.data, a.nbytes))

    prompt = 314
    m.set_token(prompt)
    seq, logits = [], []
    for i in range(n):
        m.step_fused(start + i)
        ctx.flush()
        logits.append(m.read(m.logits, cfg.vocab).astype(np.float64))
        seq.append(m.get_token())
    restore()
    B = m.verify_forward([prompt] + seq[:-1], start)
    ctx.flush()
    vl = m.read(B["logits"], n * cfg.vocab).reshape(n, cfg.vocab).astype(np.float64)
    check_rows(vl, np.stack(logits), "verify vs decode")
    # rows whose top-2 gap is clear of the tolerance must pick the decode's token
    ties = [r for r in range(n)
            if np.sort(logits[r])[-1] - np.sort(logits[r])[-2]
            <= 2e-3 * (logits[r].max() - logits[r].min())]
    assert not ties, ties  # this seed's greedy tokens are clear of the tolerance
    restore()
    assert m.verify_draft(prompt, seq[:-1], start) == (n - 1, seq[-1])
    restore()
    wrong = list(seq[:-1])
    wrong[2] = (wrong[2] + 1) % cfg.vocab
    assert m.verify_draft(prompt, wrong, start) == (2, seq[2])
    m.free()


# ───────────────────────── multi-row GEMVs ─────────────────────────

from gpu_helpers import check_close, device_weights  # noqa: E402
from test_gpu_fused import ffn_check  # noqa: E402

ROWS_FMTS = ["q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg", "q5kg", "q6kg"]


@pytest.mark.parametrize("fmt", ROWS_FMTS)
@pytest.mark.parametrize("rows,n,k", [(1, 300, 512), (5, 896, 896), (8, 130, 3584),
                                      (13, 70, 1024), (3, 64, 18944)])
def test_gemv_rows_plain_and_residual(ctx, fmt, rows, n, k):
    """y = x·Wᵀ and y = res + x·Wᵀ for rows activation rows: every output
    within the GEMV bound of the per-row oracle (13 rows: two launches; k =
    18944: K split over workgroups)."""
    if fmt in ("q4k", "q6k", "q5k", "q4kg", "q5kg", "q6kg") and k % 256:
        k = 1024
    wbuf, raw = device_weights(ctx, fmt, n, k, seed=rows + n)
    x = np.random.default_rng(rows).standard_normal((rows, k)).astype(np.float32)
    res = np.random.default_rng(rows + 1).standard_normal((rows, n)).astype(np.float32)
    yref, sabs = ora.gemv(fmt, raw, x, n, k)
    bx = ctx.buffer_from(x)
    y = ctx.new_buffer(4 * rows * n)
    d.gemv_rows_f32(ctx, fmt, wbuf, bx, y, rows, n, k)
    ctx.flush()
    check_close(y.read(np.float32, rows * n), yref.ravel(), sabs.ravel(), f"rows {fmt}")
    br = ctx.buffer_from(res)
    d.gemv_rows_add_f32(ctx, fmt, wbuf, bx, br, br, rows, n, k)  # in place
    ctx.flush()
    check_close(br.read(np.float32, rows * n), (yref + res).ravel(), sabs.ravel(),
                f"rows add {fmt}", extra=2 ** -24 * np.abs(res).ravel() * 2)


@pytest.mark.parametrize("fmt", ["q8_0", "q4k", "q6k", "q4kg", "q6kg", "q4_0"])
@pytest.mark.parametrize("rows", [4, 8, 11])
def test_qkv_bias_and_ffn_rows_with_norm(ctx, fmt, rows):
    """Q/K/V (+ bias) and gate+up+SiLU of rows RMS-normalised activation
    rows (0.5B head layout; K-quants at hidden 1024) against the oracle's
    rms_norm + GEMVs; the Q/K/V call with V skipped leaves V untouched."""
    h = 896 if fmt in ("q8_0", "q4_0") else 1024
    qd, kvd, ff = h, 128, 2 * h
    rng = np.random.default_rng(rows + 7)
    x = rng.standard_normal((rows, h)).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    eps = 1e-6
    xn = np.stack([ora.rms_norm(x[r], g, eps) for r in range(rows)]).astype(np.float32)
    ws = [device_weights(ctx, fmt, n_, h, seed=s) for n_, s in ((qd, 1), (kvd, 2), (kvd, 3))]
    bias = [rng.standard_normal(n_).astype(np.float16) * 0.1 for n_ in (qd, kvd, kvd)]
    outs = [ctx.new_buffer(4 * rows * n_) for n_ in (qd, kvd, kvd)]
    outs[2].write(np.full(rows * kvd, 7.0, np.float32))
    bx, bg = ctx.buffer_from(x), ctx.buffer_from(g)
    bb = [ctx.buffer_from(b) for b in bias]
    d.qkv_bias_rows_f32(ctx, fmt, ws[0][0], ws[1][0], None, bx, outs[0], outs[1], None,
                        bb[0], bb[1], None, rows, qd, kvd, h, gamma=bg, eps=eps)
    ctx.flush()
    for i, n_ in enumerate((qd, kvd)):
        yref, sabs = ora.gemv(fmt, ws[i][1], xn, n_, h)
        check_close(outs[i].read(np.float32, rows * n_),
                    (yref + bias[i].astype(np.float64)).ravel(), sabs.ravel(),
                    f"qkv rows {fmt} mat {i}")
    assert np.all(outs[2].read(np.float32, rows * kvd) == 7.0)
    wg, rg = device_weights(ctx, fmt, ff, h, seed=11)
    wu, ru = device_weights(ctx, fmt, ff, h, seed=12)
    act = ctx.new_buffer(4 * rows * ff)
    d.fused_ffn_rows_f32(ctx, fmt, wg, wu, bx, act, rows, ff, h, gamma=bg, eps=eps)
    ctx.flush()
    got = act.read(np.float32, rows * ff).reshape(rows, ff)
    for r in range(rows):
        g_ref, g_s = ora.gemv(fmt, rg, xn[r], ff, h)
        u_ref, u_s = ora.gemv(fmt, ru, xn[r], ff, h)
        ffn_check(got[r], g_ref, g_s, u_ref, u_s, f"ffn rows {fmt} r={r}")


@pytest.mark.parametrize("quant,cfg_kw,M", [
    (None, dict(layers=2, max_seq=600), 5),
    (None, dict(layers=2, max_seq=600), 40),
    (Q4K_M, dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, ff=1024, vocab=1000,
                 max_seq=300), 24),
])
def test_prefill_equals_sequential_steps(ctx, quant, cfg_kw, M):
    """prefill.rs:29-257: the prompt's last logits equal the CPU reference
    model's after stepping the prompt token by token from position 0, and
    decoding continues from the prefilled cache: the next fused step equals
    the reference's next step."""
    cfg = DecodeConfig(**cfg_kw)
    m = DecodeModel(ctx, cfg, seed=23, quant=quant)
    host = ora.HostStepModel.from_recipe(m)
    toks = [(37 * i + 11) % cfg.vocab for i in range(M)]
    got = m.prefill(toks).astype(np.float64)
    ref = None
    for pos, t in enumerate(toks):
        htok, ref = host.step(t, pos, threads=8)
    check_rows(got[None], ref.astype(np.float64)[None], "prefill last logits")
    tok = m.get_token()
    assert tok == ora.argmax(got.astype(np.float32)) or \
        ref[int(np.argmax(ref))] - ref[tok] <= 2e-3 * (ref.max() - ref.min())
    m.step_fused(M)
    ctx.flush()
    _, ref2 = host.step(tok, M, threads=8)
    check_rows(m.read(m.logits, cfg.vocab).astype(np.float64)[None], ref2.astype(np.float64)[None],
               "decode after prefill")
    m.free()
