"""A full Qwen2-shape decode step on the GPU (BASELINE config 2 shapes, fewer
layers where the CPU check needs it): the fused 5-launch sequence against the
reference's 10-launch sequence, and against a CPU composition of the oracle."""
import numpy as np
import pytest

import oracle_lib as ora
from runit_mac_amd import dispatch as d
from runit_mac_amd.decode import Q4K_M, DecodeConfig, DecodeModel

pytestmark = pytest.mark.gpu


def cpu_step(m: DecodeModel, tok: int, pos: int) -> np.ndarray:
    """forward.rs:1494-1771 on the CPU with the oracle (f64 arithmetic), every
    matrix decoded in its own format (the model's per-layer routing)."""
    c = m.cfg
    h, qd, kvd, hd = c.hidden, c.q_dim, c.kv_dim, c.head_dim

    def rdw(p, n, k, fmt):
        nb = d.weight_bytes(fmt, n, k)
        return m.read(p, (nb + 3) // 4).view(np.uint8)[:nb]

    def gemv(fmt, p, x, n, k):
        y, _ = ora.gemv(fmt, rdw(p, n, k, fmt), x.astype(np.float32), n, k)
        return y

    emb = rdw(m.embd, c.vocab, h, m.embd_fmt)
    row = len(emb) // c.vocab
    x = ora.dequant(m.embd_fmt, emb[tok * row:(tok + 1) * row]).astype(np.float64)
    return cpu_step_from(m, x, pos, emb)


def cpu_step_from(m: DecodeModel, x: np.ndarray, pos: int, emb=None) -> np.ndarray:
    """cpu_step from a given embedding row x (f64)."""
    c = m.cfg
    h, qd, kvd, hd = c.hidden, c.q_dim, c.kv_dim, c.head_dim

    def rdw(p, n, k, fmt):
        nb = d.weight_bytes(fmt, n, k)
        return m.read(p, (nb + 3) // 4).view(np.uint8)[:nb]

    def gemv(fmt, p, x, n, k):
        y, _ = ora.gemv(fmt, rdw(p, n, k, fmt), x.astype(np.float32), n, k)
        return y

    for L, F in zip(m.layers, m.fmts):
        g = m.read(L["attn_norm"], h)
        xn = ora.rms_norm(x.astype(np.float32), g, c.eps)
        outs = []
        for role, w, b, n in (("q", L["wq"], L["bq"], qd), ("k", L["wk"], L["bk"], kvd),
                              ("v", L["wv"], L["bv"], kvd)):
            y = gemv(F[role], w, xn, n, h)
            bias = m.read(b, n // 2 + 1).view(np.float16)[:n].astype(np.float64)
            outs.append(y + bias)
        q, k, v = outs
        q = ora.rope(q, c.heads, hd, pos, c.theta)
        k = ora.rope(k, c.kv_heads, hd, pos, c.theta)
        kc = m.read(L["kc"], c.kv_heads * c.max_seq * hd).reshape(c.kv_heads, c.max_seq, hd)
        vc = m.read(L["vc"], c.kv_heads * c.max_seq * hd).reshape(c.kv_heads, c.max_seq, hd)
        kc[:, pos] = k.reshape(c.kv_heads, hd)
        vc[:, pos] = v.reshape(c.kv_heads, hd)
        att = ora.attention(q, kc, vc, c.heads, c.kv_heads, hd, pos + 1, c.max_seq)
        x = x + gemv(F["o"], L["wo"], att, h, qd)
        xn = ora.rms_norm(x.astype(np.float32), m.read(L["ffn_norm"], h), c.eps)
        gt = gemv(F["gate"], L["wg"], xn, c.ff, h)
        up = gemv(F["up"], L["wu"], xn, c.ff, h)
        act = gt / (1.0 + np.exp(-gt)) * up
        x = x + gemv(F["down"], L["wd"], act, h, c.ff)
    xn = ora.rms_norm(x.astype(np.float32), m.read(m.final_norm, h), c.eps)
    if m.lm_head == m.embd:
        logits, _ = ora.gemv(m.embd_fmt, emb, xn.astype(np.float32), c.vocab, h)
    else:
        logits = gemv(m.lm_fmt, m.lm_head, xn, c.vocab, h)
    return logits


def snapshot_cache(m):
    c = m.cfg
    return [(m.read(L["kc"], c.kv_heads * c.max_seq * c.head_dim),
             m.read(L["vc"], c.kv_heads * c.max_seq * c.head_dim)) for L in m.layers]


def restore_cache(m, snap):
    for L, (kc, vc) in zip(m.layers, snap):
        for p, a in ((L["kc"], kc), (L["vc"], vc)):
            m.ctx._check(d.load_library().rt_upload(m.ctx.handle, p, a.ctypes.data, a.nbytes))


@pytest.mark.parametrize("layers", [2])
def test_step_matches_cpu_oracle(ctx, layers):
    cfg = DecodeConfig(layers=layers, max_seq=600)
    m = DecodeModel(ctx, cfg, seed=3)
    tok, pos = 1234, 511
    snap = snapshot_cache(m)
    ref = cpu_step(m, tok, pos)
    for fused in (False, True):
        restore_cache(m, snap)
        m.set_token(tok)
        (m.step_fused if fused else m.step_reference)(pos)
        ctx.flush()
        got = m.read(m.logits, cfg.vocab).astype(np.float64)
        # errors of ~1e-4·Σ|w·x| per GEMV compound over the layers; logits must
        # agree to 1e-3 of their spread, and the greedy token must be the same
        assert np.max(np.abs(got - ref)) <= 1e-3 * (ref.max() - ref.min()), \
            (fused, np.max(np.abs(got - ref)))
        assert m.get_token() == int(np.argmax(ref)) == ora.argmax(got.astype(np.float32))
    m.free()


def test_q4k_m_mix_step_matches_cpu_oracle(ctx):
    """A Q4_K_M-style model (Q/K/O/gate/up Q4_K; V, down and the LM head
    Q6_K; head size 128): the fused step routes each matrix to its format's
    kernels, eagerly and replayed as a graph."""
    cfg = DecodeConfig(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, ff=1024,
                       vocab=1000, max_seq=300)
    m = DecodeModel(ctx, cfg, seed=11, quant=Q4K_M)
    with pytest.raises(ValueError):
        m.step_reference(0)
    tok, pos = 77, 257
    snap = snapshot_cache(m)
    ref = cpu_step(m, tok, pos)
    restore_cache(m, snap)
    m.set_token(tok)
    g = m.capture(pos, fused=True)
    for replay in range(3):
        restore_cache(m, snap)
        m.set_token(tok)
        if replay == 0:
            m.step_fused(pos)
        else:
            g.launch()
        ctx.flush()
        got = m.read(m.logits, cfg.vocab).astype(np.float64)
        assert np.max(np.abs(got - ref)) <= 1e-3 * (ref.max() - ref.min()), \
            (replay, np.max(np.abs(got - ref)))
        assert m.get_token() == int(np.argmax(ref))
    m.free()


def check_logits(got, ref, what):
    """Logits within 1e-3 of the oracle's spread; the greedy token equal to
    the oracle's unless its top-2 gap is inside that tolerance (then the GPU's
    token must be one of the tied candidates)."""
    tol = 1e-3 * (ref.max() - ref.min())
    err = np.max(np.abs(got - ref))
    assert err <= tol, (what, err, tol)
    top = int(np.argmax(ref))
    tok = ora.argmax(got.astype(np.float32))
    if tok != top:
        assert ref[top] - ref[tok] <= 2 * tol, (what, tok, top, ref[top] - ref[tok])
    return tok


def test_full_depth_step_matches_cpu_oracle(ctx):
    """BASELINE config 2 as specified: 24 layers at 0.5B shapes, kv_len 512.
    The reference's 10-launch sequence (eager) and the fused 5-launch
    sequence (captured graph, replayed 3 times with the cache restored) are
    both compared with the f64 oracle composition of forward.rs:1494-1771."""
    cfg = DecodeConfig()
    m = DecodeModel(ctx, cfg, seed=5)
    tok, pos = 42, 511
    snap = snapshot_cache(m)
    ref = cpu_step(m, tok, pos)
    restore_cache(m, snap)
    m.set_token(tok)
    m.step_reference(pos)
    ctx.flush()
    t_ref = check_logits(m.read(m.logits, cfg.vocab).astype(np.float64), ref, "reference seq")
    assert m.get_token() == t_ref
    restore_cache(m, snap)
    m.set_token(tok)
    g = m.capture(pos, fused=True)
    for replay in range(3):
        restore_cache(m, snap)
        m.set_token(tok)
        g.launch()
        ctx.flush()
        t = check_logits(m.read(m.logits, cfg.vocab).astype(np.float64), ref, f"replay {replay}")
        assert m.get_token() == t
    del g
    # the CPU baseline's model (rebuilt on the host from the seeds) computes
    # the same step: the f32 reference CPU path lands on the oracle too
    host = ora.HostStepModel.from_recipe(m)
    htok, hlog = host.step(tok, pos, threads=8)
    assert check_logits(hlog.astype(np.float64), ref, "host f32 step") == htok == t
    m.free()


@pytest.mark.parametrize("quant", [None, Q4K_M])
def test_host_twin_rebuilds_device_model_bytes(ctx, quant):
    """Every tensor the CPU baseline's host model regenerates from the decode
    model's recipe equals the device's bytes."""
    cfg = DecodeConfig(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, ff=1024,
                       vocab=1000, max_seq=64)
    m = DecodeModel(ctx, cfg, seed=4, quant=quant)
    host = ora.HostStepModel.from_recipe(m)
    for L, HL in zip(m.layers, host.layers):
        for key, arr in HL.items():
            dev = m.read(L[key], (arr.nbytes + 3) // 4).view(np.uint8)[:arr.nbytes]
            assert np.array_equal(dev, arr.view(np.uint8)), key
    m.free()


@pytest.mark.gpu
def test_step_fused_counts_its_launches(ctx):
    """step_fused reports the launches the library enqueued (rt_launch_count):
    for the 2-layer 0.5B-shape model, 1 embedding + 5 per layer + norm-fused
    LM head + argmax."""
    from runit_mac_amd.decode import DecodeConfig, DecodeModel
    m = DecodeModel(ctx, DecodeConfig(layers=2), seed=3)
    m.set_token(1)
    before = d.launch_count(ctx)
    n = m.step_fused(5)
    ctx.flush()
    assert n == d.launch_count(ctx) - before == 1 + 5 * 2 + 2


def test_full_depth_q4k_m_7b_step_matches_cpu_oracle(ctx):
    """BASELINE config 4 as one decode step at its real shapes: 28 layers of
    Qwen2.5-7B (hidden 3584, 28/4 heads × 128, ff 18944, vocab 152064) in the
    Q4_K_M mix (Q/K/O/gate/up Q4_K; V, down and the LM head Q6_K), kv_len
    512 — the model, position and graph that bench.py's q4k_m_7b_decode
    times — against the f64 oracle composition of forward.rs:1470-1787.
    The captured graph is replayed twice with the cache restored."""
    cfg = DecodeConfig(layers=28, hidden=3584, heads=28, kv_heads=4, head_dim=128, ff=18944,
                       vocab=152064, max_seq=1024)
    m = DecodeModel(ctx, cfg, seed=9, quant=Q4K_M)
    tok, pos = 1, 511
    snap = snapshot_cache(m)
    print(f"[7B Q4_K_M step] oracle, {cfg.layers} layers", flush=True)
    ref = cpu_step(m, tok, pos)
    restore_cache(m, snap)
    m.set_token(tok)
    g = m.capture(pos, fused=True)
    for replay in range(2):
        restore_cache(m, snap)
        m.set_token(tok)
        print(f"[7B Q4_K_M step] replay {replay}", flush=True)
        g.launch()
        ctx.flush()
        t = check_logits(m.read(m.logits, cfg.vocab).astype(np.float64), ref, f"7B replay {replay}")
        assert m.get_token() == t
    del g
    m.free()
