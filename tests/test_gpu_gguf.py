"""Qwen2-shaped models written as GGUF, loaded through the C++ reader
(rt_gguf_*) into the decode engine, decoded on the GPU and checked against the
CPU oracle step; the uploaded tensors are compared with the file's bytes.

Besides Q8_0 files, mixed files route every tensor by its own dtype, as the
reference's upload_weight_wb does (forward.rs:1137-1222): a Q4_K_M-style
file (Q4_K matrices, V and down in Q6_K in some layers only, Q4_K embedding,
Q6_K output), a Q5_K_M-style file (Q5_K / Q6_K, whose mixed Q/K/V take the
reference's separate-dispatch fallback) and a Q4_0 / Q5_0 file, in ggml's
block layouts (upstream files) and in the reference's."""
import numpy as np
import pytest

import gguf_writer as gw
import oracle_lib as ora
from runit_mac_amd import gguf as G
from runit_mac_amd.decode import DecodeModel
from test_gpu_step import cpu_step

pytestmark = pytest.mark.gpu

H, HEADS, KVH, HD, FF, VOCAB, LAYERS = 256, 4, 2, 64, 512, 320, 2


def make_model(path, tied: bool):
    rng = np.random.default_rng(5)
    seed = [100]

    def q8(n, k):
        seed[0] += 1
        return ora.synth_weights("q8_0", n, k, seed[0])

    def f32(n, mean, std):
        return (mean + std * rng.standard_normal(n)).astype(np.float32)

    q, kv = HEADS * HD, KVH * HD
    T = []
    for i in range(LAYERS):
        b = f"blk.{i}."
        T += [(b + "attn_norm.weight", [H], 0, f32(H, 1, 0.02).tobytes()),
              (b + "attn_q.weight", [H, q], 8, q8(q, H)), (b + "attn_k.weight", [H, kv], 8, q8(kv, H)),
              (b + "attn_v.weight", [H, kv], 8, q8(kv, H)),
              (b + "attn_q.bias", [q], 0, f32(q, 0, 0.02).tobytes()),
              (b + "attn_k.bias", [kv], 0, f32(kv, 0, 0.02).tobytes()),
              (b + "attn_v.bias", [kv], 0, f32(kv, 0, 0.02).tobytes()),
              (b + "attn_output.weight", [q, H], 8, q8(H, q)),
              (b + "ffn_norm.weight", [H], 0, f32(H, 1, 0.02).tobytes()),
              (b + "ffn_gate.weight", [H, FF], 8, q8(FF, H)), (b + "ffn_up.weight", [H, FF], 8, q8(FF, H)),
              (b + "ffn_down.weight", [FF, H], 8, q8(H, FF))]
    T += [("output_norm.weight", [H], 0, f32(H, 1, 0.02).tobytes()),
          ("token_embd.weight", [H, VOCAB], 8, q8(VOCAB, H))]
    if not tied:
        T.append(("output.weight", [H, VOCAB], 8, q8(VOCAB, H)))
    md = [("general.architecture", gw.STR, "qwen2"), ("qwen2.embedding_length", gw.U32, H),
          ("qwen2.feed_forward_length", gw.U32, FF), ("qwen2.block_count", gw.U32, LAYERS),
          ("qwen2.attention.head_count", gw.U32, HEADS),
          ("qwen2.attention.head_count_kv", gw.U32, KVH),
          ("qwen2.attention.layer_norm_rms_epsilon", gw.F32, 1e-6),
          ("qwen2.rope.freq_base", gw.F32, 1e6), ("tokenizer.ggml.token_count", gw.U32, VOCAB)]
    gw.write(path, md, [(n, dims, dt, bytes(raw)) for n, dims, dt, raw in T])
    return {n: raw for n, dims, dt, raw in T}


@pytest.mark.parametrize("tied", [True, False])
def test_gguf_model_decodes_like_the_oracle(ctx, tmp_path, tied):
    path = str(tmp_path / "qwen2_tiny.gguf")
    raw = make_model(path, tied)
    f = G.GgufFile(path)
    m = DecodeModel.from_gguf(ctx, f, max_seq=64)
    c = m.cfg
    assert (c.layers, c.hidden, c.heads, c.kv_heads, c.head_dim, c.ff, c.vocab) == \
        (LAYERS, H, HEADS, KVH, HD, FF, VOCAB)
    # the device holds the file's bytes (biases converted f32 → f16, RNE)
    L = m.layers[1]
    wq = m.read(L["wq"], len(raw["blk.1.attn_q.weight"]) // 4).view(np.uint8)
    assert np.array_equal(wq, np.frombuffer(raw["blk.1.attn_q.weight"], np.uint8))
    bq = m.read(L["bq"], HEADS * HD // 2).view(np.float16)
    assert np.array_equal(bq, np.frombuffer(raw["blk.1.attn_q.bias"], np.float32).astype(np.float16))
    assert (m.lm_head == m.embd) == tied
    # three greedy steps from an empty cache, each against the oracle
    tok = 7
    for pos in range(3):
        ref = cpu_step(m, tok, pos)
        m.set_token(tok)
        m.step_fused(pos)
        ctx.flush()
        got = m.read(m.logits, VOCAB).astype(np.float64)
        assert np.max(np.abs(got - ref)) <= 1e-3 * (ref.max() - ref.min()), pos
        nxt = m.get_token()
        assert nxt == int(np.argmax(ref))
        tok = nxt
    m.free()
    f.close()


# GGUF dtype ids (crates/gguf/src/types.rs:46-76)
DT = {"F32": 0, "F16": 1, "Q4_0": 2, "Q5_0": 6, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
LAYOUT_FMT = {"ggml": {"Q8_0": "q8_0", "Q4_0": "q4_0g", "Q4_K": "q4kg", "Q5_0": "q5_0",
                       "Q5_K": "q5kg", "Q6_K": "q6kg"},
              "reference": {"Q8_0": "q8_0", "Q4_0": "q4_0", "Q4_K": "q4k", "Q5_0": "q5_0",
                            "Q5_K": "q5k", "Q6_K": "q6k"}}
MIXES = {
    # per layer: dtype of q, k, v, o, gate, up, down; then embedding, output
    "q4_k_m": ([("Q4_K", "Q4_K", "Q6_K", "Q4_K", "Q4_K", "Q4_K", "Q6_K"),
                ("Q4_K", "Q4_K", "Q4_K", "Q4_K", "Q4_K", "Q4_K", "Q4_K")], "Q4_K", "Q6_K"),
    "q5_k_m": ([("Q5_K", "Q5_K", "Q6_K", "Q5_K", "Q5_K", "Q5_K", "Q6_K"),
                ("Q5_K", "Q5_K", "Q5_K", "Q5_K", "Q5_K", "Q5_K", "Q5_K")], "Q5_K", "Q6_K"),
    "q4_0_q5_0": ([("Q4_0", "Q4_0", "Q8_0", "Q4_0", "Q4_0", "Q4_0", "Q5_0"),
                   ("Q5_0", "Q5_0", "Q5_0", "Q4_0", "Q5_0", "Q5_0", "Q4_0")], "F16", "Q8_0"),
}


def make_mixed_model(path, mix, layout):
    layers_dt, embd_dt, out_dt = MIXES[mix]
    fmt = LAYOUT_FMT[layout]
    rng = np.random.default_rng(9)
    seed = [300]

    def wq(dt, n, k):
        seed[0] += 1
        if dt == "F16":
            return (0.02 * rng.standard_normal(n * k)).astype(np.float16).tobytes()
        return ora.synth_weights(fmt[dt], n, k, seed[0]).tobytes()

    def f32(n, mean, std):
        return (mean + std * rng.standard_normal(n)).astype(np.float32).tobytes()

    q, kv = HEADS * HD, KVH * HD
    T = []
    for i, dts in enumerate(layers_dt):
        b = f"blk.{i}."
        dq, dk, dv, do, dg, du, dd = dts
        T += [(b + "attn_norm.weight", [H], 0, f32(H, 1, 0.02)),
              (b + "attn_q.weight", [H, q], DT[dq], wq(dq, q, H)),
              (b + "attn_k.weight", [H, kv], DT[dk], wq(dk, kv, H)),
              (b + "attn_v.weight", [H, kv], DT[dv], wq(dv, kv, H)),
              (b + "attn_q.bias", [q], 0, f32(q, 0, 0.02)),
              (b + "attn_k.bias", [kv], 0, f32(kv, 0, 0.02)),
              (b + "attn_v.bias", [kv], 0, f32(kv, 0, 0.02)),
              (b + "attn_output.weight", [q, H], DT[do], wq(do, H, q)),
              (b + "ffn_norm.weight", [H], 0, f32(H, 1, 0.02)),
              (b + "ffn_gate.weight", [H, FF], DT[dg], wq(dg, FF, H)),
              (b + "ffn_up.weight", [H, FF], DT[du], wq(du, FF, H)),
              (b + "ffn_down.weight", [FF, H], DT[dd], wq(dd, H, FF))]
    T += [("output_norm.weight", [H], 0, f32(H, 1, 0.02)),
          ("token_embd.weight", [H, VOCAB], DT[embd_dt], wq(embd_dt, VOCAB, H)),
          ("output.weight", [H, VOCAB], DT[out_dt], wq(out_dt, VOCAB, H))]
    md = [("general.architecture", gw.STR, "qwen2"), ("qwen2.embedding_length", gw.U32, H),
          ("qwen2.feed_forward_length", gw.U32, FF), ("qwen2.block_count", gw.U32, LAYERS),
          ("qwen2.attention.head_count", gw.U32, HEADS),
          ("qwen2.attention.head_count_kv", gw.U32, KVH),
          ("qwen2.attention.layer_norm_rms_epsilon", gw.F32, 1e-6),
          ("qwen2.rope.freq_base", gw.F32, 1e6), ("tokenizer.ggml.token_count", gw.U32, VOCAB)]
    gw.write(path, md, T)
    return {n: raw for n, dims, dt, raw in T}


@pytest.mark.parametrize("layout", ["ggml", "reference"])
@pytest.mark.parametrize("mix", list(MIXES))
def test_mixed_gguf_routes_each_tensor_by_dtype(ctx, tmp_path, mix, layout):
    if mix == "q4_0_q5_0" and layout == "reference":
        pytest.skip("Q4_0 / Q5_0 / Q8_0: covered by the ggml run (Q5_0, Q8_0 layouts agree)")
    path = str(tmp_path / f"qwen2_{mix}_{layout}.gguf")
    raw = make_mixed_model(path, mix, layout)
    f = G.GgufFile(path)
    m = DecodeModel.from_gguf(ctx, f, max_seq=64, layout=layout)
    layers_dt, embd_dt, out_dt = MIXES[mix]
    fmt = LAYOUT_FMT[layout]
    roles = ("q", "k", "v", "o", "gate", "up", "down")
    for F, dts in zip(m.fmts, layers_dt):
        assert F == {r: fmt[dt] for r, dt in zip(roles, dts)}
    assert m.lm_fmt == fmt[out_dt] and m.lm_head != m.embd
    # the device holds the file's bytes for a Q6_K / Q5_K / Q5_0 matrix
    wd = m.read(m.layers[0]["wd"], len(raw["blk.0.ffn_down.weight"]) // 4 + 1).view(np.uint8)
    assert np.array_equal(wd[:len(raw["blk.0.ffn_down.weight"])],
                          np.frombuffer(raw["blk.0.ffn_down.weight"], np.uint8))
    tok = 11
    for pos in range(3):
        if embd_dt == "F16":
            row = np.frombuffer(raw["token_embd.weight"], np.float16)[tok * H:(tok + 1) * H]
            ref = _cpu_step_embedded(m, row.astype(np.float64), pos)
        else:
            ref = cpu_step(m, tok, pos)
        m.set_token(tok)
        n = m.step_fused(pos)
        ctx.flush()
        got = m.read(m.logits, VOCAB).astype(np.float64)
        assert np.max(np.abs(got - ref)) <= 1e-3 * (ref.max() - ref.min()), (mix, layout, pos)
        nxt = m.get_token()
        assert nxt == int(np.argmax(ref)), (mix, layout, pos)
        tok = nxt
    assert n == m.launches_fused() > 0
    m.free()
    f.close()


def _cpu_step_embedded(m, x0, pos):
    """cpu_step with the embedding row given (F16 tables: the row's halves)."""
    import test_gpu_step as ts
    return ts.cpu_step_from(m, x0, pos)
