"""A Qwen2-shaped Q8_0 model written as GGUF, loaded through the C++ reader
(rt_gguf_*) into the decode engine, decoded on the GPU and checked against the
CPU oracle step; the uploaded tensors are compared with the file's bytes."""
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
