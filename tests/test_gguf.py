"""GGUF reader (rt_gguf_*, C++) and model config: CPU tests, no GPU needed.

Known answers come from the reference's own tests: the minimal GGUF of
crates/gguf/src/parser.rs:240-345 (parse, bad magic, bad version, Q4_K data
size, alignment) and the Qwen2 metadata of crates/engine/src/config.rs:
308-356."""
import os

import numpy as np
import pytest

import gguf_writer as gw
from runit_mac_amd import gguf as G


def write(tmp_path, data, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_reference_minimal_gguf(tmp_path):
    f = G.GgufFile(write(tmp_path, gw.reference_test_gguf()))
    assert f.version == 3
    assert len(f.tensors) == 1
    t = f.tensors[0]
    assert (t.name, t.shape, t.dtype_name, t.offset) == ("test.weight", (4, 8), "F32", 0)
    assert f.data_offset % 32 == 0
    assert f.metadata["general.architecture"] == "qwen2"
    assert np.array_equal(f.tensor_bytes("test.weight").view(np.float32), np.arange(32))


def test_reference_invalid_magic_and_version(tmp_path):
    data = bytearray(gw.reference_test_gguf())
    data[0] = 0xFF
    with pytest.raises(G.InvalidMagic):
        G.GgufFile(write(tmp_path, bytes(data), "a.gguf"))
    data = bytearray(gw.reference_test_gguf())
    data[4:8] = (99).to_bytes(4, "little")
    with pytest.raises(G.UnsupportedVersion, match="99"):
        G.GgufFile(write(tmp_path, bytes(data), "b.gguf"))


def test_reference_q4k_data_size(tmp_path):
    # GgufTensorInfo { shape [256, 512], Q4K } → 512 blocks × 144 bytes
    raw = bytes(512 * 144)
    f = G.GgufFile(write(tmp_path, gw.build([], [("q", [256, 512], 12, raw)])))
    assert f.tensors[0].nbytes == 512 * 144


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_alignment_and_offsets(tmp_path, alignment):
    a = np.arange(10, dtype=np.float32)
    b = np.arange(7, dtype=np.float16)
    f = G.GgufFile(write(tmp_path, gw.build([("general.architecture", gw.STR, "x")],
                                            [("a", [10], 0, a.tobytes()),
                                             ("b", [7], 1, b.tobytes())], alignment=alignment)))
    al = alignment or 32
    assert f.alignment == al and f.data_offset % al == 0
    assert f.tensor("b").offset % al == 0
    assert np.array_equal(f.tensor_bytes("a").view(np.float32), a)
    assert np.array_equal(f.tensor_bytes("b").view(np.float16), b)


def test_every_metadata_type(tmp_path):
    md = [("u8", gw.U8, 200), ("i8", gw.I8, -5), ("u16", gw.U16, 60000), ("i16", gw.I16, -300),
          ("u32", gw.U32, 4000000000), ("i32", gw.I32, -7), ("f32", gw.F32, 0.25),
          ("b", gw.BOOL, True), ("s", gw.STR, "héllo"), ("u64", gw.U64, 2 ** 40),
          ("i64", gw.I64, -(2 ** 40)), ("f64", gw.F64, 1e300),
          ("arr_i", gw.ARR, (gw.I32, [1, -2, 3])), ("arr_f", gw.ARR, (gw.F32, [0.5, 1.5])),
          ("arr_s", gw.ARR, (gw.STR, ["a", "", "ccc"])),
          ("nested", gw.ARR, (gw.ARR, [(gw.U8, [1, 2]), (gw.U8, [])]))]
    f = G.GgufFile(write(tmp_path, gw.build(md, [], version=2)))
    m = f.metadata
    assert f.version == 2
    assert (m["u8"], m["i8"], m["u16"], m["i16"], m["u32"], m["i32"]) == \
        (200, -5, 60000, -300, 4000000000, -7)
    assert m["f32"] == 0.25 and m["b"] is True and m["s"] == "héllo"
    assert (m["u64"], m["i64"], m["f64"]) == (2 ** 40, -(2 ** 40), 1e300)
    assert m["arr_i"] == [1, -2, 3] and m["arr_f"] == [0.5, 1.5] and m["arr_s"] == ["a", "", "ccc"]
    assert len(m["nested"]) == 2
    assert f.metadata_types["u32"] == gw.U32 and f.metadata_types["arr_s"] == gw.ARR


def test_errors(tmp_path):
    good = gw.build([("k", gw.STR, "v")], [("t", [4], 0, bytes(16))])
    with pytest.raises(G.UnexpectedEof):  # truncated inside the tensor table
        G.GgufFile(write(tmp_path, good[:60], "t1.gguf"))
    with pytest.raises(G.UnknownDtype):
        G.GgufFile(write(tmp_path, gw.build([], [("t", [4], 99, bytes(16))]), "t2.gguf"))
    bad_type = bytearray(gw.build([("k", gw.U32, 1)], []))
    bad_type[24 + 8 + 1: 24 + 8 + 1 + 4] = (77).to_bytes(4, "little")  # value type after key "k"
    with pytest.raises(G.UnknownMetadataType):
        G.GgufFile(write(tmp_path, bytes(bad_type), "t3.gguf"))
    bad_utf8 = gw.build([("k", gw.STR, "ok")], []).replace(b"ok", b"\xff\xfe")
    with pytest.raises(G.InvalidUtf8):
        G.GgufFile(write(tmp_path, bad_utf8, "t4.gguf"))
    with pytest.raises(G.DataRegionOverflow):  # tensor data cut off
        G.GgufFile(write(tmp_path, good[:-24], "t5.gguf"))  # 16 data bytes + 16 padding
    with pytest.raises(G.Io):
        G.GgufFile(str(tmp_path / "missing.gguf"))


def qwen2_metadata():
    """config.rs:311-326."""
    return [("general.architecture", gw.STR, "qwen2"), ("qwen2.embedding_length", gw.U32, 3584),
            ("qwen2.feed_forward_length", gw.U32, 18944), ("qwen2.block_count", gw.U32, 28),
            ("qwen2.attention.head_count", gw.U32, 28),
            ("qwen2.attention.head_count_kv", gw.U32, 4),
            ("qwen2.attention.layer_norm_rms_epsilon", gw.F32, 1e-6),
            ("qwen2.context_length", gw.U32, 32768), ("tokenizer.ggml.token_count", gw.U32, 152064),
            ("tokenizer.ggml.bos_token_id", gw.U32, 151643),
            ("tokenizer.ggml.eos_token_id", gw.U32, 151645)]


def test_reference_qwen2_config(tmp_path):
    """config.rs:328-345 through a real file."""
    f = G.GgufFile(write(tmp_path, gw.build(qwen2_metadata(), [])))
    cfg = G.ModelConfig.from_metadata(f.metadata, f.metadata_types)
    assert (cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers) == (3584, 18944, 28)
    assert (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) == (28, 4, 128)
    assert cfg.vocab_size == 152064 and abs(cfg.rope_theta - 1e6) < 1.0
    assert (cfg.bos_token_id, cfg.eos_token_id) == (151643, 151645)
    assert abs(cfg.rms_norm_eps - 1e-6) < 1e-12 and cfg.activation == "silu_mul"


def test_reference_missing_required_field(tmp_path):
    md = [kv for kv in qwen2_metadata() if kv[0] != "qwen2.embedding_length"]
    f = G.GgufFile(write(tmp_path, gw.build(md, [])))
    with pytest.raises(G.LoadError, match="missing metadata"):
        G.ModelConfig.from_metadata(f.metadata, f.metadata_types)


def test_config_fallbacks(tmp_path):
    # vocab from the token list; explicit head_dim; u16 ints are not accepted
    # for required keys (req_u32 takes u32 / u64 / i32 only)
    md = [kv for kv in qwen2_metadata() if kv[0] != "tokenizer.ggml.token_count"]
    md += [("tokenizer.ggml.tokens", gw.ARR, (gw.STR, ["a", "b", "c"])),
           ("qwen2.attention.key_length", gw.U32, 64)]
    f = G.GgufFile(write(tmp_path, gw.build(md, [])))
    cfg = G.ModelConfig.from_metadata(f.metadata, f.metadata_types)
    assert cfg.vocab_size == 3 and cfg.head_dim == 64
    md2 = [kv if kv[0] != "qwen2.block_count" else ("qwen2.block_count", gw.U16, 28)
           for kv in qwen2_metadata()]
    f2 = G.GgufFile(write(tmp_path, gw.build(md2, []), "u16.gguf"))
    with pytest.raises(G.LoadError):
        G.ModelConfig.from_metadata(f2.metadata, f2.metadata_types)


def test_qwen2_names_tied_head(tmp_path):
    f = G.GgufFile(write(tmp_path, gw.build([], [("token_embd.weight", [32, 2], 0, bytes(256))])))
    names = G.qwen2_tensor_names(1, f)
    assert names["output"] == "token_embd.weight"
    assert names["blk.0.attn_q.bias"] == "blk.0.attn_q.bias"
