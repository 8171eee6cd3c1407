"""GGUF files over the C ABI (rt_gguf_*): the wire format in front of the path.

* `GgufFile` mirrors the reference's `crates/gguf` parser output (`GgufFile`
  with version, metadata, tensor infos, data offset; parser.rs:22-57) and the
  engine loader's zero-copy tensor access (crates/engine/src/loader.rs:
  124-218).  Parsing and the read-only mapping are done in C++
  (csrc/gguf.cpp); errors raise `GgufError` subclasses named after the
  reference's `GgufError` variants (crates/gguf/src/error.rs:4-31).
* `ModelConfig.from_metadata` restates crates/engine/src/config.rs:96-265.
* `qwen2_tensor_names` gives the tensor names the engine's `Executor::new`
  uploads (forward.rs:1239-1330), including the tied LM head
  (forward.rs:1271-1276).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import dispatch as d

# GgufDtype ids (crates/gguf/src/types.rs:46-76) → name
DTYPES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1",
          10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K",
          16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S",
          22: "IQ2_S", 23: "IQ4_XS", 24: "I8", 25: "I16", 26: "I32", 27: "I64", 28: "F64",
          29: "IQ1_M", 30: "BF16"}


class GgufError(Exception):
    """Base of the GgufError variants."""


class Io(GgufError):
    pass


class InvalidMagic(GgufError):
    pass


class UnsupportedVersion(GgufError):
    pass


class UnknownDtype(GgufError):
    pass


class UnknownMetadataType(GgufError):
    pass


class UnexpectedEof(GgufError):
    pass


class InvalidUtf8(GgufError):
    pass


class DataRegionOverflow(GgufError):
    pass


_ERRORS = {16: Io, 17: InvalidMagic, 18: UnsupportedVersion, 19: UnknownDtype,
           20: UnknownMetadataType, 21: UnexpectedEof, 22: InvalidUtf8, 23: DataRegionOverflow}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: tuple
    dtype: int
    offset: int  # within the data region
    nbytes: int

    @property
    def dtype_name(self) -> str:
        return DTYPES.get(self.dtype, str(self.dtype))

    def num_elements(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return max(n, 1)


class GgufFile:
    """A parsed, memory-mapped GGUF file."""

    def __init__(self, path: str):
        self.lib = d.load_library()
        h = ctypes.c_void_p()
        st = self.lib.rt_gguf_open(str(path).encode(), ctypes.byref(h))
        if st != 0:
            raise _ERRORS.get(st, GgufError)(self.lib.rt_gguf_last_error().decode())
        self.handle = h.value
        self.version = int(self.lib.rt_gguf_version(self.handle))
        self.alignment = int(self.lib.rt_gguf_alignment(self.handle))
        self.data_offset = int(self.lib.rt_gguf_data_offset(self.handle))
        self.tensors = [self._tensor(i) for i in range(self.lib.rt_gguf_tensor_count(self.handle))]
        self._by_name = {t.name: i for i, t in enumerate(self.tensors)}
        self.metadata = {}
        self.metadata_types = {}  # key → GGUF value type id
        for i in range(self.lib.rt_gguf_meta_count(self.handle)):
            key, val, t = self._meta(i)
            self.metadata[key] = val
            self.metadata_types[key] = t

    def _tensor(self, i: int) -> TensorInfo:
        name = ctypes.c_char_p()
        nd = ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 8)()
        dt = ctypes.c_uint32()
        off = ctypes.c_uint64()
        nb = ctypes.c_uint64()
        self.lib.rt_gguf_tensor_info(self.handle, i, ctypes.byref(name), ctypes.byref(nd), dims,
                                     ctypes.byref(dt), ctypes.byref(off), ctypes.byref(nb))
        return TensorInfo(name.value.decode(), tuple(int(dims[k]) for k in range(nd.value)),
                          int(dt.value), int(off.value), int(nb.value))

    def _meta(self, i: int):
        key = ctypes.c_char_p()
        t = ctypes.c_uint32()
        et = ctypes.c_uint32()
        cnt = ctypes.c_uint64()
        self.lib.rt_gguf_meta_info(self.handle, i, ctypes.byref(key), ctypes.byref(t),
                                   ctypes.byref(et), ctypes.byref(cnt))
        t = t.value
        if t in (6, 12):
            v = ctypes.c_double()
            self.lib.rt_gguf_meta_float(self.handle, i, ctypes.byref(v))
            val = v.value
        elif t == 8:
            val = self.lib.rt_gguf_meta_string(self.handle, i).decode()
        elif t == 9:
            n = cnt.value
            if et.value == 8:
                val = []
                for k in range(n):
                    p = ctypes.c_void_p()
                    ln = ctypes.c_uint64()
                    self.lib.rt_gguf_meta_array_string(self.handle, i, k, ctypes.byref(p),
                                                       ctypes.byref(ln))
                    val.append(ctypes.string_at(p.value, ln.value).decode())
            elif et.value == 9:
                val = [None] * n  # nested arrays: length only
            else:
                buf = (ctypes.c_double * max(n, 1))()
                self.lib.rt_gguf_meta_array_numbers(self.handle, i, buf, n)
                val = [buf[k] for k in range(n)]
                if et.value not in (6, 12):
                    val = [int(x) for x in val]
        else:
            v = ctypes.c_int64()
            self.lib.rt_gguf_meta_int(self.handle, i, ctypes.byref(v))
            val = bool(v.value) if t == 7 else int(v.value)
        return key.value.decode(), val, t

    # ── tensors ──
    def __contains__(self, name: str) -> bool:
        return name in self._by_name

    def tensor(self, name: str) -> TensorInfo:
        return self.tensors[self._by_name[name]]

    def tensor_bytes(self, name: str) -> np.ndarray:
        """Copy of a tensor's raw bytes (the mapping stays read-only)."""
        i = self._by_name[name]
        p = self.lib.rt_gguf_tensor_data(self.handle, i)
        return np.frombuffer(ctypes.string_at(p, self.tensors[i].nbytes), dtype=np.uint8).copy()

    def upload(self, ctx: d.HipContext, name: str, dst) -> None:
        i = self._by_name[name]
        ctx._check(self.lib.rt_gguf_upload(ctx.handle, self.handle, i, d._ptr(dst)))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.rt_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ───────────────────────────── model config ─────────────────────────────

class LoadError(Exception):
    """crates/engine/src/loader.rs LoadError (MissingMetadata / InvalidConfig)."""


@dataclass
class ModelConfig:
    arch_str: str
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rope_theta: float
    max_position_embeddings: int
    vocab_size: int
    rms_norm_eps: float
    activation: str
    bos_token_id: int | None
    eos_token_id: int | None

    @staticmethod
    def from_metadata(m: dict, types: dict | None = None) -> "ModelConfig":
        """config.rs:96-265.  `types` (GGUF value type per key, as
        GgufFile.metadata_types) restricts integer keys to u32 / u64 / i32 and
        float keys to f32 / f64, as the reference's accessors do."""
        arch = m.get("general.architecture")
        if not isinstance(arch, str):
            raise LoadError("missing metadata: general.architecture")
        p = arch

        def int_ok(key):
            v = m.get(key)
            if isinstance(v, bool) or not isinstance(v, int):
                return False
            return types is None or types.get(key) in (4, 10, 5)

        def req_u32(key):
            if not int_ok(key):
                raise LoadError(f"missing metadata: {key}")
            return m[key] & 0xFFFFFFFF

        def opt_int(key, default):
            return m[key] if int_ok(key) else default

        def opt_f32(key, default):
            v = m.get(key)
            ok = isinstance(v, float) and (types is None or types.get(key) in (6, 12))
            return float(np.float32(v)) if ok else default

        hidden = req_u32(f"{p}.embedding_length")
        ff = req_u32(f"{p}.feed_forward_length")
        layers = req_u32(f"{p}.block_count")
        heads = req_u32(f"{p}.attention.head_count")
        kv_heads = opt_int(f"{p}.attention.head_count_kv", heads)
        if int_ok(f"{p}.attention.key_length"):
            head_dim = m[f"{p}.attention.key_length"]
        else:
            if hidden % heads:
                raise LoadError(f"invalid config: hidden_size ({hidden}) not divisible by "
                                f"num_attention_heads ({heads})")
            head_dim = hidden // heads
        theta = opt_f32(f"{p}.rope.freq_base", 1_000_000.0 if arch == "qwen2" else 10_000.0)
        ctx_len = opt_int(f"{p}.context_length", 32768)
        try:
            vocab = req_u32("tokenizer.ggml.token_count")
        except LoadError:
            try:
                vocab = req_u32(f"{p}.vocab_size")
            except LoadError:
                toks = m.get("tokenizer.ggml.tokens")
                if not isinstance(toks, list):
                    raise LoadError("missing metadata: tokenizer.ggml.tokens (vocab size fallback)")
                vocab = len(toks)
        eps = opt_f32(f"{p}.attention.layer_norm_rms_epsilon", 1e-6)
        act = m.get(f"{p}.feed_forward_act", "silu")
        act = {"gelu": "gelu", "gelu_new": "gelu", "relu": "relu"}.get(act, "silu_mul")
        bos = m.get("tokenizer.ggml.bos_token_id")
        eos = m.get("tokenizer.ggml.eos_token_id")
        return ModelConfig(arch, hidden, ff, layers, heads, kv_heads, head_dim, theta, ctx_len,
                           vocab, eps, act, bos if isinstance(bos, int) else None,
                           eos if isinstance(eos, int) else None)


def qwen2_tensor_names(layers: int, gguf: GgufFile | None = None) -> dict:
    """Tensor names per role (forward.rs:1271-1330); the LM head falls back to
    token_embd.weight when output.weight is absent (tied, forward.rs:1271-1276)."""
    names = {"token_embd": "token_embd.weight", "output_norm": "output_norm.weight",
             "output": "output.weight"}
    if gguf is not None and "output.weight" not in gguf:
        names["output"] = "token_embd.weight"
    for layer in range(layers):
        for role in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                     "ffn_gate", "ffn_up", "ffn_down"):
            names[f"blk.{layer}.{role}"] = f"blk.{layer}.{role}.weight"
        for b in ("attn_q", "attn_k", "attn_v"):
            names[f"blk.{layer}.{b}.bias"] = f"blk.{layer}.{b}.bias"
    return names
