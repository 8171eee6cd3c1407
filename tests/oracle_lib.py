"""ctypes access to the CPU oracle (oracle/liboracle.so) — tests only."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(REPO, "oracle")
LIB = os.path.join(ORACLE_DIR, "liboracle.so")

FMT = {"q8_0": 0, "q4_0": 1, "q4k": 2, "q6k": 3, "q5_0": 4, "q5k": 5,
       "q4_0g": 6, "q4kg": 7, "q5kg": 8, "q6kg": 9}  # …g: ggml layouts
BLOCK = {"q8_0": (32, 34), "q4_0": (32, 18), "q4k": (256, 144), "q6k": (256, 210),
         "q5_0": (32, 22), "q5k": (256, 176),
         "q4_0g": (32, 18), "q4kg": (256, 144), "q5kg": (256, 176), "q6kg": (256, 210)}


def _load():
    srcs = [os.path.join(ORACLE_DIR, f) for f in ("oracle.c", "oracle.h")]
    if not os.path.exists(LIB) or os.path.getmtime(LIB) < max(map(os.path.getmtime, srcs)):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
    return ctypes.CDLL(LIB)


_lib = _load()
_P, _S = ctypes.c_void_p, ctypes.c_size_t
_lib.ora_h2f.argtypes = [ctypes.c_uint16]
_lib.ora_h2f.restype = ctypes.c_float
_lib.ora_f2h.argtypes = [ctypes.c_float]
_lib.ora_f2h.restype = ctypes.c_uint16
_lib.ora_dequant.argtypes = [ctypes.c_int, _P, _S, _P]
_lib.ora_dequant_q4k_f16.argtypes = [_P, _S, _P]
_lib.ora_gemv_packed.argtypes = [ctypes.c_int, _P, _P, _S, _S, _S, _P, _P]
_lib.ora_gemv_ref_f32.argtypes = [ctypes.c_int, _P, _P, _S, _S, _P, ctypes.c_int]
_lib.ora_silu.argtypes = [ctypes.c_double]
_lib.ora_silu.restype = ctypes.c_double
_lib.ora_argmax_f32.argtypes = [_P, _S]
_lib.ora_argmax_f32.restype = ctypes.c_uint32
_lib.ora_synth_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
_lib.ora_synth_normal.restype = ctypes.c_float
_lib.ora_synth_normal_f32.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                      ctypes.c_float, _P]
_lib.ora_synth_weights.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_float, _S, _P]
_lib.ora_rms_norm.argtypes = [_P, _P, ctypes.c_double, _S, _S, _P]
_lib.ora_rope.argtypes = [_P, _S, _S, ctypes.c_uint32, ctypes.c_float]
_lib.ora_attention.argtypes = [_P, _P, _P, _S, _S, _S, _S, _S, ctypes.c_double, _P]
for _n in FMT:
    getattr(_lib, f"ora_quantize_{_n}").argtypes = [_P, _S, _P]
_lib.ora_relayout_to_ggml.argtypes = [ctypes.c_int, _P, _S, _P]


def _p(a: np.ndarray):
    return a.ctypes.data


def h2f(h: int) -> float:
    return _lib.ora_h2f(h)


def f2h(f: float) -> int:
    return _lib.ora_f2h(f)


def dequant(fmt: str, packed: np.ndarray) -> np.ndarray:
    el, by = BLOCK[fmt]
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    nblk = packed.size // by
    out = np.empty(nblk * el, dtype=np.float32)
    _lib.ora_dequant(FMT[fmt], _p(packed), nblk, _p(out))
    return out


def dequant_q4k_f16(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    nblk = packed.size // 144
    out = np.empty(nblk * 256, dtype=np.uint16)
    _lib.ora_dequant_q4k_f16(_p(packed), nblk, _p(out))
    return out


def gemv(fmt: str, packed: np.ndarray, x: np.ndarray, n: int, k: int):
    """f64 reference y and Σ|w·x| per row; x may be (k,) or (m, k)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = 1 if x.ndim == 1 else x.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    s = np.empty((m, n), dtype=np.float64)
    _lib.ora_gemv_packed(FMT[fmt], _p(packed), _p(x), m, n, k, _p(y), _p(s))
    if x.ndim == 1:
        return y[0], s[0]
    return y, s


def gemv_ref_f32(fmt: str, packed: np.ndarray, x: np.ndarray, n: int, k: int, threads: int = 1):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n, dtype=np.float32)
    _lib.ora_gemv_ref_f32(FMT[fmt], _p(packed), _p(x), n, k, _p(y), threads)
    return y


def silu(x: float) -> float:
    return _lib.ora_silu(x)


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(_lib.ora_argmax_f32(_p(v), v.size))


def synth_normal(seed: int, n: int, start: int = 0, mean: float = 0.0,
                 std: float = 1.0) -> np.ndarray:
    """mean + std·N(seed, i) for i in [start, start + n), in f32 arithmetic."""
    out = np.empty(start + n, dtype=np.float32)
    _lib.ora_synth_normal_f32(seed, start + n, mean, std, _p(out))
    return out[start:]


def quantize(fmt: str, w: np.ndarray) -> np.ndarray:
    el, by = BLOCK[fmt]
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    nblk = w.size // el
    out = np.zeros(nblk * by, dtype=np.uint8)
    getattr(_lib, f"ora_quantize_{fmt}")(_p(w), nblk, _p(out))
    return out


def relayout_to_ggml(fmt: str, packed: np.ndarray) -> np.ndarray:
    """Reference-layout blocks (q4_0 / q4k / q5k) re-laid out in ggml's."""
    el, by = BLOCK[fmt]
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty_like(packed)
    _lib.ora_relayout_to_ggml(FMT[fmt], _p(packed), packed.size // by, _p(out))
    return out


def synth_weights(fmt: str, n: int, k: int, seed: int, std: float = 0.02) -> np.ndarray:
    """Host twin of the device generators (rt_synth_*): the same bytes."""
    el, by = BLOCK[fmt]
    nblk = n * k // el
    if fmt.endswith("g"):  # ggml layouts: the reference-layout blocks re-laid out
        return quantize(fmt, synth_normal(seed, n * k, std=std))
    out = np.empty(nblk * by, dtype=np.uint8)
    _lib.ora_synth_weights(FMT[fmt], seed, std, nblk, _p(out))
    return out


_lib.ora_rope_batch.argtypes = [_P, _S, _S, _S, ctypes.c_uint32, ctypes.c_float]
_lib.ora_argmax_rows_first_f32.argtypes = [_P, _S, _S, _P]


def rope_batch(v: np.ndarray, seq: int, heads: int, head_dim: int, start_pos: int,
               theta: float) -> np.ndarray:
    out = np.ascontiguousarray(v, dtype=np.float64).copy()
    _lib.ora_rope_batch(_p(out), seq, heads, head_dim, start_pos, theta)
    return out


def argmax_rows_first(v: np.ndarray, rows: int) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(rows, np.uint32)
    _lib.ora_argmax_rows_first_f32(_p(v), rows, v.size // max(rows, 1), _p(out))
    return out


def causal_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_len: int, num_heads: int,
                     num_kv_heads: int, head_dim: int, kv_len: int, kv_stride: int,
                     q_start: int) -> np.ndarray:
    """flash_attention_f16 (attention.metal:36-160) for one sequence: query
    row r attends to cache positions j < kv_len with j <= q_start + r — each
    row is the decode attention over its prefix."""
    q = np.asarray(q, dtype=np.float64).reshape(q_len, num_heads * head_dim)
    return np.stack([attention(q[r], k, v, num_heads, num_kv_heads, head_dim,
                               min(kv_len, q_start + r + 1), kv_stride) for r in range(q_len)])


def rms_norm(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    gamma = np.ascontiguousarray(gamma, dtype=np.float32)
    hidden = gamma.size
    rows = x.size // hidden
    y = np.empty(x.size, dtype=np.float64)
    _lib.ora_rms_norm(_p(x), _p(gamma), eps, hidden, rows, _p(y))
    return y.reshape(x.shape)


def rope(v: np.ndarray, heads: int, head_dim: int, pos: int, theta: float) -> np.ndarray:
    out = np.ascontiguousarray(v, dtype=np.float64).copy()
    _lib.ora_rope(_p(out), heads, head_dim, pos, theta)
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, num_heads: int, num_kv_heads: int,
              head_dim: int, kv_len: int, kv_stride: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float64)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(num_heads * head_dim, dtype=np.float64)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
    _lib.ora_attention(_p(q), _p(k), _p(v), num_heads, num_kv_heads, head_dim, kv_len,
                       kv_stride, scale, _p(out))
    return out


# ───────────────────────── whole decode step (f32, CPU baseline) ─────────────────────────

class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "bq", "bk", "bv", "attn_norm",
                 "ffn_norm", "kc", "vc")] + \
               [(n, ctypes.c_int32) for n in ("fq", "fk", "fv", "fo", "fg", "fu", "fd")]


class _Model(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("layers", "hidden", "heads", "kv_heads", "head_dim", "ff", "vocab", "max_seq")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float),
                ("layer", ctypes.POINTER(_Layer)), ("final_norm", ctypes.c_void_p),
                ("embd", ctypes.c_void_p), ("lm_head", ctypes.c_void_p), ("f_lm", ctypes.c_int32),
                ("f_embd", ctypes.c_int32)]


_lib.ora_decode_step_ref_f32.argtypes = [ctypes.POINTER(_Model), ctypes.c_uint32, ctypes.c_uint32,
                                         _P, ctypes.c_int]
_lib.ora_decode_step_ref_f32.restype = ctypes.c_uint32

_ROLE_KEYS = (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo"), ("gate", "wg"), ("up", "wu"),
              ("down", "wd"))


class HostStepModel:
    """A Qwen2-shape model in host memory for ora_decode_step_ref_f32.

    layers: list of dicts with the keys of runit_mac_amd.decode.DecodeModel's
    layers (wq … wd packed uint8, bq/bk/bv float16, attn_norm/ffn_norm
    float32, kc/vc float32 [kv_heads·max_seq·head_dim]); fmts: one dict per
    layer giving each role's format (or one dict for every layer); lm_fmt /
    embd_fmt: the LM head's and the embedding table's formats."""

    def __init__(self, cfg, layers, final_norm, embd, lm_head, fmts, lm_fmt, embd_fmt="q8_0"):
        if isinstance(fmts, dict):
            fmts = [fmts] * len(layers)
        self.cfg, self.layers, self.fmts = cfg, layers, fmts
        self.keep = [final_norm, embd, lm_head]
        arr = (_Layer * len(layers))()
        for i, L in enumerate(layers):
            for k, v in L.items():
                setattr(arr[i], k, v.ctypes.data)
            for role, key in _ROLE_KEYS:
                setattr(arr[i], "f" + key[1], FMT[fmts[i][role]])
        self.m = _Model(cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ff,
                        cfg.vocab, cfg.max_seq, cfg.eps, cfg.theta, arr, final_norm.ctypes.data,
                        embd.ctypes.data, lm_head.ctypes.data, FMT[lm_fmt], FMT[embd_fmt])
        self.arr = arr

    def step(self, token: int, pos: int, threads: int = 1):
        logits = np.empty(self.cfg.vocab, np.float32)
        tok = _lib.ora_decode_step_ref_f32(ctypes.byref(self.m), token, pos, _p(logits), threads)
        return int(tok), logits

    @classmethod
    def from_recipe(cls, dm) -> "HostStepModel":
        """The host twin of a synthetic runit_mac_amd.decode.DecodeModel: every
        tensor regenerated from the model's recipe with the oracle's
        generators (byte-identical to the device's)."""
        spec = {p: (kind, seed, n, extra) for p, kind, seed, n, extra in dm.recipe}

        def make(ptr):
            kind, seed, n, extra = spec[ptr]
            if kind == "w":
                el, _ = BLOCK[extra]
                out = np.empty(n // el * BLOCK[extra][1], np.uint8)
                _lib.ora_synth_weights(FMT[extra], seed, 0.02, n // el, _p(out))
                return out
            mean, std = extra
            v = synth_normal(seed, n, mean=mean, std=std)
            return v.astype(np.float16) if kind == "f16" else v

        layers = [{k: make(v) for k, v in L.items()} for L in dm.layers]
        embd = make(dm.embd)
        lm = embd if dm.lm_head == dm.embd else make(dm.lm_head)
        return cls(dm.cfg, layers, make(dm.final_norm), embd, lm, dm.fmts, dm.lm_fmt, dm.embd_fmt)
