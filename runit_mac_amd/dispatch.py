"""Python mirror of RunIT's `crates/kernels` dispatch API over the C ABI.

The reference exposes `MetalContext` (crates/kernels/src/context.rs) and about
80 `dispatch::<kernel>(ctx, &Buffer.., dims) -> Result<()>` functions
(crates/kernels/src/dispatch.rs).  This module keeps those names, argument
order and meaning, and the `KernelError` variants (crates/kernels/src/error.rs:
4-21), on top of `librunit_hip.so` (include/runit_hip.h).  Every call only
enqueues; `ctx.flush()` waits, as in the reference.

There is no CPU fallback: if the native library or the gfx950 code object is
missing, or no GPU is visible, constructing a context raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_size_t, c_uint32, c_uint64, c_void_p

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "librunit_hip.so")
HSACO_PATH = os.path.join(_PKG, "lib", "kernels")  # one code object per kernel unit


# ───────────────────────────── errors (error.rs:4-21) ─────────────────────────────

class KernelError(Exception):
    """Base of the KernelError variants."""


class NoDevice(KernelError):
    pass


class LibraryLoad(KernelError):
    pass


class PipelineNotFound(KernelError):
    pass


class PipelineCreate(KernelError):
    pass


class Dispatch(KernelError):
    pass


class BufferSize(KernelError):
    pass


_STATUS = {1: NoDevice, 2: LibraryLoad, 3: PipelineNotFound, 4: PipelineCreate, 5: Dispatch,
           6: BufferSize}


# ───────────────────────────── library loading ─────────────────────────────

_lib = None

# (name, argtypes) for every exported symbol; restype is c_int unless noted.
_P, _U32, _U64, _F = c_void_p, c_uint32, c_uint64, c_float
_ROWS_FMTS = ("q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg", "q5kg", "q6kg")
_SIGS = {
    "rt_ctx_create": [POINTER(c_void_p), c_char_p],
    "rt_gemm_set_f32": [_P, _U32, _P, _P, _P, _P, _P, _P, _P, _U32, _U32, _P, _F, _P, _U32],
    "rt_gemm_qkv_rope_f32": [_P, c_char_p, _P, c_char_p, _P, c_char_p, _P, _P, _P, _P, _P, _P, _F,
                             _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _F, _U32],
    "rt_gemm_ffn_block_f32": [_P, c_char_p, _P, c_char_p, _P, c_char_p, _P, c_char_p, _P, _P, _P,
                              _P, _P, _F, _P, _P, _P, _U32, _U32, _U32, _U32],
    "rt_gemm_attn_ffn_block_f32": [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _P,
                                   c_char_p, _P, c_char_p, _P, c_char_p, _P, c_char_p, _P, _P, _P,
                                   _P, _F, _P, _P, _P, _U32, _U32, _U32],
    "rt_flush": [_P],
    "rt_device_cu_count": [_P],
    "rt_has_kernel": [_P, c_char_p],
    "rt_malloc": [_P, c_size_t, POINTER(c_void_p)],
    "rt_free": [_P, _P],
    "rt_upload": [_P, _P, _P, c_size_t],
    "rt_download": [_P, _P, _P, c_size_t],
    "rt_memset": [_P, _P, c_int, c_size_t],
    "rt_copy_d2d": [_P, _P, _P, c_size_t],
    "rt_event_create": [_P, POINTER(c_void_p)],
    "rt_event_record": [_P, _P],
    "rt_event_elapsed_ms": [_P, _P, _P, POINTER(c_float)],
    "rt_capture_begin": [_P],
    "rt_capture_end": [_P, POINTER(c_void_p)],
    "rt_graph_launch": [_P, _P],
    # GEMV family: (ctx, weight, input, output, [residual,] m, k)
    **{n: [_P, _P, _P, _P, _U32, _U32] for n in (
        "rt_gemv_q8_0_f32in_f32out", "rt_gemv_q8_0_f32in", "rt_gemv_q8_0_f16",
        "rt_gemv_q8_0_f32in_f32out_mr",
        "rt_gemv_q4_0_f32in_f32out", "rt_gemv_q4_0_f32in", "rt_gemv_q4_0_f16",
        "rt_gemv_q4k_f32in_f32out", "rt_gemv_q4k_f16",
        "rt_gemv_q6k_f32in_f32out", "rt_gemv_q6k_f32in",
        "rt_gemv_q5_0_f32in_f32out", "rt_gemv_q5_0_f32in",
        "rt_gemv_q5k_f32in_f32out", "rt_gemv_q5k_f32in",
        *[f"rt_gemv_{g}_{v}" for g in ("q4_0g", "q4kg", "q5kg", "q6kg")
          for v in ("f32in_f32out", "f32in")])},
    **{n: [_P, _P, _P, _P, _P, _U32, _U32] for n in (
        "rt_gemv_q8_0_add_f32_f32in", "rt_gemv_q8_0_add_f16", "rt_gemv_q8_0_add_f32res_f16",
        "rt_gemv_q8_0_add_f32_f32in_mr",
        "rt_gemv_q4_0_add_f32_f32in", "rt_gemv_q4_0_add_f16",
        "rt_gemv_q4k_add_f32_f32in", "rt_gemv_q4k_add_f16", "rt_gemv_q4k_add_f32res_f16",
        "rt_gemv_q6k_add_f32_f32in", "rt_gemv_q5_0_add_f32_f32in", "rt_gemv_q5k_add_f32_f32in",
        "rt_gemv_q4_0g_add_f32_f32in", "rt_gemv_q4kg_add_f32_f32in", "rt_gemv_q5kg_add_f32_f32in",
        "rt_gemv_q6kg_add_f32_f32in", "rt_gemv_q6k_add_f32_f32in_noalloc")},
    "rt_fused_qkv_q8_0_f32": [_P] + [_P] * 7 + [_U32] * 3,
    "rt_fused_qkv_bias_q8_0_f32": [_P] + [_P] * 10 + [_U32] * 3,
    "rt_fused_qkv_bias_q4_0_f32": [_P] + [_P] * 10 + [_U32] * 3,
    "rt_fused_qkv_bias_q5_0_f32": [_P] + [_P] * 10 + [_U32] * 3,
    "rt_fused_qkv_bias_q5k_f32": [_P] + [_P] * 10 + [_U32] * 3,
    **{n: [_P] + [_P] * 10 + [_U32] * 3 for n in (
        "rt_fused_qkv_bias_q4k_f32", "rt_fused_qkv_bias_q4kg_f32",
        "rt_fused_qkv_bias_q4k_q6k_f32", "rt_fused_qkv_bias_q4kg_q6kg_f32")},
    **{n: [_P, _P, _P, _P, _P, _U32, _U32] for n in (
        "rt_fused_ffn_q8_0_f32", "rt_fused_ffn_q4_0_f32", "rt_fused_ffn_q4k_f32",
        "rt_fused_ffn_q5_0_f32", "rt_fused_ffn_q5k_f32", "rt_fused_ffn_q4_0g_f32",
        "rt_fused_ffn_q4kg_f32", "rt_fused_ffn_q5kg_f32")},
    **{n: [_P, _P, _P, _U32] for n in (
        "rt_dequant_q8_0_f32", "rt_dequant_q4_0_f32", "rt_dequant_q4k_f32",
        "rt_dequant_q6k_f32", "rt_dequant_q4k_f16", "rt_dequant_q5_0_f32", "rt_dequant_q5k_f32",
        "rt_dequant_q4_0g_f32", "rt_dequant_q4kg_f32", "rt_dequant_q5kg_f32", "rt_dequant_q6kg_f32", "rt_argmax_f32", "rt_argmax_f16")},
    **{n: [_P, _P, _P, _P, _U32, _U32, _U32] for n in (
        "rt_gemm_q8_0_f32", "rt_gemm_q4_0_f32", "rt_gemm_q4k_f32", "rt_gemm_q5_0_f32",
        "rt_gemm_q5k_f32", "rt_gemm_q6k_f32", "rt_gemm_q4_0g_f32", "rt_gemm_q4kg_f32",
        "rt_gemm_q5kg_f32", "rt_gemm_q6kg_f32")},
    "rt_rms_norm_f32_f32_f32g": [_P, _P, _P, _P, _F, _U32, _U32],
    "rt_fused_rope_qk_f32": [_P, _P, _P, _U32, _U32, _U32, _U32, _F],
    "rt_kv_copy_to_cache_f32": [_P, _P, _P, _U32, _U32, _U32, _U32],
    "rt_decode_attention_f32": [_P, _P, _P, _P, _P] + [_U32] * 6,
    "rt_decode_attention_rope_f32": [_P] + [_P] * 6 + [_U32] * 5 + [_F],
    "rt_decode_attention_rope_oproj_q8_0_f32": [_P] + [_P] * 7 + [_U32] * 5 + [_F, _U32],
    "rt_decode_attention_rope_oproj_q4k_f32": [_P] + [_P] * 7 + [_U32] * 5 + [_F, _U32],
    "rt_launch_count": [_P],
    "rt_decode_attention_rope_oproj_q4kg_f32": [_P] + [_P] * 7 + [_U32] * 5 + [_F, _U32],
    "rt_add_f16_into_f32": [_P, _P, _P, _U32],
    **{f"rt_embed_{_f}_f32": [_P, _P, _P, _P, _U32] for _f in (
        "q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg", "q5kg", "q6kg", "f16", "f32")},
    **{f"rt_embed_rows_{_f}_f32": [_P, _P, _P, _P, _U32, _U32] for _f in (
        "q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg", "q5kg", "q6kg", "f16", "f32")},
    **{f"rt_gemv_rows_{_f}_f32": [_P, _P, _P, _P, _F, _P, _U32, _U32, _U32] for _f in _ROWS_FMTS},
    **{f"rt_gemv_rows_{_f}_add_f32": [_P, _P, _P, _P, _P, _U32, _U32, _U32] for _f in _ROWS_FMTS},
    **{f"rt_qkv_bias_rows_{_f}_f32": [_P, _P, _P, _P, _P, _P, _F] + [_P] * 6 + [_U32] * 4
       for _f in _ROWS_FMTS},
    **{f"rt_fused_ffn_rows_{_f}_f32": [_P, _P, _P, _P, _P, _F, _P, _U32, _U32, _U32]
       for _f in _ROWS_FMTS},
    "rt_add_bias_broadcast_f32": [_P, _P, _P, _U32, _U32],
    "rt_rope_batch_inplace_f32": [_P, _P, _U32, _U32, _U32, _F, _U32],
    "rt_kv_write_batch_f32": [_P] + [_P] * 4 + [_U32] * 5,
    "rt_rope_kv_write_batch_f32": [_P] + [_P] * 5 + [_U32] * 4 + [_F, _U32, _U32],
    "rt_flash_attention_f32": [_P] + [_P] * 4 + [_U32] * 8,
    "rt_add_f32": [_P, _P, _P, _P, _U32],
    "rt_silu_mul_f32": [_P, _P, _P, _P, _U32],
    "rt_argmax_rows_first_f32": [_P, _P, _P, _U32, _U32],
    "rt_rms_norm_fused_qkv_bias_q8_0_f32": [_P, _P, _P, _P, _P, _P, _F] + [_P] * 6 + [_U32] * 3,
    "rt_rms_norm_fused_ffn_q8_0_f32": [_P, _P, _P, _P, _P, _F, _P, _U32, _U32],
    "rt_rms_norm_fused_ffn_q8_0_f32_ssq": [_P, _P, _P, _P, _P, _F, _P, _U32, _U32, _P, _U32],
    "rt_rms_norm_fused_qkv_bias_q8_0_f32_ssq": [_P, _P, _P, _P, _P, _P, _F] + [_P] * 6 +
                                               [_U32] * 3 + [_P, _U32],
    "rt_gemv_q8_0_add_f32_f32in_ssq": [_P, _P, _P, _P, _P, _U32, _U32, _P],
    "rt_decode_attention_rope_oproj_q8_0_f32_ssq": [_P] + [_P] * 7 + [_U32] * 5 + [_F, _U32, _P],
    "rt_rms_norm_gemv_q8_0_f32in_f32out": [_P, _P, _P, _P, _F, _P, _U32, _U32],
    "rt_rms_norm_fused_qkv_bias_q4k_q6k_f32": [_P, _P, _P, _P, _P, _P, _F] + [_P] * 6 + [_U32] * 3,
    "rt_rms_norm_fused_ffn_q4k_f32": [_P, _P, _P, _P, _P, _F, _P, _U32, _U32],
    "rt_rms_norm_gemv_q6k_f32in_f32out": [_P, _P, _P, _P, _F, _P, _U32, _U32],
    "rt_stream_read": [_P, _P, c_size_t, _P, c_size_t],
    "rt_stream_copy": [_P, _P, _P, c_size_t],
    "rt_synth_normal_f32": [_P, _P, _U64, _U64, _F, _F],
    "rt_synth_normal_f16": [_P, _P, _U64, _U64, _F, _F],
    **{n: [_P, _P, _U64, _U64, _F] for n in (
        "rt_synth_q8_0", "rt_synth_q4_0", "rt_synth_q4k", "rt_synth_q6k", "rt_synth_q5_0",
        "rt_synth_q5k")},
}


class StepLayer(ctypes.Structure):
    """rt_step_layer (include/runit_hip.h)."""
    _fields_ = [(n, c_void_p) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "bq", "bk",
                                        "bv", "attn_norm", "ffn_norm", "k_cache", "v_cache")]


class StepModel(ctypes.Structure):
    """rt_step_model (include/runit_hip.h)."""
    _fields_ = [(n, c_uint32) for n in ("layers", "hidden", "heads", "kv_heads", "head_dim", "ff",
                                        "vocab", "max_seq")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float),
                ("layer", POINTER(StepLayer))] + \
               [(n, c_void_p) for n in ("token_embd", "lm_head", "output_norm", "token", "logits")]


class DecodeStep:
    """A planned persistent decode step (rt_decode_step_*): one launch for the
    embedding and every layer, then the LM head and the argmax."""

    def __init__(self, ctx: "HipContext", model: StepModel, pos: int):
        self.ctx, self._model = ctx, model
        h = c_void_p()
        ctx._check(ctx.lib.rt_decode_step_q8_0_create(ctx.handle, ctypes.byref(model), pos,
                                                      ctypes.byref(h)))
        self.handle = h.value

    def run(self) -> None:
        self.ctx._check(self.ctx.lib.rt_decode_step_run(self.ctx.handle, self.handle))

    def check(self) -> None:
        """Flushes; raises Dispatch if a grid barrier of any run timed out."""
        self.ctx._check(self.ctx.lib.rt_decode_step_status(self.ctx.handle, self.handle))

    def __del__(self):
        if getattr(self, "handle", None):
            self.ctx.lib.rt_decode_step_destroy(self.handle)
            self.handle = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads librunit_hip.so and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise LibraryLoad(f"native library missing: {path} (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, argtypes in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = c_int
    lib.rt_last_error.argtypes = [_P]
    lib.rt_last_error.restype = c_char_p
    lib.rt_global_last_error.argtypes = []
    lib.rt_global_last_error.restype = c_char_p
    lib.rt_ctx_destroy.argtypes = [_P]
    lib.rt_ctx_destroy.restype = None
    lib.rt_event_destroy.argtypes = [_P]
    lib.rt_event_destroy.restype = None
    lib.rt_graph_destroy.argtypes = [_P]
    lib.rt_graph_destroy.restype = None
    lib.rt_decode_step_q8_0_create.argtypes = [_P, POINTER(StepModel), c_uint32, POINTER(c_void_p)]
    lib.rt_decode_step_q8_0_create.restype = c_int
    lib.rt_decode_step_run.argtypes = [_P, _P]
    lib.rt_decode_step_run.restype = c_int
    lib.rt_decode_step_status.argtypes = [_P, _P]
    lib.rt_decode_step_status.restype = c_int
    lib.rt_decode_step_destroy.argtypes = [_P]
    lib.rt_decode_step_destroy.restype = None
    lib.rt_launch_count.restype = c_uint64
    lib.rt_last_launch_name.argtypes = [_P]
    lib.rt_last_launch_name.restype = c_char_p
    # GGUF reader: (name, argtypes, restype)
    PU64 = POINTER(c_uint64)
    for name, argtypes, restype in (
            ("rt_gguf_open", [c_char_p, POINTER(c_void_p)], c_int),
            ("rt_gguf_close", [_P], None),
            ("rt_gguf_last_error", [], c_char_p),
            ("rt_gguf_version", [_P], c_uint32),
            ("rt_gguf_alignment", [_P], c_uint64),
            ("rt_gguf_data_offset", [_P], c_uint64),
            ("rt_gguf_tensor_count", [_P], c_uint64),
            ("rt_gguf_find_tensor", [_P, c_char_p], ctypes.c_int64),
            ("rt_gguf_tensor_info", [_P, c_uint64, POINTER(c_char_p), POINTER(c_uint32), PU64,
                                     POINTER(c_uint32), PU64, PU64], c_int),
            ("rt_gguf_tensor_data", [_P, c_uint64], c_void_p),
            ("rt_gguf_upload", [_P, _P, c_uint64, _P], c_int),
            ("rt_gguf_meta_count", [_P], c_uint64),
            ("rt_gguf_find_meta", [_P, c_char_p], ctypes.c_int64),
            ("rt_gguf_meta_info", [_P, c_uint64, POINTER(c_char_p), POINTER(c_uint32),
                                   POINTER(c_uint32), PU64], c_int),
            ("rt_gguf_meta_int", [_P, c_uint64, POINTER(ctypes.c_int64)], c_int),
            ("rt_gguf_meta_float", [_P, c_uint64, POINTER(ctypes.c_double)], c_int),
            ("rt_gguf_meta_string", [_P, c_uint64], c_char_p),
            ("rt_gguf_meta_array_numbers", [_P, c_uint64, POINTER(ctypes.c_double), c_uint64],
             c_int),
            ("rt_gguf_meta_array_string", [_P, c_uint64, c_uint64, POINTER(c_void_p), PU64],
             c_int)):
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    _lib = lib
    return lib


def _ptr(b) -> int | None:
    if b is None:
        return None
    if isinstance(b, Buffer):
        return b.ptr
    if isinstance(b, bool) or not isinstance(b, (int, np.integer)):
        raise TypeError(f"device pointer expected, got {type(b).__name__}")
    return int(b)


# ───────────────────────────── context / buffers ─────────────────────────────

class Buffer:
    """A device allocation (the analogue of a Metal `Buffer`)."""

    def __init__(self, ctx: "HipContext", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = c_void_p()
        ctx._check(ctx.lib.rt_malloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def write(self, data, offset: int = 0) -> "Buffer":
        arr = np.ascontiguousarray(data)
        n = arr.nbytes
        if offset + n > self.nbytes:
            raise BufferSize(f"buffer size mismatch: expected {offset + n} bytes, got {self.nbytes}")
        self.ctx._check(self.ctx.lib.rt_upload(self.ctx.handle, self.ptr + offset,
                                               arr.ctypes.data, n))
        return self

    def read(self, dtype=np.uint8, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        out = np.empty(count, dtype=dt)
        if out.nbytes + offset > self.nbytes:
            raise BufferSize(f"buffer size mismatch: expected {out.nbytes + offset} bytes, "
                             f"got {self.nbytes}")
        self.ctx._check(self.ctx.lib.rt_download(self.ctx.handle, out.ctypes.data,
                                                 self.ptr + offset, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            self.ctx.lib.rt_free(self.ctx.handle, self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and self.ctx.handle:
                self.free()
        except Exception:
            pass


class Graph:
    def __init__(self, ctx: "HipContext", handle: int):
        self.ctx, self.handle = ctx, handle

    def launch(self) -> None:
        self.ctx._check(self.ctx.lib.rt_graph_launch(self.ctx.handle, self.handle))

    def __del__(self):
        try:
            if self.handle:
                self.ctx.lib.rt_graph_destroy(self.handle)
                self.handle = 0
        except Exception:
            pass


class Event:
    def __init__(self, ctx: "HipContext"):
        self.ctx = ctx
        h = c_void_p()
        ctx._check(ctx.lib.rt_event_create(ctx.handle, ctypes.byref(h)))
        self.handle = h.value

    def record(self) -> None:
        self.ctx._check(self.ctx.lib.rt_event_record(self.ctx.handle, self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        self.ctx._check(self.ctx.lib.rt_event_elapsed_ms(self.ctx.handle, self.handle,
                                                         end.handle, ctypes.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                self.ctx.lib.rt_event_destroy(self.handle)
                self.handle = 0
        except Exception:
            pass


class HipContext:
    """MetalContext analogue (context.rs:139-304): device, code object, stream."""

    def __init__(self, code_object: str | None = None):
        self.lib = load_library()
        h = c_void_p()
        path = (code_object or HSACO_PATH).encode()
        st = self.lib.rt_ctx_create(ctypes.byref(h), path)
        if st != 0:
            raise _STATUS.get(st, KernelError)(self.lib.rt_global_last_error().decode())
        self.handle = h.value

    def _check(self, status: int) -> None:
        if status != 0:
            msg = self.lib.rt_last_error(self.handle).decode()
            raise _STATUS.get(status, KernelError)(msg)

    @property
    def cu_count(self) -> int:
        return int(self.lib.rt_device_cu_count(self.handle))

    def new_buffer(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def buffer_from(self, data) -> Buffer:
        arr = np.ascontiguousarray(data)
        return Buffer(self, max(arr.nbytes, 1)).write(arr)

    def flush(self) -> None:
        self._check(self.lib.rt_flush(self.handle))

    def has_kernel(self, name: str) -> None:
        self._check(self.lib.rt_has_kernel(self.handle, name.encode()))

    def event(self) -> Event:
        return Event(self)

    def capture_begin(self) -> None:
        self._check(self.lib.rt_capture_begin(self.handle))

    def capture_end(self) -> Graph:
        g = c_void_p()
        self._check(self.lib.rt_capture_end(self.handle, ctypes.byref(g)))
        return Graph(self, g.value)

    def close(self) -> None:
        if self.handle:
            self.lib.rt_ctx_destroy(self.handle)
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ───────────────────────────── dispatch functions ─────────────────────────────
# Same names and argument order as crates/kernels/src/dispatch.rs.

def _call(ctx: HipContext, name: str, *args) -> None:
    ctx._check(getattr(ctx.lib, name)(ctx.handle, *[_ptr(a) if isinstance(a, Buffer) else a
                                                   for a in args]))


def _gemv(name):
    def f(ctx, weight, input, output, m, k):
        _call(ctx, "rt_" + name, _ptr(weight), _ptr(input), _ptr(output), m, k)
    f.__name__ = name
    f.__doc__ = f"dispatch::{name}(ctx, weight, input, output, m, k)"
    return f


def _gemv_add(name):
    def f(ctx, weight, input, output, residual, m, k):
        _call(ctx, "rt_" + name, _ptr(weight), _ptr(input), _ptr(output), _ptr(residual), m, k)
    f.__name__ = name
    f.__doc__ = f"dispatch::{name}(ctx, weight, input, output, residual, m, k)"
    return f


gemv_q8_0_f32in_f32out = _gemv("gemv_q8_0_f32in_f32out")
gemv_q8_0_f32in = _gemv("gemv_q8_0_f32in")
gemv_q8_0_f16 = _gemv("gemv_q8_0_f16")
gemv_q8_0_f32in_f32out_mr = _gemv("gemv_q8_0_f32in_f32out_mr")
gemv_q8_0_add_f32_f32in = _gemv_add("gemv_q8_0_add_f32_f32in")
gemv_q8_0_add_f16 = _gemv_add("gemv_q8_0_add_f16")
gemv_q8_0_add_f32res_f16 = _gemv_add("gemv_q8_0_add_f32res_f16")
gemv_q8_0_add_f32_f32in_mr = _gemv_add("gemv_q8_0_add_f32_f32in_mr")
gemv_q4_0_f32in_f32out = _gemv("gemv_q4_0_f32in_f32out")
gemv_q4_0_f32in = _gemv("gemv_q4_0_f32in")
gemv_q4_0_f16 = _gemv("gemv_q4_0_f16")
gemv_q4_0_add_f32_f32in = _gemv_add("gemv_q4_0_add_f32_f32in")
gemv_q4_0_add_f16 = _gemv_add("gemv_q4_0_add_f16")
gemv_q4k_f32in_f32out = _gemv("gemv_q4k_f32in_f32out")
gemv_q4k_f16 = _gemv("gemv_q4k_f16")
gemv_q4k_add_f32_f32in = _gemv_add("gemv_q4k_add_f32_f32in")
gemv_q4k_add_f16 = _gemv_add("gemv_q4k_add_f16")
gemv_q4k_add_f32res_f16 = _gemv_add("gemv_q4k_add_f32res_f16")
gemv_q6k_f32in_f32out = _gemv("gemv_q6k_f32in_f32out")
gemv_q6k_f32in = _gemv("gemv_q6k_f32in")
gemv_q6k_add_f32_f32in = _gemv_add("gemv_q6k_add_f32_f32in")
# no reference counterpart: the same GEMV with no device allocation (a fixed
# scratch array in the code object), for callers that cannot allocate
gemv_q6k_add_f32_f32in_noalloc = _gemv_add("gemv_q6k_add_f32_f32in_noalloc")
# Q5_0 / Q5_K (new: the reference dequantises both on the CPU, forward.rs:900-920, 979-1012)
gemv_q5_0_f32in_f32out = _gemv("gemv_q5_0_f32in_f32out")
gemv_q5_0_f32in = _gemv("gemv_q5_0_f32in")
gemv_q5_0_add_f32_f32in = _gemv_add("gemv_q5_0_add_f32_f32in")
gemv_q5k_f32in_f32out = _gemv("gemv_q5k_f32in_f32out")
gemv_q5k_f32in = _gemv("gemv_q5k_f32in")
gemv_q5k_add_f32_f32in = _gemv_add("gemv_q5k_add_f32_f32in")
# ggml layouts (upstream GGUF files): q4_0g, q4kg, q5kg, q6kg
for _g in ("q4_0g", "q4kg", "q5kg", "q6kg"):
    globals()[f"gemv_{_g}_f32in_f32out"] = _gemv(f"gemv_{_g}_f32in_f32out")
    globals()[f"gemv_{_g}_f32in"] = _gemv(f"gemv_{_g}_f32in")
    globals()[f"gemv_{_g}_add_f32_f32in"] = _gemv_add(f"gemv_{_g}_add_f32_f32in")


def fused_qkv_q8_0_f32(ctx, w_q, w_k, w_v, x_vec, out_q, out_k, out_v, q_dim, kv_dim, k):
    """dispatch.rs:813-838"""
    _call(ctx, "rt_fused_qkv_q8_0_f32", *map(_ptr, (w_q, w_k, w_v, x_vec, out_q, out_k, out_v)),
          q_dim, kv_dim, k)


def fused_qkv_bias_q8_0_f32(ctx, w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k,
                            bias_v, q_dim, kv_dim, k):
    """dispatch.rs:842-871"""
    _call(ctx, "rt_fused_qkv_bias_q8_0_f32",
          *map(_ptr, (w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k, bias_v)),
          q_dim, kv_dim, k)


def fused_qkv_bias_q4_0_f32(ctx, w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k,
                            bias_v, q_dim, kv_dim, k):
    """Q4_0 twin of dispatch.rs:842-871 (new)."""
    _call(ctx, "rt_fused_qkv_bias_q4_0_f32",
          *map(_ptr, (w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k, bias_v)),
          q_dim, kv_dim, k)


def fused_qkv_bias_q5_0_f32(ctx, w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k,
                            bias_v, q_dim, kv_dim, k):
    """Q5_0 twin of dispatch.rs:842-871 (new)."""
    _call(ctx, "rt_fused_qkv_bias_q5_0_f32",
          *map(_ptr, (w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k, bias_v)),
          q_dim, kv_dim, k)


def fused_qkv_bias_q5k_f32(ctx, w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k,
                           bias_v, q_dim, kv_dim, k):
    """Q5_K twin of dispatch.rs:842-871 (new)."""
    _call(ctx, "rt_fused_qkv_bias_q5k_f32",
          *map(_ptr, (w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k, bias_v)),
          q_dim, kv_dim, k)


def _qkv_mixed(sym, doc):
    def fn(ctx, w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k, bias_v, q_dim,
           kv_dim, k):
        _call(ctx, sym,
              *map(_ptr, (w_q, w_k, w_v, x_vec, out_q, out_k, out_v, bias_q, bias_k, bias_v)),
              q_dim, kv_dim, k)
    fn.__name__ = sym[3:]
    fn.__doc__ = doc
    return fn


_QKV_FALLBACK = ("Replaces the reference's non-Q8_0 projection sequence (three GEMVs, each "
                 "followed by add_f16_into_f32 of its bias, forward.rs:1561-1568) with one "
                 "launch (new). Biases: all three or all None.")
fused_qkv_bias_q4k_f32 = _qkv_mixed("rt_fused_qkv_bias_q4k_f32", "Q/K/V in Q4_K. " + _QKV_FALLBACK)
fused_qkv_bias_q4kg_f32 = _qkv_mixed("rt_fused_qkv_bias_q4kg_f32",
                                     "Q/K/V in ggml Q4_K. " + _QKV_FALLBACK)
fused_qkv_bias_q4k_q6k_f32 = _qkv_mixed("rt_fused_qkv_bias_q4k_q6k_f32",
                                        "Q/K in Q4_K, V in Q6_K. " + _QKV_FALLBACK)
fused_qkv_bias_q4kg_q6kg_f32 = _qkv_mixed("rt_fused_qkv_bias_q4kg_q6kg_f32",
                                          "Q/K in ggml Q4_K, V in ggml Q6_K. " + _QKV_FALLBACK)


def fused_ffn_q8_0_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """dispatch.rs:903-921"""
    _call(ctx, "rt_fused_ffn_q8_0_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def fused_ffn_q4_0_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """dispatch.rs:1531-1544"""
    _call(ctx, "rt_fused_ffn_q4_0_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def fused_ffn_q4k_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """Q4_K twin of dispatch.rs:903-921 (new)."""
    _call(ctx, "rt_fused_ffn_q4k_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def fused_ffn_q5_0_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """Q5_0 twin of dispatch.rs:903-921 (new)."""
    _call(ctx, "rt_fused_ffn_q5_0_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def fused_ffn_q5k_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """Q5_K twin of dispatch.rs:903-921 (new)."""
    _call(ctx, "rt_fused_ffn_q5k_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def fused_ffn_q4_0g_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """ggml-layout Q4_0 twin of dispatch.rs:903-921 (new)."""
    _call(ctx, "rt_fused_ffn_q4_0g_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def fused_ffn_q4kg_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """ggml-layout Q4_K twin of dispatch.rs:903-921 (new)."""
    _call(ctx, "rt_fused_ffn_q4kg_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def fused_ffn_q5kg_f32(ctx, w_gate, w_up, x_vec, act_out, ff_dim, k):
    """ggml-layout Q5_K twin of dispatch.rs:903-921 (new)."""
    _call(ctx, "rt_fused_ffn_q5kg_f32", *map(_ptr, (w_gate, w_up, x_vec, act_out)), ff_dim, k)


def dequant_q4k_f16(ctx, input, output, n_blocks):
    """dispatch.rs:756-772"""
    _call(ctx, "rt_dequant_q4k_f16", _ptr(input), _ptr(output), n_blocks)


def dequant_f32(ctx, fmt: str, input, output, n_blocks):
    """Bit-exact dequantisation to f32 for fmt in {q8_0, q4_0, q4k, q6k, q5_0, q5k}."""
    _call(ctx, f"rt_dequant_{fmt}_f32", _ptr(input), _ptr(output), n_blocks)


def gemm_set_f32(ctx, fmts, weights, ys, ns, x, m_rows, k, biases=None, res=None, gamma=None,
                 eps=0.0, xn=None, silu_pair=False):
    """The batched GEMMs of verify_draft over one activation matrix with the
    kernels between them folded in (new; forward.rs:2186-2271): y[i] =
    X·W[i]ᵀ (+ f16 bias[i]), X = x or RMSNorm(x)·γ (also written to xn);
    res: y[0] = res + X·W[0]ᵀ; silu_pair: y[0] = silu(X·W[0]ᵀ)·(X·W[1]ᵀ)."""
    cnt = len(fmts)
    if not (len(weights) == len(ys) == len(ns) == cnt) or (biases is not None and len(biases) != cnt):
        raise ValueError("gemm_set_f32: one weight, output and n per format")
    names = (c_char_p * cnt)(*[f.encode() for f in fmts])
    wv = (c_void_p * cnt)(*[_ptr(w) for w in weights])
    yv = (c_void_p * cnt)(*[_ptr(y) for y in ys])
    nv = (c_uint32 * cnt)(*ns)
    bv = (c_void_p * cnt)(*[_ptr(b) if b is not None else None for b in biases]) if biases else None
    adr = ctypes.addressof
    _call(ctx, "rt_gemm_set_f32", cnt, adr(names), adr(wv), adr(yv), adr(nv),
          adr(bv) if bv is not None else None, _ptr(res) if res is not None else None,
          _ptr(x), m_rows, k, _ptr(gamma) if gamma is not None else None, eps,
          _ptr(xn) if xn is not None else None, int(bool(silu_pair)))


def gemm_qkv_rope_f32(ctx, fmts, w_q, w_k, w_v, b_q, b_k, b_v, x, gamma, eps, xn, q, k, v,
                      k_cache, v_cache, m_rows, hidden, q_dim, kv_dim, head_dim, start_pos, theta,
                      max_seq):
    """verify_draft's Q/K/V of RMSNorm(x)·γ + biases, RoPE of q and k at
    start_pos + r, k / v into the caches, in one call (new;
    forward.rs:2186-2231).  fmts: the formats of (q, k, v)."""
    fq, fk, fv = (f.encode() for f in fmts)
    _call(ctx, "rt_gemm_qkv_rope_f32", fq, _ptr(w_q), fk, _ptr(w_k), fv, _ptr(w_v), _ptr(b_q),
          _ptr(b_k), _ptr(b_v), _ptr(x), _ptr(gamma), eps, _ptr(xn), _ptr(q), _ptr(k), _ptr(v),
          _ptr(k_cache), _ptr(v_cache), m_rows, hidden, q_dim, kv_dim, head_dim, start_pos, theta,
          max_seq)


def gemm_ffn_block_f32(ctx, fmts, w_o, w_gate, w_up, w_down, att, x, x_mid, gamma, eps, g, u, xn,
                       m_rows, h, qd, ff):
    """The part of a verify_draft layer after the attention (new;
    forward.rs:2227-2271): x_mid = x + att·W_oᵀ, then x = x_mid +
    (silu(X2·W_gᵀ)·(X2·W_uᵀ))·W_dᵀ with X2 = RMSNorm(x_mid)·γ.  fmts: the
    formats of (o, gate, up, down)."""
    fo, fg, fu, fd = (f.encode() for f in fmts)
    _call(ctx, "rt_gemm_ffn_block_f32", fo, _ptr(w_o), fg, _ptr(w_gate), fu, _ptr(w_up), fd,
          _ptr(w_down), _ptr(att), _ptr(x), _ptr(x_mid), _ptr(gamma), eps, _ptr(g), _ptr(u),
          _ptr(xn), m_rows, h, qd, ff)


def gemm_attn_ffn_block_f32(ctx, q, k_cache, v_cache, kv_len, num_heads, num_kv_heads, head_dim,
                            kv_head_stride, q_start, att, fmts, w_o, w_gate, w_up, w_down, x, x_mid,
                            gamma, eps, g, u, xn, m_rows, h, ff):
    """flash_attention_f32 (batch 1, q_len = m_rows) then gemm_ffn_block_f32
    over its output as one call (new; forward.rs:2225-2271)."""
    fo, fg, fu, fd = (f.encode() for f in fmts)
    _call(ctx, "rt_gemm_attn_ffn_block_f32", _ptr(q), _ptr(k_cache), _ptr(v_cache), kv_len,
          num_heads, num_kv_heads, head_dim, kv_head_stride, q_start, _ptr(att), fo, _ptr(w_o), fg,
          _ptr(w_gate), fu, _ptr(w_up), fd, _ptr(w_down), _ptr(x), _ptr(x_mid), _ptr(gamma), eps,
          _ptr(g), _ptr(u), _ptr(xn), m_rows, h, ff)


def gemm_q8_0_f32(ctx, weight, x, y, m_rows, n, k):
    """Batched Y[M,N] = X[M,K]·W[N,K]ᵀ (new; replaces gemm_f16 in verify_draft)."""
    _call(ctx, "rt_gemm_q8_0_f32", _ptr(weight), _ptr(x), _ptr(y), m_rows, n, k)


def gemm_q4_0_f32(ctx, weight, x, y, m_rows, n, k):
    """Batched GEMM on reference-layout Q4_0 weights (new)."""
    _call(ctx, "rt_gemm_q4_0_f32", _ptr(weight), _ptr(x), _ptr(y), m_rows, n, k)


def gemm_q4k_f32(ctx, weight, x, y, m_rows, n, k):
    """Batched GEMM on reference-layout Q4_K weights (new)."""
    _call(ctx, "rt_gemm_q4k_f32", _ptr(weight), _ptr(x), _ptr(y), m_rows, n, k)


def _gemm_fn(fmt, doc):
    def fn(ctx, weight, x, y, m_rows, n, k):
        _call(ctx, f"rt_gemm_{fmt}_f32", _ptr(weight), _ptr(x), _ptr(y), m_rows, n, k)
    fn.__name__ = f"gemm_{fmt}_f32"
    fn.__doc__ = doc
    return fn


gemm_q5_0_f32 = _gemm_fn("q5_0", "Batched GEMM on Q5_0 weights (new).")
gemm_q5k_f32 = _gemm_fn("q5k", "Batched GEMM on reference-layout Q5_K weights (new).")
gemm_q6k_f32 = _gemm_fn("q6k", "Batched GEMM on reference-layout Q6_K weights (new).")
gemm_q4_0g_f32 = _gemm_fn("q4_0g", "Batched GEMM on ggml-layout Q4_0 weights (new).")
gemm_q4kg_f32 = _gemm_fn("q4kg", "Batched GEMM on ggml-layout Q4_K weights (new).")
gemm_q5kg_f32 = _gemm_fn("q5kg", "Batched GEMM on ggml-layout Q5_K weights (new).")
gemm_q6kg_f32 = _gemm_fn("q6kg", "Batched GEMM on ggml-layout Q6_K weights (new).")


def argmax_f32(ctx, input, result, n):
    """greedy_argmax_f32 (sampler.rs:111-116) on the GPU."""
    _call(ctx, "rt_argmax_f32", _ptr(input), _ptr(result), n)


def argmax_f16(ctx, input, result, n):
    """dispatch.rs:1615-1631"""
    _call(ctx, "rt_argmax_f16", _ptr(input), _ptr(result), n)


def synth_normal_f32(ctx, out, n, seed, mean=0.0, std=1.0):
    _call(ctx, "rt_synth_normal_f32", _ptr(out), n, seed, mean, std)


def synth_normal_f16(ctx, out, n, seed, mean=0.0, std=1.0):
    _call(ctx, "rt_synth_normal_f16", _ptr(out), n, seed, mean, std)


def synth_weights(ctx, fmt: str, out, n_blocks, seed, std=0.02):
    """Seeded N(0, std) weights quantised per block (fmt in q8_0/q4_0/q4k/q6k/q5_0/q5k)."""
    _call(ctx, f"rt_synth_{fmt}", _ptr(out), n_blocks, seed, std)


# ───────────────────────────── decode-step glue ─────────────────────────────

def rms_norm_f32_f32_f32g(ctx, x, y, gamma, eps, hidden, num_rows):
    """dispatch.rs:177-200"""
    _call(ctx, "rt_rms_norm_f32_f32_f32g", _ptr(x), _ptr(y), _ptr(gamma), eps, hidden, num_rows)


def fused_rope_qk_f32(ctx, q, k, head_dim, q_heads, kv_heads, pos, theta):
    """dispatch.rs:945-971"""
    _call(ctx, "rt_fused_rope_qk_f32", _ptr(q), _ptr(k), head_dim, q_heads, kv_heads, pos, theta)


def kv_copy_to_cache_f32(ctx, src, dst, pos, max_seq, head_dim, num_kv_heads):
    """dispatch.rs:1183-1205"""
    _call(ctx, "rt_kv_copy_to_cache_f32", _ptr(src), _ptr(dst), pos, max_seq, head_dim,
          num_kv_heads)


def decode_attention_f32(ctx, q, k, v, out, batch, kv_len, num_heads, num_kv_heads, head_dim,
                         kv_head_stride):
    """dispatch.rs:1575-1612"""
    _call(ctx, "rt_decode_attention_f32", _ptr(q), _ptr(k), _ptr(v), _ptr(out), batch, kv_len,
          num_heads, num_kv_heads, head_dim, kv_head_stride)


def decode_attention_rope_f32(ctx, q_raw, k_raw, v_raw, k_cache, v_cache, out, pos, max_seq,
                              num_heads, num_kv_heads, head_dim, theta):
    """RoPE + KV-cache write + decode attention in one launch (new)."""
    _call(ctx, "rt_decode_attention_rope_f32", *map(_ptr, (q_raw, k_raw, v_raw, k_cache, v_cache,
                                                           out)),
          pos, max_seq, num_heads, num_kv_heads, head_dim, theta)


def decode_attention_rope_oproj_q8_0_f32(ctx, q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io,
                                         pos, max_seq, num_heads, num_kv_heads, head_dim, theta,
                                         hidden):
    """Attention (RoPE, KV write) and x_io += W_o·attention in two launches,
    the split merge folded into the projection's staging (new)."""
    _call(ctx, "rt_decode_attention_rope_oproj_q8_0_f32",
          *map(_ptr, (q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io)), pos, max_seq,
          num_heads, num_kv_heads, head_dim, theta, hidden)


def _attention_oproj(fmt):
    def fn(ctx, q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io, pos, max_seq, num_heads,
           num_kv_heads, head_dim, theta, hidden):
        _call(ctx, f"rt_decode_attention_rope_oproj_{fmt}_f32",
              *map(_ptr, (q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io)), pos, max_seq,
              num_heads, num_kv_heads, head_dim, theta, hidden)
    fn.__name__ = f"decode_attention_rope_oproj_{fmt}_f32"
    fn.__doc__ = (f"decode_attention_rope_oproj_q8_0_f32 for a {fmt} output projection (new).")
    return fn


def launch_count(ctx) -> int:
    """Kernel launches enqueued on the context so far (new)."""
    return int(ctx.lib.rt_launch_count(ctx.handle))


def last_launch_name(ctx) -> str:
    """Name of the kernel the context launched last (new)."""
    return ctx.lib.rt_last_launch_name(ctx.handle).decode()


decode_attention_rope_oproj_q4k_f32 = _attention_oproj("q4k")
decode_attention_rope_oproj_q4kg_f32 = _attention_oproj("q4kg")


def add_f16_into_f32(ctx, src, acc, n):
    """dispatch.rs:316-330: acc += f32(src) (f16 bias into an f32 vector)."""
    _call(ctx, "rt_add_f16_into_f32", _ptr(src), _ptr(acc), n)


def embed_f32(ctx, fmt: str, table, token, out, k):
    """Embedding row of the device-resident token id, dequantised from a
    `fmt` table (q8_0 … q6kg, f16, f32) (new)."""
    _call(ctx, f"rt_embed_{fmt}_f32", _ptr(table), _ptr(token), _ptr(out), k)


def embed_rows_f32(ctx, fmt: str, table, tokens, out, k, rows):
    """embed_f32 for `rows` device-resident token ids at once (new)."""
    _call(ctx, f"rt_embed_rows_{fmt}_f32", _ptr(table), _ptr(tokens), _ptr(out), k, rows)


# ──────────────────── multi-row GEMVs (verify / prefill) ────────────────────

def gemv_rows_f32(ctx, fmt, w, x, y, rows, n, k, gamma=None, eps=0.0):
    """y[rows][n] = (RMSNorm(x)·γ if gamma) · Wᵀ, weights read once per 8 rows (new)."""
    _call(ctx, f"rt_gemv_rows_{fmt}_f32", _ptr(w), _ptr(x), _ptr(gamma) if gamma else None, eps,
          _ptr(y), rows, n, k)


def gemv_rows_add_f32(ctx, fmt, w, x, res, y, rows, n, k):
    """y = res + x·Wᵀ for rows activation rows (new)."""
    _call(ctx, f"rt_gemv_rows_{fmt}_add_f32", _ptr(w), _ptr(x), _ptr(res), _ptr(y), rows, n, k)


def qkv_bias_rows_f32(ctx, fmt, wq, wk, wv, x, q, k_out, v, bq, bk, bv, rows, q_dim, kv_dim, k,
                      gamma=None, eps=0.0):
    """Q/K/V (+ f16 bias) of rows activation rows; a None weight skips its matrix (new)."""
    p = lambda b: _ptr(b) if b is not None else None
    _call(ctx, f"rt_qkv_bias_rows_{fmt}_f32", p(wq), p(wk), p(wv), _ptr(x), p(gamma), eps,
          p(q), p(k_out), p(v), p(bq), p(bk), p(bv), rows, q_dim, kv_dim, k)


def fused_ffn_rows_f32(ctx, fmt, wg, wu, x, act, rows, ff, k, gamma=None, eps=0.0):
    """act = silu(x̂·W_gᵀ)·(x̂·W_uᵀ) for rows activation rows (new)."""
    _call(ctx, f"rt_fused_ffn_rows_{fmt}_f32", _ptr(wg), _ptr(wu), _ptr(x),
          _ptr(gamma) if gamma is not None else None, eps, _ptr(act), rows, ff, k)


# ──────────────────── batched verify / prefill glue ────────────────────

def add_bias_broadcast_f32(ctx, x, bias, seq, dim):
    """dispatch.rs:1660-1680: x[s][i] += f32(bias[i])."""
    _call(ctx, "rt_add_bias_broadcast_f32", _ptr(x), _ptr(bias), seq, dim)


def rope_batch_inplace_f32(ctx, x, head_dim, num_heads, start_pos, theta, seq):
    """dispatch.rs:1125-1150: row s of [seq][heads][hd] rotated at start_pos + s."""
    _call(ctx, "rt_rope_batch_inplace_f32", _ptr(x), head_dim, num_heads, start_pos, theta, seq)


def kv_write_batch_f32(ctx, k, v, k_cache, v_cache, start_pos, seq, max_seq, head_dim,
                       num_kv_heads):
    """KvCache::write_at (kv_cache.rs:132-150) for seq consecutive positions."""
    _call(ctx, "rt_kv_write_batch_f32", *map(_ptr, (k, v, k_cache, v_cache)), start_pos, seq,
          max_seq, head_dim, num_kv_heads)


def rope_kv_write_batch_f32(ctx, q, k, v, k_cache, v_cache, head_dim, num_heads, num_kv_heads,
                            start_pos, theta, seq, max_seq):
    """Batched RoPE of q and k + KV-cache write of k and v in one launch (new)."""
    _call(ctx, "rt_rope_kv_write_batch_f32", *map(_ptr, (q, k, v, k_cache, v_cache)), head_dim,
          num_heads, num_kv_heads, start_pos, theta, seq, max_seq)


def flash_attention_f32(ctx, q, k, v, out, batch, q_len, kv_len, num_heads, num_kv_heads,
                        head_dim, kv_head_stride, q_start=0):
    """dispatch.rs:645-687 (causal; row r sees positions ≤ q_start + r)."""
    _call(ctx, "rt_flash_attention_f32", *map(_ptr, (q, k, v, out)), batch, q_len, kv_len,
          num_heads, num_kv_heads, head_dim, kv_head_stride, q_start)


def add_f32(ctx, a, b, out, n):
    """dispatch.rs:57-75 on f32: out = a + b."""
    _call(ctx, "rt_add_f32", _ptr(a), _ptr(b), _ptr(out), n)


def silu_mul_f32(ctx, gate, up, out, n):
    """dispatch.rs:35-55: out = silu(gate)·up."""
    _call(ctx, "rt_silu_mul_f32", _ptr(gate), _ptr(up), _ptr(out), n)


def argmax_rows_first_f32(ctx, input, result, rows, n):
    """verify_draft's per-row argmax (forward.rs:2283-2293): first max wins."""
    _call(ctx, "rt_argmax_rows_first_f32", _ptr(input), _ptr(result), rows, n)


def embed_q8_0_f32(ctx, table, token, out, k):
    """Q8_0 embedding row of the device-resident token id (new)."""
    embed_f32(ctx, "q8_0", table, token, out, k)


def rms_norm_fused_qkv_bias_q8_0_f32(ctx, w_q, w_k, w_v, x, gamma, eps, out_q, out_k, out_v,
                                     bias_q, bias_k, bias_v, q_dim, kv_dim, k):
    """rms_norm_f32_f32_f32g + fused_qkv_bias_q8_0_f32 in one launch (new)."""
    _call(ctx, "rt_rms_norm_fused_qkv_bias_q8_0_f32", _ptr(w_q), _ptr(w_k), _ptr(w_v), _ptr(x),
          _ptr(gamma), eps, *map(_ptr, (out_q, out_k, out_v, bias_q, bias_k, bias_v)),
          q_dim, kv_dim, k)


def rms_norm_fused_qkv_bias_q8_0_f32_ssq(ctx, w_q, w_k, w_v, x, gamma, eps, out_q, out_k, out_v,
                                         bias_q, bias_k, bias_v, q_dim, kv_dim, k, ssq, nparts):
    """rms_norm_fused_qkv_bias_q8_0_f32 with Σx² given as the producing
    launch's nparts partial sums (new)."""
    _call(ctx, "rt_rms_norm_fused_qkv_bias_q8_0_f32_ssq", _ptr(w_q), _ptr(w_k), _ptr(w_v),
          _ptr(x), _ptr(gamma), eps, *map(_ptr, (out_q, out_k, out_v, bias_q, bias_k, bias_v)),
          q_dim, kv_dim, k, _ptr(ssq), nparts)


def rms_norm_fused_ffn_q8_0_f32_ssq(ctx, w_gate, w_up, x, gamma, eps, act_out, ff_dim, k, ssq,
                                    nparts):
    """rms_norm_fused_ffn_q8_0_f32 with Σx² given as partial sums (new)."""
    _call(ctx, "rt_rms_norm_fused_ffn_q8_0_f32_ssq", _ptr(w_gate), _ptr(w_up), _ptr(x),
          _ptr(gamma), eps, _ptr(act_out), ff_dim, k, _ptr(ssq), nparts)


def gemv_q8_0_add_f32_f32in_ssq(ctx, weight, input, output, residual, m, k, ssq):
    """gemv_q8_0_add_f32_f32in that also writes Σy² per 4 output rows (new)."""
    _call(ctx, "rt_gemv_q8_0_add_f32_f32in_ssq", *map(_ptr, (weight, input, output, residual)),
          m, k, _ptr(ssq))


def decode_attention_rope_oproj_q8_0_f32_ssq(ctx, q_raw, k_raw, v_raw, k_cache, v_cache, w_o,
                                             x_io, pos, max_seq, num_heads, num_kv_heads,
                                             head_dim, theta, hidden, ssq):
    """decode_attention_rope_oproj_q8_0_f32 that also writes Σy² per 4 rows
    of the updated x (new)."""
    _call(ctx, "rt_decode_attention_rope_oproj_q8_0_f32_ssq",
          *map(_ptr, (q_raw, k_raw, v_raw, k_cache, v_cache, w_o, x_io)), pos, max_seq,
          num_heads, num_kv_heads, head_dim, theta, hidden, _ptr(ssq))


def rms_norm_fused_qkv_bias_q4k_q6k_f32(ctx, w_q, w_k, w_v, x, gamma, eps, out_q, out_k, out_v,
                                       bias_q, bias_k, bias_v, q_dim, kv_dim, k):
    """rms_norm_f32_f32_f32g + fused_qkv_bias_q4k_q6k_f32 in one launch (new)."""
    _call(ctx, "rt_rms_norm_fused_qkv_bias_q4k_q6k_f32", _ptr(w_q), _ptr(w_k), _ptr(w_v), _ptr(x),
          _ptr(gamma), eps, *map(_ptr, (out_q, out_k, out_v, bias_q, bias_k, bias_v)),
          q_dim, kv_dim, k)


def rms_norm_fused_ffn_q4k_f32(ctx, w_gate, w_up, x, gamma, eps, act_out, ff_dim, k):
    """rms_norm_f32_f32_f32g + fused_ffn_q4k_f32 in one launch (new)."""
    _call(ctx, "rt_rms_norm_fused_ffn_q4k_f32", _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(gamma),
          eps, _ptr(act_out), ff_dim, k)


def rms_norm_gemv_q6k_f32in_f32out(ctx, weight, x, gamma, eps, output, m, k):
    """rms_norm_f32_f32_f32g + gemv_q6k_f32in_f32out in one launch (new)."""
    _call(ctx, "rt_rms_norm_gemv_q6k_f32in_f32out", _ptr(weight), _ptr(x), _ptr(gamma), eps,
          _ptr(output), m, k)


def rms_norm_fused_ffn_q8_0_f32(ctx, w_gate, w_up, x, gamma, eps, act_out, ff_dim, k):
    """rms_norm_f32_f32_f32g + fused_ffn_q8_0_f32 in one launch (new)."""
    _call(ctx, "rt_rms_norm_fused_ffn_q8_0_f32", _ptr(w_gate), _ptr(w_up), _ptr(x), _ptr(gamma),
          eps, _ptr(act_out), ff_dim, k)


def rms_norm_gemv_q8_0_f32in_f32out(ctx, weight, x, gamma, eps, output, m, k):
    """rms_norm_f32_f32_f32g + gemv_q8_0_f32in_f32out in one launch (new)."""
    _call(ctx, "rt_rms_norm_gemv_q8_0_f32in_f32out", _ptr(weight), _ptr(x), _ptr(gamma), eps,
          _ptr(output), m, k)


def stream_read(ctx, src, nbytes, sink, sink_dwords):
    """Calibration: plain HBM read of nbytes."""
    _call(ctx, "rt_stream_read", _ptr(src), nbytes, _ptr(sink), sink_dwords)


def stream_copy(ctx, dst, src, nbytes):
    """Calibration: plain HBM copy of nbytes."""
    _call(ctx, "rt_stream_copy", _ptr(dst), _ptr(src), nbytes)


# Block geometry (crates/gguf/src/types.rs:158-191).
BLOCK = {"q8_0": (32, 34), "q4_0": (32, 18), "q4k": (256, 144), "q6k": (256, 210),
         "q5_0": (32, 22), "q5k": (256, 176),
         "q4_0g": (32, 18), "q4kg": (256, 144), "q5kg": (256, 176), "q6kg": (256, 210)}


def weight_bytes(fmt: str, n: int, k: int) -> int:
    el, by = BLOCK[fmt]
    return n * (k // el) * by
