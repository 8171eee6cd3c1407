"""Writes GGUF v2/v3 files for the tests (test infrastructure only).

Follows the layout the reference's parser reads (crates/gguf/src/parser.rs:
22-57 and its test builder): magic, version, tensor count, metadata count,
metadata (key, type, value), tensor infos (name, n_dims, dims, dtype,
offset), padding to the alignment, then tensor data at the recorded offsets.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v) -> bytes:
    if t == STR:
        return _s(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, i) for i in items)
    return struct.pack(_FMT[t], v)


def build(metadata, tensors, version=3, alignment=None) -> bytes:
    """metadata: list of (key, type, value) (arrays: (ARR, (elem_type, items)));
    tensors: list of (name, dims, dtype_id, raw bytes)."""
    align = alignment or 32
    md = list(metadata)
    if alignment is not None:
        md.append(("general.alignment", U32, alignment))
    out = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(md))
    for k, t, v in md:
        out += _s(k) + struct.pack("<I", t) + _value(t, v)
    off = 0
    offs = []
    for name, dims, dt, raw in tensors:
        offs.append(off)
        out += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", x) for x in dims)
        out += struct.pack("<IQ", dt, off)
        off += (len(raw) + align - 1) // align * align
    out += b"\0" * ((-len(out)) % align)
    for (name, dims, dt, raw), o in zip(tensors, offs):
        out += bytes(raw) + b"\0" * ((-len(raw)) % align)
    return out


def write(path, metadata, tensors, **kw) -> None:
    with open(path, "wb") as f:
        f.write(build(metadata, tensors, **kw))


def reference_test_gguf() -> bytes:
    """The byte string of the reference's parser test (parser.rs:240-283):
    general.architecture = "qwen2", one F32 tensor "test.weight" [4, 8] with
    values 0..31, data aligned to 32."""
    return build([("general.architecture", STR, "qwen2")],
                 [("test.weight", [4, 8], 0, np.arange(32, dtype=np.float32).tobytes())])
