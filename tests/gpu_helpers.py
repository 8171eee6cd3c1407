"""Shared helpers for the GPU parity tests (tolerances are stated here)."""
from __future__ import annotations

import numpy as np

import oracle_lib as ora
from runit_mac_amd import dispatch as d

# BASELINE tolerance: every output satisfies |y − y_ref| ≤ 1e-4 · Σ_i |w_i·x_i|
# (fp32 accumulate), against the f64 oracle on identical inputs.
REL = 1e-4
F16_HALF_ULP = 2.0 ** -11  # relative half-ulp of binary16 (normal range)
F16_SUB = 2.0 ** -25       # half the smallest binary16 subnormal
F32_EPS = 2.0 ** -24


GGML = ("q4_0g", "q4kg", "q5kg", "q6kg")


def ggml_from_reference(fmt: str, raw: np.ndarray) -> np.ndarray:
    """ggml-layout bytes for a reference-layout stream (values preserved;
    Q6_K's odd scale slots, unused by the reference layout, get a value next
    to their even neighbour so that the 16-scale indexing is exercised)."""
    base = fmt[:-1]
    if base != "q6k":
        return ora.relayout_to_ggml(base, raw)
    blk = raw.reshape(-1, 210).copy()
    sc = blk[:, 192:208].view(np.int8)
    delta = (np.arange(blk.shape[0])[:, None] + np.arange(8)[None, :]) % 5 - 2
    sc[:, 1::2] = np.clip(sc[:, 0::2].astype(np.int32) + delta, -127, 127).astype(np.int8)
    return blk.reshape(-1)


def device_weights(ctx, fmt: str, n: int, k: int, seed: int, std: float = 0.02):
    """Generates N(0, std) weights quantised per block on the device and
    returns (device buffer, host copy of the packed bytes).  ggml layouts:
    the reference-layout stream re-laid out on the host."""
    if fmt in GGML:
        buf, raw = device_weights(ctx, fmt[:-1], n, k, seed, std)
        g = ggml_from_reference(fmt, raw)
        buf.write(g)
        return buf, g
    nbytes = d.weight_bytes(fmt, n, k)
    buf = ctx.new_buffer(nbytes)
    el, _ = d.BLOCK[fmt]
    d.synth_weights(ctx, fmt, buf, n * k // el, seed, std)
    ctx.flush()
    return buf, buf.read(np.uint8, nbytes)


def device_normal(ctx, n: int, seed: int, mean=0.0, std=1.0):
    buf = ctx.new_buffer(max(4 * n, 16))
    d.synth_normal_f32(ctx, buf, n, seed, mean, std)
    ctx.flush()
    return buf, buf.read(np.float32, n)


def check_close(got: np.ndarray, ref: np.ndarray, sabs: np.ndarray, what: str,
                extra: np.ndarray | float = 0.0):
    got = got.astype(np.float64)
    tol = REL * sabs + extra
    err = np.abs(got - ref)
    bad = ~(err <= tol)
    if bad.any():
        i = int(np.argmax(np.where(bad, err / np.maximum(tol, 1e-300), 0)))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{got.size} outside tolerance; worst row {i}: "
            f"got {got[i]!r} ref {ref[i]!r} |err| {err[i]:.3e} tol {tol[i]:.3e}")


def f16_extra(ref: np.ndarray, sabs: np.ndarray) -> np.ndarray:
    """Extra allowance for an f16 output: one RNE rounding of a value already
    within REL·sabs of ref."""
    return F16_HALF_ULP * (np.abs(ref) + REL * sabs) + F16_SUB


def f16_to_f64(u16: np.ndarray) -> np.ndarray:
    return u16.view(np.float16).astype(np.float64)
