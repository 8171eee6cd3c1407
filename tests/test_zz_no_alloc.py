"""The no-allocation entry point rt_gemv_q6k_add_f32_f32in_noalloc (no
reference counterpart; for callers that cannot allocate device memory):
through the C ABI, two calls in a row — the second with a smaller input —
each bit-identical to rt_gemv_q6k_add_f32_f32in (the same kernels) and
within the BASELINE tolerance of the oracle, plus the size limit."""
import ctypes

import numpy as np
import pytest

import oracle_lib as ora
from gpu_helpers import check_close, device_normal, device_weights
from runit_mac_amd import dispatch as d

pytestmark = pytest.mark.gpu


def _run(ctx, fn, w, x, res, n, k):
    y = ctx.buffer_from(res)
    fn(ctx, w, x, y, y, n, k)  # output aliases the residual, as forward.rs:1702
    ctx.flush()
    return y.read(np.float32, n)


# K = 24576: past the workgroup-local K split's record limit, so both calls
# split K through the scratch (the LDS-streamed body, then the matrix-core
# body for the smaller one)
@pytest.mark.parametrize("shapes", [((3584, 24576), (512, 24576))])
def test_noalloc_matches_allocating_entry_point(ctx, shapes):
    for i, (n, k) in enumerate(shapes):
        print(f"noalloc call {i}: q6k add {n}x{k}", flush=True)
        w, raw = device_weights(ctx, "q6k", n, k, 500 + i)
        xb, x = device_normal(ctx, k, 600 + i)
        res = np.random.default_rng(700 + i).standard_normal(n).astype(np.float32)
        got = _run(ctx, d.gemv_q6k_add_f32_f32in_noalloc, w, xb, res, n, k)
        ref = _run(ctx, d.gemv_q6k_add_f32_f32in, w, xb, res, n, k)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (n, k)
        yref, sabs = ora.gemv("q6k", raw, x, n, k)
        check_close(got, yref + res, sabs, f"noalloc q6k {n}x{k}")
        w.free()
        xb.free()


def test_noalloc_rejects_oversized_split(ctx):
    """49152×65536 Q6_K: 16 K chunks × 49152 rows of partial sums (3 MiB)
    exceed the scratch's partial-sum region: a clear error.  The buffers are
    real allocations of the full size (weights uninitialised), so the call is
    safe whatever it does."""
    n, k = 49152, 65536
    w = ctx.new_buffer(d.weight_bytes("q6k", n, k))
    x, y = ctx.new_buffer(4 * k), ctx.new_buffer(4 * n)
    lib = d.load_library()
    st = lib.rt_gemv_q6k_add_f32_f32in_noalloc(ctx.handle, w.ptr, x.ptr, y.ptr, y.ptr, n, k)
    ctx.flush()
    assert st != 0
    assert b"scratch" in lib.rt_last_error(ctx.handle)
    for b in (w, x, y):
        b.free()
