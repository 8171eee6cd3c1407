"""The device generators (rt_synth_*) against the oracle's BASELINE
definitions, byte for byte: every GPU test and bench input is built by them,
so "identical seeded inputs" means these bytes.

Config 1 defines W as N(0, 0.02) weights quantised per 32-element block (Q8_0:
d = f16(max|w|/127), q = round(w/d)); configs 3-4 define Q4_0 / Q4_K / Q6_K
the same way.  The oracle restates those quantisers (ora_quantize_*) and the
normal stream (splitmix64 → Box–Muller, pinned against libm in
test_oracle.py); here the device must reproduce them exactly."""
import numpy as np
import pytest

import oracle_lib as ora
from runit_mac_amd import dispatch as d

pytestmark = pytest.mark.gpu

FMTS = ["q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k"]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("seed", [0, 7, 123456789])
def test_device_synth_weights_byte_identical(ctx, fmt, seed):
    el, by = d.BLOCK[fmt]
    n, k = 96, 2048  # 6,144 Q8_0 blocks / 768 super-blocks
    nbytes = d.weight_bytes(fmt, n, k)
    buf = ctx.new_buffer(nbytes)
    d.synth_weights(ctx, fmt, buf, n * k // el, seed, 0.02)
    ctx.flush()
    got = buf.read(np.uint8, nbytes)
    ref = ora.synth_weights(fmt, n, k, seed, 0.02)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, (fmt, seed, f"{bad.size} bytes differ, first at block {bad[0] // by}")
    buf.free()


def test_device_synth_weights_config1_full_size(ctx):
    """The config-1 matrix itself (4864×896 Q8_0, the bench's seed)."""
    n, k = 4864, 896
    nbytes = d.weight_bytes("q8_0", n, k)
    buf = ctx.new_buffer(nbytes)
    d.synth_weights(ctx, "q8_0", buf, n * k // 32, 1, 0.02)
    ctx.flush()
    assert np.array_equal(buf.read(np.uint8, nbytes), ora.synth_weights("q8_0", n, k, 1, 0.02))
    buf.free()


@pytest.mark.parametrize("mean,std", [(0.0, 1.0), (1.0, 0.02)])
def test_device_synth_normal_bit_identical(ctx, mean, std):
    n = 100_003
    buf = ctx.new_buffer(4 * n)
    d.synth_normal_f32(ctx, buf, n, 42, mean, std)
    h = ctx.new_buffer(2 * n + 2)
    d.synth_normal_f16(ctx, h, n, 42, mean, std)
    ctx.flush()
    ref = ora.synth_normal(42, n, mean=mean, std=std)
    assert np.array_equal(buf.read(np.float32, n).view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(h.read(np.uint16, n), ref.astype(np.float16).view(np.uint16))
    buf.free()
    h.free()
