"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

The reference's own tests hold no golden vectors for quantized GEMV, fused
QKV/FFN, Q4_0, Q4_K or Q6_K numerics (its only kernel tests are f16 GEMV /
attention / norm tests, crates/kernels/src/dispatch.rs:1777-2004).  So each
oracle function is pinned here by checks that a plausible mistake would fail:
hand-built known-answer blocks for every layout quirk of the reference, the
reference's own zero-quant fixtures (crates/engine/tests/qwen2_load_test.rs:
105-134), the closed-form GEMV cases of crates/engine/src/bin/test_gemv.rs:
58-85 re-expressed with quantized blocks, an independent library routine
(numpy's IEEE float16 conversion), brute-force dot products, invariants of the
quantisers, and the Rust `max_by` fold semantics for argmax.
"""
import struct

import numpy as np
import pytest

import oracle_lib as ora


def h16(v: float) -> bytes:
    return np.float16(v).tobytes()


# ───────────────────────── f16 conversions ─────────────────────────

def test_h2f_all_halves_match_numpy():
    hs = np.arange(65536, dtype=np.uint16)
    ref = hs.view(np.float16).astype(np.float32)
    got = np.array([ora.h2f(int(h)) for h in hs], dtype=np.float32)
    both_nan = np.isnan(ref) & np.isnan(got)
    assert np.array_equal(ref.view(np.uint32)[~both_nan], got.view(np.uint32)[~both_nan])


def test_f2h_round_to_nearest_even_matches_numpy():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        # exact ties between adjacent halves, subnormal ties, overflow edge
        (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),
        (np.arange(0, 1024, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
        np.array([65504, 65519.99, 65520, 65536, 1e-8, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                  -0.0, np.inf, -np.inf], dtype=np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([ora.f2h(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(ref, got)


# ───────────────────────── dequant known answers ─────────────────────────

def test_q8_0_known_block():
    # d = 1, q = i − 16  →  v = i − 16 ; second block d = 0.5 → halves
    b1 = h16(1.0) + bytes((i - 16) & 255 for i in range(32))
    b2 = h16(0.5) + bytes((i - 16) & 255 for i in range(32))
    v = ora.dequant("q8_0", np.frombuffer(b1 + b2, np.uint8))
    assert np.array_equal(v[:32], np.arange(32) - 16)
    assert np.array_equal(v[32:], (np.arange(32) - 16) * 0.5)


def test_q4_0_reference_nibble_order():
    # byte i holds element 2i (low nibble) and 2i+1 (high nibble)
    # (gemv_q4_0.metal:13-14, forward.rs:974-976) — not ggml's j / j+16 split.
    qs = bytes(((2 * i) & 15) | (((2 * i + 1) & 15) << 4) for i in range(16))
    v = ora.dequant("q4_0", np.frombuffer(h16(2.0) + qs, np.uint8))
    expect = 2.0 * (((np.arange(32)) & 15) - 8)
    assert np.array_equal(v, expect)
    # a single byte 0x21 → elements [1−8, 2−8]
    qs = bytes([0x21]) + bytes([0x88] * 15)
    v = ora.dequant("q4_0", np.frombuffer(h16(1.0) + qs, np.uint8))
    assert v[0] == -7 and v[1] == -6 and np.all(v[2:] == 0)


def _q4k_block(d, dmin, sc, m, q):
    """Packs a Q4_K block with 6-bit (sc, m) per scale index s (0..7) and
    4-bit codes q[256] in the reference layout (element 64j+l low nibble,
    64j+32+l high nibble of qs[32j+l])."""
    S = [0] * 12
    for j in range(4):
        S[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        S[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        S[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    qs = bytearray(128)
    for j in range(4):
        for l in range(32):
            qs[32 * j + l] = q[64 * j + l] | (q[64 * j + 32 + l] << 4)
    return h16(d) + h16(dmin) + bytes(S) + bytes(qs)


def test_q4k_scale_pairing_j_and_j_plus_4():
    # Only scale index 5 (= pair j=1, high nibbles) is non-zero: elements
    # 96..127 get d·sc5·q; the reference pairs (j, j+4), ggml pairs (2j, 2j+1),
    # which would light up elements 160..191 instead.
    sc = [0, 0, 0, 0, 0, 37, 0, 0]
    m = [0] * 8
    q = [(i * 7) & 15 for i in range(256)]
    v = ora.dequant("q4k", np.frombuffer(_q4k_block(0.25, 0.0, sc, m, q), np.uint8))
    nz = np.nonzero(v)[0]
    assert nz.min() >= 96 and nz.max() <= 127
    for e in range(96, 128):
        assert v[e] == np.float32(0.25 * 37) * np.float32(q[e])


def test_q4k_six_bit_high_scales_and_mins():
    # 6-bit values ≥ 16 in scale indices 4..7 exercise the split packing
    # (low 4 bits in bytes 8..11, top 2 bits in bytes 0..7) of get_scale_min_k4
    sc = [1, 2, 3, 4, 63, 17, 48, 33]
    m = [5, 6, 7, 8, 62, 31, 16, 47]
    q = [((i * 5) + 3) & 15 for i in range(256)]
    d, dmin = 0.0625, 0.03125
    v = ora.dequant("q4k", np.frombuffer(_q4k_block(d, dmin, sc, m, q), np.uint8))
    for e in range(256):
        s = (e // 64) + 4 * ((e // 32) & 1)
        expect = np.float32(np.float32(d * sc[s]) * np.float32(q[e])) - np.float32(dmin * m[s])
        assert v[e] == expect, e


def test_q4k_zero_quant_fixture_from_reference_test():
    # qwen2_load_test.rs:105-119: d = 1, dmin = 0, scales = 0, qs = 0
    blk = bytearray(144)
    blk[0:2] = h16(1.0)
    v = ora.dequant("q4k", np.frombuffer(bytes(blk) * 3, np.uint8))
    assert np.all(v == 0)


def _q6k_block(d, sc16, q):
    ql = bytearray(128)
    qh = bytearray(64)
    for h in (0, 128):
        for l in range(32):
            q1, q2, q3, q4 = q[h + l], q[h + l + 32], q[h + l + 64], q[h + l + 96]
            ql[h // 2 + l] = (q1 & 15) | ((q3 & 15) << 4)
            ql[h // 2 + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            qh[h // 4 + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    return bytes(ql) + bytes(qh) + bytes(s & 255 for s in sc16) + h16(d)


def test_q6k_only_even_scale_slots_are_read():
    # forward.rs:935 uses is = n_half/16 and slots is+0,2,4,6: the odd slots
    # (which ggml would use for elements 16..31 of each 32) are ignored.
    q = [(i * 11 + 5) % 64 for i in range(256)]
    sc_a = [3, -7, 5, 9, -2, 4, 6, 1, -8, 2, 7, -5, 11, 3, -1, 6]
    sc_b = list(sc_a)
    for i in range(1, 16, 2):
        sc_b[i] = 100 - i
    va = ora.dequant("q6k", np.frombuffer(_q6k_block(0.5, sc_a, q), np.uint8))
    vb = ora.dequant("q6k", np.frombuffer(_q6k_block(0.5, sc_b, q), np.uint8))
    assert np.array_equal(va, vb)
    for e in range(256):
        h, t = (e // 128) * 128, (e % 128) // 32
        s = sc_a[h // 16 + 2 * t]
        assert va[e] == np.float32(np.float32(0.5 * s) * np.float32(q[e] - 32)), e


def test_q6k_zero_quant_fixture_from_reference_test():
    # qwen2_load_test.rs:121-134: d = 1, ql = qh = scales = 0 → d·0·(0−32) = −0.0
    blk = bytearray(210)
    blk[208:210] = h16(1.0)
    v = ora.dequant("q6k", np.frombuffer(bytes(blk), np.uint8))
    assert np.all(v == 0) and np.all(np.signbit(v))


def test_q4k_f16_matches_f32_then_rne():
    rng = np.random.default_rng(3)
    raw = ora.synth_weights("q4k", 4, 256, seed=5)
    v32 = ora.dequant("q4k", raw)
    v16 = ora.dequant_q4k_f16(raw)
    assert np.array_equal(v32.astype(np.float16).view(np.uint16), v16)
    del rng


# ───────────────────────── GEMV closed forms / brute force ─────────────────────────

def _ones_blocks(fmt, n, k):
    """Blocks whose every element decodes to exactly 1.0."""
    if fmt == "q8_0":
        blk = h16(1.0) + bytes([1] * 32)
        nb = k // 32
    elif fmt == "q4_0":
        blk = h16(1.0) + bytes([0x99] * 16)  # nib 9 → 9 − 8 = 1
        nb = k // 32
    elif fmt == "q4k":
        blk = _q4k_block(1.0, 0.0, [1] * 8, [0] * 8, [1] * 256)
        nb = k // 256
    else:
        blk = _q6k_block(1.0, [1] * 16, [33] * 256)
        nb = k // 256
    return np.frombuffer(blk * (n * nb), np.uint8)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4k", "q6k"])
def test_gemv_all_ones_closed_form(fmt):
    # test_gemv.rs:58-85: all-ones 32×32 · [1..32] = 528 per row; at K=256:
    # Σ 1..256 = 32896.
    k = 32 if fmt in ("q8_0", "q4_0") else 256
    n = 5
    w = _ones_blocks(fmt, n, k)
    x = np.arange(1, k + 1, dtype=np.float32)
    y, s = ora.gemv(fmt, w, x, n, k)
    assert np.all(y == k * (k + 1) / 2)
    assert np.all(s == k * (k + 1) / 2)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg",
                                 "q5kg", "q6kg"])
def test_gemv_brute_force(fmt):
    n, k = 7, 512
    w = ora.synth_weights(fmt, n, k, seed=11)
    x = np.random.default_rng(2).standard_normal(k).astype(np.float32)
    y, s = ora.gemv(fmt, w, x, n, k)
    W = ora.dequant(fmt, w).reshape(n, k).astype(np.float64)
    for r in range(n):
        acc = 0.0
        sa = 0.0
        for c in range(k):
            acc += W[r, c] * float(x[c])
            sa += abs(W[r, c] * float(x[c]))
        assert abs(acc - y[r]) <= 1e-12 * sa
        assert abs(sa - s[r]) <= 1e-12 * sa
    # identity-like: one-hot x picks a column exactly
    e = np.zeros(k, np.float32)
    e[37] = 1.0
    y1, _ = ora.gemv(fmt, w, e, n, k)
    assert np.array_equal(y1, W[:, 37])


def test_gemv_ref_f32_is_sequential_f32_sum():
    n, k = 3, 64
    w = ora.synth_weights("q8_0", n, k, seed=4)
    x = np.random.default_rng(5).standard_normal(k).astype(np.float32)
    W = ora.dequant("q8_0", w).reshape(n, k)
    y = ora.gemv_ref_f32("q8_0", w, x, n, k)
    for r in range(n):
        acc = np.float32(0.0)
        for c in range(k):
            acc = np.float32(acc + np.float32(W[r, c] * x[c]))
        assert y[r] == acc


# ───────────────────────── silu / argmax ─────────────────────────

def test_silu_closed_forms():
    assert ora.silu(0.0) == 0.0
    assert abs(ora.silu(1.0) - 1.0 / (1.0 + np.exp(-1.0))) < 1e-15
    assert abs(ora.silu(-30.0)) < 1e-11
    assert abs(ora.silu(30.0) - 30.0) < 1e-11


def test_argmax_rust_max_by_semantics():
    nan = np.float32("nan")
    cases = [
        ([], 0),
        ([5.0], 0),
        ([1.0, 3.0, 3.0, 2.0], 2),             # ties → last maximal index
        ([3.0, 1.0, 3.0], 2),
        ([-np.inf, -np.inf], 1),
        ([1.0, nan, 0.5], 2),                  # NaN compares Equal: replaced, then replaced
        ([9.0, 1.0, nan], 2),                  # trailing NaN wins
        ([nan, 2.0, 7.0, 3.0], 2),
        ([4.0, nan, 1.0, 2.0, 2.0], 4),
    ]
    for vals, expect in cases:
        assert ora.argmax(np.array(vals, np.float32)) == expect, vals


# ───────────────────────── quantiser invariants ─────────────────────────

@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k", "q4_0g", "q4kg",
                                 "q5kg"])
def test_quantizer_round_trip_error_bounded(fmt):
    n_el = 256 * 16
    w = (0.02 * ora.synth_normal(99, n_el)).astype(np.float32)
    v = ora.dequant(fmt, ora.quantize(fmt, w))
    err = np.abs(v - w)
    el = 32 if fmt in ("q8_0", "q4_0", "q5_0", "q4_0g") else 256
    amax = np.abs(w).reshape(-1, el).max(axis=1).repeat(el)
    # half a step plus the f16 rounding of the scale: Q8_0 step amax/127
    # (q uses the unrounded d, so up to 127·2^-11 steps more), Q4_0 amax/8
    # (plus one clamped step at +8), Q4_K ≈ range/15, Q6_K amax/32
    # Q5_0 amax/16 (plus one clamped step at +16), Q5_K ≈ range/31
    bound = {"q8_0": 0.6 / 127, "q4_0": 1.01 / 8, "q4k": 0.2, "q6k": 0.08, "q5_0": 1.01 / 16,
             "q5k": 0.1, "q4_0g": 1.01 / 8, "q4kg": 0.2, "q5kg": 0.1}[fmt]
    assert np.all(err <= bound * amax + 1e-7)


def test_synth_normal_moments():
    z = ora.synth_normal(7, 20000)
    assert abs(z.mean()) < 0.03 and abs(z.std() - 1.0) < 0.03


def _splitmix64(z: int) -> int:
    m = (1 << 64) - 1
    z = (z + 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def test_synth_normal_is_box_muller_of_splitmix():
    """The generator's definition, written independently with Python's
    integers and libm in f64: u1 = (h>>40 + 1)·2^-24, u2 = (h & 2^24−1)·2^-24,
    z = √(−2 ln u1)·cos(2π u2).  The oracle's own ln / cos (correctly rounded
    f32 operations only, so that the device reproduces its bits) stay within
    a few f32 ulps of it."""
    import math
    seed, n = 1234, 4000
    got = ora.synth_normal(seed, n).astype(np.float64)
    worst = 0.0
    for i in range(n):
        h = _splitmix64(seed ^ _splitmix64(i))
        u1 = ((h >> 40) + 1) * 2.0 ** -24
        u2 = (h & 0xFFFFFF) * 2.0 ** -24
        z = math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)
        worst = max(worst, abs(got[i] - z) / max(1.0, abs(z)))
    assert worst < 4e-6, worst
    # shifted windows are slices of the same stream; mean / std scale in f32
    assert np.array_equal(ora.synth_normal(seed, 10, start=100), ora.synth_normal(seed, 110)[100:])
    z32 = ora.synth_normal(seed, 64)
    assert np.array_equal(ora.synth_normal(seed, 64, mean=1.0, std=0.02),
                          np.float32(1.0) + np.float32(0.02) * z32)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4k", "q6k", "q5_0", "q5k"])
def test_synth_weights_are_the_quantised_stream(fmt):
    """synth_weights(fmt) = the BASELINE quantiser applied to 0.02·N(seed, i)."""
    el, _ = ora.BLOCK[fmt]
    n, k = 8, 2 * 256
    raw = ora.synth_weights(fmt, n, k, seed=77)
    w = np.float32(0.02) * ora.synth_normal(77, n * k)
    assert np.array_equal(raw, ora.quantize(fmt, w))


# ───────────────────────── decode glue oracles ─────────────────────────

def test_rms_norm_closed_forms():
    # constant vector c: mean(x²) = c², so y = c/|c| · γ (eps → 0)
    x = np.full(64, -3.0, np.float32)
    g = np.linspace(0.5, 2.0, 64).astype(np.float32)
    y = ora.rms_norm(x, g, 0.0)
    assert np.allclose(y, -1.0 * g, rtol=0, atol=1e-12)
    # scale invariance: rms_norm(a·x) = rms_norm(x) for a > 0 (eps = 0)
    x = np.random.default_rng(0).standard_normal((3, 128)).astype(np.float32)
    g = np.ones(128, np.float32)
    assert np.allclose(ora.rms_norm(x, g, 0.0), ora.rms_norm(4 * x, g, 0.0), atol=1e-12)


def test_rope_pos0_identity_and_pair_norms():
    v = np.random.default_rng(1).standard_normal(4 * 64)
    assert np.array_equal(ora.rope(v, 4, 64, 0, 1e6), v)
    r = ora.rope(v, 4, 64, 511, 1e6).reshape(4, 64)
    vv = v.reshape(4, 64)
    # each (d, d+32) pair is rotated: its norm is preserved
    assert np.allclose(r[:, :32] ** 2 + r[:, 32:] ** 2, vv[:, :32] ** 2 + vv[:, 32:] ** 2,
                       rtol=1e-12)
    # pair 0 has frequency 1: angle = pos exactly
    c, s = np.cos(511.0), np.sin(511.0)
    assert np.allclose(r[:, 0], vv[:, 0] * c - vv[:, 32] * s, rtol=1e-12)


def test_attention_closed_forms_and_gqa_mapping():
    rng = np.random.default_rng(2)
    H, KVH, hd, L, S = 14, 2, 64, 37, 48
    q = rng.standard_normal(H * hd)
    k = rng.standard_normal((KVH, S, hd)).astype(np.float32)
    v = rng.standard_normal((KVH, S, hd)).astype(np.float32)
    out = ora.attention(q, k, v, H, KVH, hd, L, S).reshape(H, hd)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    for h in range(H):
        kvh = h // (H // KVH)
        s = (k[kvh, :L].astype(np.float64) @ q[h * hd:(h + 1) * hd]) * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(out[h], p @ v[kvh, :L].astype(np.float64), rtol=1e-12, atol=1e-12)
    # one position: the output is that value row
    o1 = ora.attention(q, k, v, H, KVH, hd, 1, S).reshape(H, hd)
    assert np.allclose(o1[0], v[0, 0]) and np.allclose(o1[H - 1], v[1, 0])
    # equal keys: uniform weights → mean of the values
    k2 = np.repeat(k[:, :1], S, axis=1)
    o2 = ora.attention(q, k2, v, H, KVH, hd, L, S).reshape(H, hd)
    assert np.allclose(o2[0], v[0, :L].astype(np.float64).mean(axis=0), atol=1e-12)
    # kv_len = 0 → zeros (the reference's l = 0 case)
    assert np.all(ora.attention(q, k, v, H, KVH, hd, 0, S) == 0)


# ───────────────────────── Q5_0 / Q5_K ─────────────────────────

def test_q5_0_layout_j_and_j_plus_16_with_high_bits():
    # forward.rs:900-920: element j (j < 16) = low nibble of qs[j] + qh bit j,
    # element j+16 = high nibble + qh bit 16+j.  This is also ggml's published
    # Q5_0 layout (dequantize_row_q5_0), so both readings must agree.
    q = [(7 * e + 3) % 32 for e in range(32)]
    qs = bytes((q[j] & 15) | ((q[j + 16] & 15) << 4) for j in range(16))
    qh = 0
    for e in range(32):
        qh |= (q[e] >> 4) << e
    blk = h16(0.5) + qh.to_bytes(4, "little") + qs
    v = ora.dequant("q5_0", np.frombuffer(blk, np.uint8))
    assert np.array_equal(v, 0.5 * (np.array(q) - 16))
    # a single set high bit (bit 20 → element 20) moves exactly one value by 16·d
    blk0 = h16(1.0) + bytes(4) + bytes(16)
    blk1 = h16(1.0) + (1 << 20).to_bytes(4, "little") + bytes(16)
    v0 = ora.dequant("q5_0", np.frombuffer(blk0, np.uint8))
    v1 = ora.dequant("q5_0", np.frombuffer(blk1, np.uint8))
    assert np.all(v0 == -16)
    assert np.nonzero(v1 - v0)[0].tolist() == [20] and v1[20] == 0.0


def test_q5_0_without_high_bits_is_q4_offset_by_minus_8():
    # with qh = 0 a code c reads c − 16; the same nibbles under the Q4_0 rule
    # (c − 8) differ by exactly 8·d, element order aside (j / j+16 here,
    # 2i / 2i+1 there)
    rng = np.random.default_rng(3)
    qs = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
    v5 = ora.dequant("q5_0", np.frombuffer(h16(0.25) + bytes(4) + qs, np.uint8))
    v4 = ora.dequant("q4_0", np.frombuffer(h16(0.25) + qs, np.uint8))
    lo, hi = v4[0::2], v4[1::2]
    assert np.array_equal(v5[:16], lo - 2.0) and np.array_equal(v5[16:], hi - 2.0)


def _q5k_block(d, dmin, sc, m, q):
    """Q5_K in the reference layout: Q4_K scale packing, qs[32j+l] holds the
    low 4 bits of elements 64j+l (low nibble) and 64j+32+l (high nibble), the
    fifth bit of element e is bit e%8 of qh[e/8]."""
    b4 = bytearray(_q4k_block(d, dmin, sc, m, [c & 15 for c in q]))
    qh = bytearray(32)
    for e in range(256):
        qh[e // 8] |= (q[e] >> 4) << (e % 8)
    return bytes(b4[:16]) + bytes(qh) + bytes(b4[16:])


def test_q5k_high_bit_order_and_scale_pairing():
    sc = [1, 2, 3, 4, 63, 17, 48, 33]
    m = [5, 6, 7, 8, 62, 31, 16, 47]
    q = [((e * 11) + 5) % 32 for e in range(256)]
    d, dmin = 0.0625, 0.03125
    v = ora.dequant("q5k", np.frombuffer(_q5k_block(d, dmin, sc, m, q), np.uint8))
    for e in range(256):
        s = (e // 64) + 4 * ((e // 32) & 1)
        expect = np.float32(np.float32(d * sc[s]) * np.float32(q[e])) - np.float32(dmin * m[s])
        assert v[e] == expect, e
    # one qh bit: bit 3 of qh[9] is element 75 (pair j=1, high half, l=11);
    # ggml's Q5_K order would put that bit on a different element
    blk = bytearray(_q5k_block(1.0, 0.0, [1] * 8, [0] * 8, [0] * 256))
    base = ora.dequant("q5k", np.frombuffer(bytes(blk), np.uint8))
    blk[16 + 9] |= 1 << 3
    v = ora.dequant("q5k", np.frombuffer(bytes(blk), np.uint8))
    assert np.nonzero(v - base)[0].tolist() == [75] and v[75] == 16.0


def test_q5k_without_high_bits_equals_q4k():
    # qh = 0: Q5_K reduces to Q4_K with the same header and qs
    rng = np.random.default_rng(5)
    hdr = bytearray(rng.integers(0, 256, 16, dtype=np.uint8).tobytes())
    hdr[0:4] = h16(0.01) + h16(0.002)
    qs = rng.integers(0, 256, 128, dtype=np.uint8).tobytes()
    v5 = ora.dequant("q5k", np.frombuffer(bytes(hdr) + bytes(32) + qs, np.uint8))
    v4 = ora.dequant("q4k", np.frombuffer(bytes(hdr) + qs, np.uint8))
    assert np.array_equal(v5, v4)


# ───────────────────────── ggml layouts ─────────────────────────
# Known answers written from ggml's block definitions (not from the oracle):
# they pin the element ↔ nibble/bit/scale maps that differ from the
# reference's layouts.

def test_q4_0g_byte_j_holds_elements_j_and_j_plus_16():
    c = [(5 * e + 2) % 16 for e in range(32)]
    qs = bytes(c[j] | (c[j + 16] << 4) for j in range(16))
    v = ora.dequant("q4_0g", np.frombuffer(h16(0.5) + qs, np.uint8))
    assert np.array_equal(v, 0.5 * (np.array(c) - 8))


def _scale_table(sc, m):
    S = [0] * 12
    for j in range(4):
        S[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        S[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        S[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return bytes(S)


@pytest.mark.parametrize("s", range(8))
def test_q4kg_sub_block_s_covers_elements_32s(s):
    # ggml: sub-block s scales elements 32s..32s+31 (chunk s//2, low nibbles
    # for even s, high for odd); the reference layout would light up
    # 64·(s%4) + 32·(s//4) instead
    sc = [0] * 8
    sc[s] = 9
    qs = bytes([0x53] * 128)  # low nibble 3, high nibble 5
    blk = h16(0.25) + h16(0.0) + _scale_table(sc, [0] * 8) + qs
    v = ora.dequant("q4kg", np.frombuffer(blk, np.uint8))
    nz = np.nonzero(v)[0]
    assert nz.min() == 32 * s and nz.max() == 32 * s + 31
    assert np.all(v[nz] == 0.25 * 9 * (5 if s % 2 else 3))


def test_q5kg_fifth_bit_is_bit_2j_plus_half_of_qh_l():
    sc, m = [1] * 8, [0] * 8
    base = h16(1.0) + h16(0.0) + _scale_table(sc, m)
    qh = bytearray(32)
    qh[11] = 1 << 3  # j = 1, high half, l = 11 → element 64 + 32 + 11 = 107
    v0 = ora.dequant("q5kg", np.frombuffer(base + bytes(32) + bytes(128), np.uint8))
    v1 = ora.dequant("q5kg", np.frombuffer(base + bytes(qh) + bytes(128), np.uint8))
    assert np.all(v0 == 0)
    assert np.nonzero(v1)[0].tolist() == [107] and v1[107] == 16.0


def test_q6kg_every_16_elements_have_their_own_scale():
    # only sc[1] non-zero: ggml applies it to l in 16..31 of t = 0, h = 0, i.e.
    # elements 16..31; the reference layout never reads odd slots
    ql, qh = bytes([0x11] * 128), bytes(64)  # codes 1 → q = 1 − 32 = −31
    sc = bytearray(16)
    sc[1] = 3
    v = ora.dequant("q6kg", np.frombuffer(ql + qh + bytes(sc) + h16(2.0), np.uint8))
    nz = np.nonzero(v)[0]
    assert nz.tolist() == list(range(16, 32)) and np.all(v[nz] == 2.0 * 3 * -31)
    vr = ora.dequant("q6k", np.frombuffer(ql + qh + bytes(sc) + h16(2.0), np.uint8))
    assert np.all(vr == 0)


@pytest.mark.parametrize("fmt", ["q4_0", "q4k", "q5k"])
def test_relayout_to_ggml_preserves_values(fmt):
    w = (0.02 * ora.synth_normal(21, 256 * 8)).astype(np.float32)
    r = ora.quantize(fmt, w)
    assert np.array_equal(ora.dequant(fmt, r), ora.dequant(fmt + "g", ora.relayout_to_ggml(fmt, r)))


# ───────────────────────── whole-step CPU baseline ─────────────────────────

def test_decode_step_ref_f32_matches_f64_composition():
    """ora_decode_step_ref_f32 (the timed CPU baseline: the reference's f32
    CPU helpers composed into a decode step) against the same step composed in
    f64 from the oracle's checked pieces: logits within 1e-4 of their spread,
    the same greedy token, the KV cache row at pos written."""
    from types import SimpleNamespace
    cfg = SimpleNamespace(layers=2, hidden=256, heads=8, kv_heads=2, head_dim=32, ff=512,
                          vocab=300, max_seq=40, eps=1e-6, theta=1e6)
    q, kv = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    quant = dict(q="q8_0", k="q8_0", v="q4k", o="q4_0", gate="q4k", up="q4k", down="q6k",
                 lm_head="q6k")
    seed = iter(range(100, 1000))
    cache = cfg.kv_heads * cfg.max_seq * cfg.head_dim

    def w(role, n, k):
        return synth_w(quant[role], n, k, next(seed))

    def synth_w(fmt, n, k, s):
        return ora.synth_weights(fmt, n, k, s)

    layers = []
    for _ in range(cfg.layers):
        layers.append(dict(
            wq=w("q", q, cfg.hidden), wk=w("k", kv, cfg.hidden), wv=w("v", kv, cfg.hidden),
            wo=w("o", cfg.hidden, q), wg=w("gate", cfg.ff, cfg.hidden),
            wu=w("up", cfg.ff, cfg.hidden), wd=w("down", cfg.hidden, cfg.ff),
            bq=ora.synth_normal(next(seed), q, std=0.02).astype(np.float16),
            bk=ora.synth_normal(next(seed), kv, std=0.02).astype(np.float16),
            bv=ora.synth_normal(next(seed), kv, std=0.02).astype(np.float16),
            attn_norm=ora.synth_normal(next(seed), cfg.hidden, mean=1.0, std=0.02),
            ffn_norm=ora.synth_normal(next(seed), cfg.hidden, mean=1.0, std=0.02),
            kc=ora.synth_normal(next(seed), cache), vc=ora.synth_normal(next(seed), cache)))
    embd = synth_w("q8_0", cfg.vocab, cfg.hidden, next(seed))
    lm = synth_w("q6k", cfg.vocab, cfg.hidden, next(seed))
    fnorm = ora.synth_normal(next(seed), cfg.hidden, mean=1.0, std=0.02)
    tok, pos = 17, 30
    # f64 composition (before the f32 step updates the caches)
    row = (cfg.hidden // 32) * 34
    x = ora.dequant("q8_0", embd[tok * row:(tok + 1) * row]).astype(np.float64)
    for L in layers:
        xn = ora.rms_norm(x.astype(np.float32), L["attn_norm"], cfg.eps)
        qv = ora.gemv(quant["q"], L["wq"], xn.astype(np.float32), q, cfg.hidden)[0] + L["bq"]
        kk = ora.gemv(quant["k"], L["wk"], xn.astype(np.float32), kv, cfg.hidden)[0] + L["bk"]
        vv = ora.gemv(quant["v"], L["wv"], xn.astype(np.float32), kv, cfg.hidden)[0] + L["bv"]
        qv = ora.rope(qv, cfg.heads, cfg.head_dim, pos, cfg.theta)
        kk = ora.rope(kk, cfg.kv_heads, cfg.head_dim, pos, cfg.theta)
        kc = L["kc"].reshape(cfg.kv_heads, cfg.max_seq, cfg.head_dim).copy()
        vc = L["vc"].reshape(cfg.kv_heads, cfg.max_seq, cfg.head_dim).copy()
        kc[:, pos] = kk.reshape(cfg.kv_heads, -1)
        vc[:, pos] = vv.reshape(cfg.kv_heads, -1)
        att = ora.attention(qv, kc, vc, cfg.heads, cfg.kv_heads, cfg.head_dim, pos + 1, cfg.max_seq)
        x = x + ora.gemv(quant["o"], L["wo"], att.astype(np.float32), cfg.hidden, q)[0]
        xn = ora.rms_norm(x.astype(np.float32), L["ffn_norm"], cfg.eps).astype(np.float32)
        g = ora.gemv(quant["gate"], L["wg"], xn, cfg.ff, cfg.hidden)[0]
        u = ora.gemv(quant["up"], L["wu"], xn, cfg.ff, cfg.hidden)[0]
        act = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        x = x + ora.gemv(quant["down"], L["wd"], act, cfg.hidden, cfg.ff)[0]
    xn = ora.rms_norm(x.astype(np.float32), fnorm, cfg.eps).astype(np.float32)
    ref = ora.gemv("q6k", lm, xn, cfg.vocab, cfg.hidden)[0]
    m = ora.HostStepModel(cfg, layers, fnorm, embd, lm, quant, quant["lm_head"])
    for threads in (1, 3):
        got_tok, logits = m.step(tok, pos, threads)
        assert np.max(np.abs(logits - ref)) <= 1e-4 * (ref.max() - ref.min())
        assert got_tok == int(np.argmax(ref)) == ora.argmax(logits)
    kc0 = layers[0]["kc"].reshape(cfg.kv_heads, cfg.max_seq, cfg.head_dim)
    assert np.any(kc0[:, pos] != 0) and kc0.shape[1] == cfg.max_seq


# ───────────────────────── verify_draft glue ─────────────────────────

def test_rope_batch_rows_are_single_position_ropes():
    """Row s of the batched rotation is the single-token rotation at
    start_pos + s (the angle formed by division instead of multiplication by
    the inverse: equal to f32 rounding), and position 0 is the identity."""
    rng = np.random.default_rng(2)
    seq, heads, hd, start = 5, 3, 64, 507
    v = rng.standard_normal(seq * heads * hd)
    r = ora.rope_batch(v, seq, heads, hd, start, 1e6).reshape(seq, heads * hd)
    for s in range(seq):
        one = ora.rope(v.reshape(seq, -1)[s], heads, hd, start + s, 1e6)
        assert np.allclose(r[s], one, rtol=0, atol=1e-3 * np.abs(one).max()), s
    assert np.array_equal(ora.rope_batch(v[:heads * hd], 1, heads, hd, 0, 1e6), v[:heads * hd])
    # pair 0 has frequency 1: angle = position exactly
    rr = r.reshape(seq, heads, hd)
    vv = v.reshape(seq, heads, hd)
    for s in range(seq):
        c, sn = np.cos(float(start + s)), np.sin(float(start + s))
        assert np.allclose(rr[s, :, 0], vv[s, :, 0] * c - vv[s, :, 32] * sn, rtol=1e-12)


def test_argmax_rows_first_semantics():
    """forward.rs:2283-2293: strictly-greater scan from −inf — the first
    maximal index, NaN never wins, a row with nothing above −inf gives 0."""
    nan, inf = np.float32("nan"), np.float32("inf")
    cases = [
        ([1.0, 3.0, 3.0, 2.0], 1),   # ties → first maximal index
        ([3.0, 1.0, 3.0], 0),
        ([-inf, -inf], 0),
        ([nan, 2.0, 7.0, 7.0], 2),
        ([1.0, nan, 0.5], 0),
        ([nan, nan], 0),
        ([-inf, -5.0], 1),
        ([inf, inf], 0),
    ]
    for vals, expect in cases:
        assert ora.argmax_rows_first(np.array(vals, np.float32), 1)[0] == expect, vals
    # NaN-free rows: numpy's argmax also returns the first maximal index
    rng = np.random.default_rng(3)
    m = rng.integers(-4, 5, size=(7, 300)).astype(np.float32)
    assert np.array_equal(ora.argmax_rows_first(m, 7), np.argmax(m, axis=1))


def test_causal_attention_rows_are_prefix_decode_attention():
    """Row r of the causal oracle is the decode attention over the first
    q_start + r + 1 positions; a row that sees one position returns its value
    row exactly."""
    rng = np.random.default_rng(4)
    H, KVH, hd, S, M, kv_len = 4, 2, 64, 40, 3, 20
    q = rng.standard_normal(M * H * hd)
    k = rng.standard_normal(KVH * S * hd).astype(np.float32)
    v = rng.standard_normal(KVH * S * hd).astype(np.float32)
    out = ora.causal_attention(q, k, v, M, H, KVH, hd, kv_len, S, 0)
    vv = v.reshape(KVH, S, hd)
    for h in range(H):
        assert np.allclose(out[0, h * hd:(h + 1) * hd], vv[h // 2, 0], rtol=1e-12)
    full = ora.causal_attention(q, k, v, M, H, KVH, hd, kv_len, S, kv_len - M)
    for r in range(M):
        ref = ora.attention(q.reshape(M, -1)[r], k, v, H, KVH, hd, kv_len - M + r + 1, S)
        assert np.array_equal(full[r], ref)
