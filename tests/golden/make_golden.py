"""Writes the golden fixtures of the quantized-GEMV path (tests/golden/*.npz).

The reference's own tests hold no vectors for this path (its only nearby
known answers are the f16 GEMV cases of crates/engine/src/bin/test_gemv.rs:
10-85), so the fixtures are built here:

* closed_forms.npz — inputs whose outputs follow from the mathematics alone,
  written by this script without the oracle: the test_gemv.rs known answers
  re-expressed in every block format (all-ones W · [1..K] = K(K+1)/2 per row,
  identity-like W · x = x), and single-block dequant cases whose values are
  stated element by element;
* gemv_<fmt>.npz — seeded small-shape GEMVs (W packed, x, y_ref in f64,
  Σ|w·x| per row, the dequantised W), produced by the CPU oracle (oracle/).
  The oracle itself is pinned by tests/test_oracle.py; these files freeze its
  outputs so that a later change to it, or to the device path, shows up as a
  fixture mismatch;
* fused.npz — fused QKV+bias and gate/up/SiLU FFN cases, argmax vectors with
  ties and NaNs (sampler.rs:111-116 semantics).

Run:  python tests/golden/make_golden.py     (needs oracle/liboracle.so)
All files load with numpy.load(allow_pickle=False).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as ora  # noqa: E402

BLOCK = {"q8_0": (32, 34), "q4_0": (32, 18), "q4k": (256, 144), "q6k": (256, 210)}
SHAPES = {"q8_0": [(16, 96), (12, 64)], "q4_0": [(12, 64), (8, 96)],
          "q4k": [(8, 512), (4, 256)], "q6k": [(8, 512), (4, 256)]}


def f16_bytes(v: float) -> bytes:
    return np.float16(v).tobytes()


# ───────────────────────── closed forms (no oracle) ─────────────────────────

def q8_0_block(d: float, q) -> bytes:
    return f16_bytes(d) + np.asarray(q, np.int8).tobytes()


def q4_0_block(d: float, nib) -> bytes:
    """Reference nibble order: element 2i low nibble, 2i+1 high nibble
    (gemv_q4_0.metal:13-14, forward.rs:974-976)."""
    nib = np.asarray(nib, np.uint8)
    return f16_bytes(d) + (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8).tobytes()


def q4k_block(d: float, dmin: float, sc, mn, nib) -> bytes:
    """sc/mn: 8 six-bit values; packing of get_scale_min_k4 (forward.rs:359-369):
    j < 4: scales[j] & 63, scales[j+4] & 63; j ≥ 4: low nibbles from
    scales[j+4], high bits from the top two bits of scales[j-4] / scales[j]."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    # qs: pair j (0..3) holds elements 64j+l (low nibble) and 64j+32+l (high)
    nib = np.asarray(nib, np.uint8).reshape(4, 2, 32)
    qs = (nib[:, 0, :] | (nib[:, 1, :] << 4)).astype(np.uint8).ravel()
    return f16_bytes(d) + f16_bytes(dmin) + s.tobytes() + qs.tobytes()


def closed_forms():
    out = {}
    # test_gemv.rs:10-85 known answers in block formats.  All-ones rows
    # (d = 1, q = 1) against x = [1..K]: every output is K(K+1)/2.
    k = 64
    x = np.arange(1, k + 1, dtype=np.float32)
    out["ones_x"] = x
    out["ones_y"] = np.full(4, k * (k + 1) / 2)
    out["ones_q8_0"] = np.frombuffer(b"".join(q8_0_block(1.0, [1] * 32) for _ in range(4 * k // 32)),
                                     np.uint8)
    # Q4_0: nibble 9 is value (9 - 8) = 1
    out["ones_q4_0"] = np.frombuffer(b"".join(q4_0_block(1.0, [9] * 32) for _ in range(4 * k // 32)),
                                     np.uint8)
    # identity-like Q8_0: row r has q = 1 at column r, 0 elsewhere → y = x[:4]
    rows = []
    for r in range(4):
        q = np.zeros(k, np.int8)
        q[r] = 1
        rows.append(b"".join(q8_0_block(1.0, q[32 * b:32 * b + 32]) for b in range(k // 32)))
    out["eye_q8_0"] = np.frombuffer(b"".join(rows), np.uint8)
    out["eye_y"] = x[:4].astype(np.float64)
    # Q8_0 dequant: d = 1, q = i − 16 → v = i − 16 (exact)
    out["deq_q8_0_in"] = np.frombuffer(q8_0_block(1.0, np.arange(32) - 16), np.uint8)
    out["deq_q8_0_out"] = (np.arange(32) - 16).astype(np.float32)
    # Q8_0 with d = 0.5: v = 0.5·q
    out["deq_q8_0h_in"] = np.frombuffer(q8_0_block(0.5, np.arange(32) - 16), np.uint8)
    out["deq_q8_0h_out"] = (0.5 * (np.arange(32) - 16)).astype(np.float32)
    # Q4_0: d = 2, nibble i % 16 at element i → v = 2·((i % 16) − 8)
    nib = np.arange(32) % 16
    out["deq_q4_0_in"] = np.frombuffer(q4_0_block(2.0, nib), np.uint8)
    out["deq_q4_0_out"] = (2.0 * (nib - 8)).astype(np.float32)
    # Q4_K: only scale j+4 = 5 (pair j = 1, high half) non-zero, dmin = 0 →
    # elements 64·1+32 .. 64·1+63 are 5·nibble, all others 0 (scale pairing
    # (j, j+4) of dequant.metal:77-95)
    sc = [0, 0, 0, 0, 0, 5, 0, 0]
    mn = [0] * 8
    nib4 = np.arange(256) % 16
    out["deq_q4k_in"] = np.frombuffer(q4k_block(1.0, 0.0, sc, mn, nib4), np.uint8)
    v = np.zeros(256, np.float32)
    v[96:128] = 5.0 * nib4[96:128]
    out["deq_q4k_out"] = v
    # Q4_K all-zero nibbles, dmin = 1, mins m_j = j + 1 → v = −(j+1) on sub-block j
    # (qwen2_load_test.rs:105-134: zero quants dequantise to −dmin·m)
    mn2 = [1, 2, 3, 4, 5, 6, 7, 8]
    out["deq_q4kz_in"] = np.frombuffer(q4k_block(1.0, 1.0, [1] * 8, mn2, np.zeros(256, int)),
                                       np.uint8)
    vz = np.zeros(256, np.float32)
    for j in range(4):
        vz[64 * j:64 * j + 32] = -mn2[j]
        vz[64 * j + 32:64 * j + 64] = -mn2[j + 4]
    out["deq_q4kz_out"] = vz
    return out


# ───────────────────────── oracle-generated cases ─────────────────────────

def gemv_cases(fmt):
    out = {}
    for i, (n, k) in enumerate(SHAPES[fmt]):
        w = ora.synth_weights(fmt, n, k, seed=1000 + 17 * i + len(fmt))
        x = ora.synth_normal(2000 + i, k)
        y, s = ora.gemv(fmt, w, x, n, k)
        out[f"w{i}"] = w
        out[f"x{i}"] = x
        out[f"y{i}"] = y
        out[f"sabs{i}"] = s
        out[f"deq{i}"] = ora.dequant(fmt, w)
        out[f"shape{i}"] = np.array([n, k], np.int64)
    return out


def fused_cases():
    out = {}
    # fused QKV + bias (Q8_0), q_dim 64, kv_dim 32, k 96
    qd, kd, k = 64, 32, 96
    for name, n, seed in (("q", qd, 11), ("k", kd, 12), ("v", kd, 13)):
        w = ora.synth_weights("q8_0", n, k, seed)
        b = (0.02 * ora.synth_normal(seed + 100, n)).astype(np.float16)
        out[f"qkv_w{name}"] = w
        out[f"qkv_b{name}"] = b.view(np.uint16)
    out["qkv_x"] = ora.synth_normal(14, k)
    for name, n in (("q", qd), ("k", kd), ("v", kd)):
        y, s = ora.gemv("q8_0", out[f"qkv_w{name}"], out["qkv_x"], n, k)
        out[f"qkv_y{name}"] = y + out[f"qkv_b{name}"].view(np.float16).astype(np.float64)
        out[f"qkv_s{name}"] = s
    out["qkv_shape"] = np.array([qd, kd, k], np.int64)
    # fused gate/up/SiLU (Q8_0 and Q4_0), ff 48, k 64
    ff, k = 48, 64
    for fmt in ("q8_0", "q4_0"):
        wg = ora.synth_weights(fmt, ff, k, 21)
        wu = ora.synth_weights(fmt, ff, k, 22)
        x = ora.synth_normal(23, k)
        g, gs = ora.gemv(fmt, wg, x, ff, k)
        u, us = ora.gemv(fmt, wu, x, ff, k)
        out[f"ffn_{fmt}_wg"], out[f"ffn_{fmt}_wu"], out[f"ffn_{fmt}_x"] = wg, wu, x
        out[f"ffn_{fmt}_g"], out[f"ffn_{fmt}_u"] = g, u
        out[f"ffn_{fmt}_gs"], out[f"ffn_{fmt}_us"] = gs, us
        out[f"ffn_{fmt}_act"] = np.array([ora.silu(a) * b for a, b in zip(g, u)])
    out["ffn_shape"] = np.array([ff, k], np.int64)
    # argmax (sampler.rs:111-116): last maximal index; NaN compares Equal
    vecs = [np.array([1, 3, 3, 2], np.float32),
            np.array([np.nan, 1, 5, 5, 0], np.float32),
            np.array([2, np.nan, 2], np.float32),
            np.array([-np.inf, -np.inf], np.float32),
            ora.synth_normal(31, 3000)]
    for i, v in enumerate(vecs):
        out[f"argmax_v{i}"] = v
        out[f"argmax_r{i}"] = np.array(ora.argmax(v), np.int64)
    return out


def main():
    np.savez(os.path.join(HERE, "closed_forms.npz"), **closed_forms())
    for fmt in BLOCK:
        np.savez(os.path.join(HERE, f"gemv_{fmt}.npz"), **gemv_cases(fmt))
    np.savez(os.path.join(HERE, "fused.npz"), **fused_cases())


if __name__ == "__main__":
    main()
