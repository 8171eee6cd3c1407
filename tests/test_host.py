"""Host-side logic that needs no GPU: the bench's one-GPU contract and the
decode step's per-role weight accounting and format checks."""
import os
import subprocess
import sys

import numpy as np
import pytest

from runit_mac_amd import dispatch as d
from runit_mac_amd.decode import Q4K_M, Q8_ALL, ROLES, DecodeConfig, DecodeModel

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    p = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode != 0
    assert "one GPU" in p.stderr


def test_q4k_m_weight_accounting():
    c = DecodeConfig(layers=28, hidden=3584, heads=28, kv_heads=4, head_dim=128, ff=18944,
                     vocab=152064)
    h, q, kv, ff = c.hidden, c.q_dim, c.kv_dim, c.ff
    per_layer = (d.weight_bytes("q4k", q, h) + d.weight_bytes("q4k", kv, h)
                 + d.weight_bytes("q6k", kv, h) + d.weight_bytes("q4k", h, q)
                 + 2 * d.weight_bytes("q4k", ff, h) + d.weight_bytes("q6k", h, ff))
    assert c.weight_bytes(Q4K_M) == 28 * per_layer + d.weight_bytes("q6k", c.vocab, h)
    assert c.weight_bytes() == c.weight_bytes(Q8_ALL)
    # KV reads grow with the cache length; the weights do not
    assert c.step_bytes(1024, Q4K_M) - c.step_bytes(512, Q4K_M) == \
        28 * 2 * c.kv_heads * 512 * c.head_dim * 4
    assert set(Q4K_M) == set(ROLES)


def test_decode_model_rejects_unknown_roles_before_allocating():
    with pytest.raises(ValueError):
        DecodeModel(None, DecodeConfig(layers=1), quant={"attn": "q4k"})


def test_accept_drafts_follows_verify_draft():
    """forward.rs:2279-2305: accept while row r's argmax equals draft r."""
    from runit_mac_amd.decode import accept_drafts
    assert accept_drafts([5], []) == (0, 5)
    assert accept_drafts([1, 2, 3, 9], [1, 2, 3]) == (3, 9)
    assert accept_drafts([1, 7, 3, 9], [1, 2, 3]) == (1, 7)
    assert accept_drafts([4, 2, 3, 9], [1, 2, 3]) == (0, 4)
    with pytest.raises(ValueError):
        accept_drafts([1, 2], [1, 2])


def test_device_pointer_arguments_reject_non_integers():
    """A bool (or any non-integer) passed where a device pointer is expected
    is an error on the host, not address 1 on the device."""
    from runit_mac_amd.dispatch import _ptr
    assert _ptr(None) is None and _ptr(4096) == 4096 and _ptr(np.uint64(64)) == 64
    for bad in (True, False, 1.0, "0x10"):
        with pytest.raises(TypeError):
            _ptr(bad)


@pytest.mark.parametrize("ids", [[1, 2, 1000], [5, -1], [1000]])
def test_verify_and_prefill_reject_ids_outside_the_vocabulary(ids):
    """The embedding kernel indexes the table with each id unchecked, so ids
    outside [0, vocab) are refused on the host, before any upload or launch
    (the model has no context here: a launch would fail differently)."""
    m = DecodeModel.__new__(DecodeModel)
    m.ctx, m.cfg, m.lm_fmt = None, DecodeConfig(layers=1, vocab=1000, max_seq=64), "q8_0"
    with pytest.raises(ValueError, match="out of range"):
        m.verify_forward(ids, 0)
    with pytest.raises(ValueError, match="out of range"):
        m.prefill(ids)
    with pytest.raises(ValueError, match="out of range"):
        m.verify_draft(ids[0], ids[1:], 0)
