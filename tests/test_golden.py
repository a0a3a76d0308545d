"""The oracle against the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py from the oracle itself). A change to the oracle's
arithmetic, its input generators or the seeded state regeneration shows up
here as a mismatch; the fixtures are compared bit for bit."""
import os

import numpy as np
import pytest

from gdn_testlib import O, DK, DV, K

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def regen_state(seed, shape):
    return (np.random.default_rng(int(seed)).standard_normal(shape) * 0.01).astype(np.float32)


def checksum(a):
    x = np.asarray(a, np.float64).ravel()
    return np.array([x.sum(), (x * x).sum(), np.abs(x).sum()])


def test_config0_decode_fixture():
    f = load("config0_decode.npz")
    Hk, Hv = int(f["Hk"]), int(f["Hv"])
    assert str(f["conv_state_layout"]) == "channel-major [D, K-1]"
    state = regen_state(f["state_seed"], (1, Hv, DV, DK))
    assert np.array_equal(checksum(state), f["state_checksum"])
    conv = np.ascontiguousarray(f["conv_state_cm"].T)[None]
    y, conv_out, st_out = O.decode(conv, state, f["mixed_qkv"], f["ab"], f["A_log"], f["dt_bias"],
                                   f["conv_w"], Hk, Hv)
    assert np.array_equal(y, f["y"])
    assert np.array_equal(conv_out[0], f["conv_state_out"])
    assert np.array_equal(st_out.ravel()[f["state_out_index"]], f["state_out_sample"])
    assert np.array_equal(checksum(st_out), f["state_out_checksum"])


def test_config0_recurrent_fixture():
    f = load("config0_recurrent.npz")
    Hv = int(f["Hv"])
    state = regen_state(f["state_seed"], (1, Hv, DV, DK))
    assert np.array_equal(checksum(state), f["state_checksum"])
    y, st_out = O.recurrent(f["q"], f["k"], f["v"], f["g"], f["beta"], state)
    assert np.array_equal(y, f["y"])
    assert np.array_equal(st_out.ravel()[f["state_out_index"]], f["state_out_sample"])
    assert np.array_equal(checksum(st_out), f["state_out_checksum"])


def test_tiny_prefill_fixture():
    f = load("tiny_prefill.npz")
    Hk, Hv = int(f["Hk"]), int(f["Hv"])
    cu = f["cu_seqlens"]
    n = len(cu) - 1
    state = regen_state(f["state_seed"], (n, Hv, DV, DK))
    assert np.array_equal(checksum(state), f["state_checksum"])
    ys, convs, sts = [], [], []
    for i in range(n):
        a, b = cu[i], cu[i + 1]
        y, c, s = O.prefill(f["conv_state_in"][i], state[i], f["mixed_qkv"][a:b], f["ab"][a:b],
                            f["A_log"], f["dt_bias"], f["conv_w"], Hk, Hv)
        ys.append(y)
        convs.append(c)
        sts.append(s)
    st_out = np.stack(sts)
    assert np.array_equal(np.concatenate(ys), f["y"])
    assert np.array_equal(np.stack(convs), f["conv_state_out"])
    assert np.array_equal(st_out.ravel()[f["state_out_index"]], f["state_out_sample"])
    assert np.array_equal(checksum(st_out), f["state_out_checksum"])


def test_tiny_slots_fixture():
    f = load("tiny_slots.npz")
    ids = f["slot_ids"]
    assert np.array_equal(O.stack(f["pool_state"], ids), f["stacked_state"])
    assert np.array_equal(O.stack(f["pool_conv"], ids), f["stacked_conv"])
    # scatter back into a cleared pool restores exactly the gathered slots
    ps = np.zeros_like(f["pool_state"])
    O.unstack(ps, ids, f["stacked_state"])
    assert np.array_equal(ps[ids], f["pool_state"][ids])
    others = np.setdiff1d(np.arange(ps.shape[0]), ids)
    assert not ps[others].any()
