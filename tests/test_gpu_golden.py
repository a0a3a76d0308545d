"""The HIP path (through the C ABI) against the committed golden fixtures:
bf16 outputs within max-abs 2e-2, f32 state within relative L2 1e-3 (on the
fixture's subsample and its checksums), conv state and slot moves bit-exact."""
import os

import numpy as np
import pytest

from gdn_testlib import DK, DV, K, dev, host, rel_l2, say, O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
Y_TOL = 2e-2
STATE_TOL = 1e-3


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def regen_state(seed, shape):
    return (np.random.default_rng(int(seed)).standard_normal(shape) * 0.01).astype(np.float32)


def _ids(lst):
    return dev(np.asarray(lst, np.int32))


def _check_state(st, f):
    sample = st.ravel()[f["state_out_index"]]
    rs = rel_l2(sample, f["state_out_sample"])
    assert rs <= STATE_TOL
    assert abs((np.asarray(st, np.float64) ** 2).sum() - f["state_out_checksum"][1]) <= \
        STATE_TOL * f["state_out_checksum"][1]
    return rs


def test_config0_decode_golden(gpu):
    import torch
    import gdn_amd
    f = load("config0_decode.npz")
    Hk, Hv = int(f["Hk"]), int(f["Hv"])
    D = f["mixed_qkv"].shape[1]
    say("golden config0 decode", f"Hk={Hk} Hv={Hv}")
    state = regen_state(f["state_seed"], (1, Hv, DV, DK))
    pool = gdn_amd.Pool(1, 3, Hk, Hv)
    pool.write(0, _ids([1]), dev(state), dev(np.ascontiguousarray(f["conv_state_cm"].T)[None]))
    y = torch.zeros((1, Hv, DV), dtype=torch.int16, device=gpu)
    pool.decode(0, _ids([1]), dev(f["mixed_qkv"]), dev(f["ab"]), dev(f["A_log"]),
                dev(f["dt_bias"]), dev(f["conv_w"]), y)
    gs = torch.empty((1, Hv, DV, DK), dtype=torch.float32, device=gpu)
    gc = torch.empty((1, K - 1, D), dtype=torch.int16, device=gpu)
    pool.read(0, _ids([1]), gs, gc)
    assert np.array_equal(host(gc)[0], f["conv_state_out"])
    dy = float(np.max(np.abs(O.bf16_to_f32(host(y)) - O.bf16_to_f32(f["y"]))))
    rs = _check_state(host(gs), f)
    say("golden config0 decode |dy|", dy, "state sample relL2", rs)
    assert dy <= Y_TOL
    assert pool.check() == 0


def test_config0_recurrent_golden(gpu):
    import torch
    import gdn_amd
    f = load("config0_recurrent.npz")
    Hk, Hv = int(f["Hk"]), int(f["Hv"])
    say("golden config0 recurrent", f"Hk={Hk} Hv={Hv}")
    state = regen_state(f["state_seed"], (1, Hv, DV, DK))
    pool = gdn_amd.Pool(1, 2, Hk, Hv)
    pool.write(0, _ids([0]), dev(state), None)
    y = torch.zeros((1, 1, Hv, DV), dtype=torch.int16, device=gpu)
    pool.recurrent(0, _ids([0]), dev(f["q"]), dev(f["k"]), dev(f["v"]), dev(f["g"]),
                   dev(f["beta"]), y)
    gs = torch.empty((1, Hv, DV, DK), dtype=torch.float32, device=gpu)
    pool.read(0, _ids([0]), gs, None)
    dy = float(np.max(np.abs(O.bf16_to_f32(host(y)) - O.bf16_to_f32(f["y"]))))
    rs = _check_state(host(gs), f)
    say("golden config0 recurrent |dy|", dy, "state sample relL2", rs)
    assert dy <= Y_TOL
    assert pool.check() == 0


def test_tiny_prefill_golden(gpu):
    import torch
    import gdn_amd
    f = load("tiny_prefill.npz")
    Hk, Hv = int(f["Hk"]), int(f["Hv"])
    cu = f["cu_seqlens"]
    n = len(cu) - 1
    total = int(cu[-1])
    D = f["mixed_qkv"].shape[1]
    say("golden tiny prefill", f"Hk={Hk} Hv={Hv} cu={cu.tolist()}")
    state = regen_state(f["state_seed"], (n, Hv, DV, DK))
    pool = gdn_amd.Pool(1, 4, Hk, Hv)
    slots = [3, 1]
    pool.write(0, _ids(slots), dev(state), dev(f["conv_state_in"]))
    y = torch.zeros((total, Hv, DV), dtype=torch.int16, device=gpu)
    pool.prefill(0, _ids(slots), dev(cu), total, dev(f["mixed_qkv"]), dev(f["ab"]),
                 dev(f["A_log"]), dev(f["dt_bias"]), dev(f["conv_w"]), y)
    gs = torch.empty((n, Hv, DV, DK), dtype=torch.float32, device=gpu)
    gc = torch.empty((n, K - 1, D), dtype=torch.int16, device=gpu)
    pool.read(0, _ids(slots), gs, gc)
    assert np.array_equal(host(gc), f["conv_state_out"])
    dy = float(np.max(np.abs(O.bf16_to_f32(host(y)) - O.bf16_to_f32(f["y"]))))
    rs = _check_state(host(gs), f)
    say("golden tiny prefill |dy|", dy, "state sample relL2", rs)
    assert dy <= Y_TOL
    assert pool.check() == 0


def test_tiny_slots_golden(gpu):
    import torch
    import gdn_amd
    f = load("tiny_slots.npz")
    ps, pc, ids = f["pool_state"], f["pool_conv"], f["slot_ids"]
    S, Hv, Dv, Dk = ps.shape
    say("golden slots", f"S={S} ids={ids.tolist()}")
    # the pool's head dims are fixed at 128: embed the fixture's 4x4 tiles and
    # 32-channel conv rows, and compare the gathered embeddings
    Hk = 1
    pool = gdn_amd.Pool(1, S, Hk, Hv)
    D = pool.D
    big_s = np.zeros((S, Hv, DV, DK), np.float32)
    big_s[:, :, :Dv, :Dk] = ps
    big_c = np.zeros((S, K - 1, D), np.uint16)
    big_c[:, :, :pc.shape[2]] = pc
    pool.write(0, _ids(list(range(S))), dev(big_s), dev(big_c))
    gs = torch.empty((len(ids), Hv, DV, DK), dtype=torch.float32, device=gpu)
    gc = torch.empty((len(ids), K - 1, D), dtype=torch.int16, device=gpu)
    pool.read(0, _ids(ids), gs, gc)
    assert np.array_equal(host(gs)[:, :, :Dv, :Dk], f["stacked_state"])
    assert np.array_equal(host(gc)[:, :, :pc.shape[2]], f["stacked_conv"])
    assert pool.check() == 0
