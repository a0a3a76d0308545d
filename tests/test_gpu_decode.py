"""GPU parity of the decode path and the slot pool against the CPU oracle.

Tolerances: bf16 outputs max-abs <= 2e-2, f32 state relative L2 <= 1e-3 after
chained steps; slot movement and untouched slots bit-exact. The f32 kernels
differ from the oracle only in summation order and in forming the readout as
(g s).q + d (k.q), so the measured errors are far inside these bounds; the
tests also assert the tighter figures actually seen (one bf16 ulp on y).
"""
import numpy as np
import pytest

from gdn_testlib import (O, DK, DV, K, conv_dim, dev, gen_layer_params, gen_recurrent_inputs,
                         gen_states, gen_tokens, host, rel_l2, say)

pytestmark = pytest.mark.gpu

Y_TOL = 2e-2
STATE_TOL = 1e-3


def _pool(L, S, Hk=16, Hv=32):
    import gdn_amd
    return gdn_amd.Pool(L, S, Hk, Hv)


def _ids(lst):
    return dev(np.asarray(lst, np.int32))


def test_library_reports_gfx950(gpu):
    import gdn_amd
    assert b"gfx950" in gdn_amd.load().gdn_version()


def test_slot_write_read_zero_bit_exact(gpu):
    import torch
    say("slot ops", "L=2 S=12 Hk=16 Hv=32")
    rng = np.random.default_rng(100)
    pool = _pool(2, 12)
    st, cs = gen_states(rng, 12, 16, 32, state_std=1.0)
    ids_all = _ids(np.arange(12))
    for l in range(2):
        pool.write(l, ids_all, dev(st), dev(cs))
    sel = [9, 2, 5]
    st_new, cs_new = gen_states(rng, 3, 16, 32, state_std=1.0)
    pool.write(1, _ids(sel), dev(st_new), dev(cs_new))
    pool.zero(1, _ids([2]))
    out_s = torch.empty((12, 32, DV, DK), dtype=torch.float32, device=gpu)
    out_c = torch.empty((12, K - 1, conv_dim(16, 32)), dtype=torch.int16, device=gpu)
    pool.read(1, ids_all, out_s, out_c)
    exp_s, exp_c = st.copy(), cs.copy()
    exp_s[sel], exp_c[sel] = st_new, cs_new
    exp_s[2], exp_c[2] = 0.0, 0
    assert np.array_equal(host(out_s), exp_s)
    assert np.array_equal(host(out_c), exp_c)
    pool.read(0, ids_all, out_s, out_c)          # the other layer is untouched
    assert np.array_equal(host(out_s), st) and np.array_equal(host(out_c), cs)
    # gather in a scattered order = numpy fancy indexing
    order = [7, 0, 11, 2]
    g_s = torch.empty((4, 32, DV, DK), dtype=torch.float32, device=gpu)
    pool.read(1, _ids(order), g_s, None)
    assert np.array_equal(host(g_s), exp_s[order])
    # zero across all layers
    pool.zero(-1, _ids([0, 11]))
    for l in range(2):
        pool.read(l, _ids([0, 11]), g_s[:2], None)
        assert not host(g_s[:2]).any()
    assert pool.check() == 0


def test_slot_validation_and_bad_slot_flags(gpu):
    import gdn_amd
    say("slot validation", "S=8")
    pool = _pool(1, 8)
    pool.validate(_ids([1, 2, 3]))
    assert pool.check() == 0
    pool.validate(_ids([1, 2, 1]))
    assert pool.check() == gdn_amd.GDN_FLAG_DUP_SLOT
    pool.validate(_ids([1, 8]))
    assert pool.check() == gdn_amd.GDN_FLAG_BAD_SLOT
    # a long list over a larger pool (LDS bitmap path): a permutation passes,
    # one repeated id anywhere is caught
    big = _pool(1, 5000, 2, 4)
    perm = np.random.default_rng(77).permutation(5000)[:3000].astype(np.int32)
    big.validate(_ids(perm))
    assert big.check() == 0
    dup = perm.copy()
    dup[2999] = dup[17]
    big.validate(_ids(dup))
    assert big.check() == gdn_amd.GDN_FLAG_DUP_SLOT
    # a decode launch with an out-of-range slot skips that sequence, flags it,
    # and still updates the valid one
    rng = np.random.default_rng(101)
    p = gen_layer_params(rng, 16, 32)
    x, ab = gen_tokens(rng, 2, 16, 32)
    y = dev(np.zeros((2, 32, DV), np.uint16))
    before = y.clone()
    pool.decode(0, _ids([3, 99]), dev(x), dev(ab), dev(p["A_log"]), dev(p["dt_bias"]),
                dev(p["conv_w"]), y)
    assert pool.check() == gdn_amd.GDN_FLAG_BAD_SLOT
    assert (host(y[1]) == host(before[1])).all()
    assert host(y[0]).any()
    with pytest.raises(gdn_amd.GdnError):
        pool.decode(5, _ids([3]), dev(x[:1]), dev(ab[:1]), dev(p["A_log"]), dev(p["dt_bias"]),
                    dev(p["conv_w"]), y)


def test_pool_allocator(gpu):
    import gdn_amd
    pool = _pool(1, 4)
    got = [pool.alloc_slot() for _ in range(4)]
    assert got == [0, 1, 2, 3] and pool.slots_in_use() == 4
    with pytest.raises(gdn_amd.GdnError):
        pool.alloc_slot()
    pool.free_slot(2)
    pool.free_slot(0)
    assert pool.alloc_slot() == 0 and pool.slots_in_use() == 3
    with pytest.raises(gdn_amd.GdnError):
        pool.free_slot(2)


@pytest.mark.parametrize("B,T", [(1, 1), (3, 1), (2, 17)])
def test_recurrent_matches_oracle(gpu, B, T):
    """gdn_recurrent vs the restated gated_delta_kernel, config-0 shapes."""
    import torch
    say("gdn_recurrent", f"B={B} T={T} Hk=16 Hv=32 seed={200 + B + T}")
    rng = np.random.default_rng(200 + B + T)
    inp = gen_recurrent_inputs(rng, B, T, 16, 32)
    S = 2 * B + 3
    pool = _pool(1, S)
    slots = rng.choice(S, B, replace=False).astype(np.int32)
    pool.write(0, _ids(slots), dev(inp["state"]), None)
    y = torch.zeros((B, T, 32, DV), dtype=torch.int16, device=gpu)
    pool.recurrent(0, _ids(slots), dev(inp["q"]), dev(inp["k"]), dev(inp["v"]), dev(inp["g"]),
                   dev(inp["beta"]), y)
    got_s = torch.empty((B, 32, DV, DK), dtype=torch.float32, device=gpu)
    pool.read(0, _ids(slots), got_s, None)
    yr, sr = O.recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"])
    yo = O.bf16_to_f32(yr)
    dy = np.abs(O.bf16_to_f32(host(y)) - yo)
    say("gdn_recurrent worst |dy|", float(dy.max()), "of max |y|", float(np.abs(yo).max()))
    assert dy.max() <= Y_TOL
    # one bf16 ulp of the value, plus an f32 summation-order floor for y near 0
    assert np.all(dy <= 2.0 ** -7 * np.abs(yo) + 1e-5 * np.abs(yo).max())
    assert rel_l2(host(got_s), sr) < 1e-5
    assert pool.check() == 0


def test_decode_fused_matches_oracle_config0(gpu):
    """One fused decode step, single layer, B=1 (conv state drawn [8192,3]
    channel-major and transposed into the pool's [3,8192] rows)."""
    import torch
    say("gdn_decode", "config0 B=1 Hk=16 Hv=32 seed=300")
    rng = np.random.default_rng(300)
    Hk, Hv = 16, 32
    D = conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    state = (rng.standard_normal((1, Hv, DV, DK)) * 0.01).astype(np.float32)
    conv_cm = O.f32_to_bf16(rng.standard_normal((D, K - 1)).astype(np.float32))  # [8192,3]
    conv = np.ascontiguousarray(conv_cm.T)[None]                                  # [1,3,8192]
    x, ab = gen_tokens(rng, 1, Hk, Hv)
    pool = _pool(1, 4)
    pool.write(0, _ids([2]), dev(state), dev(conv))
    y = torch.zeros((1, Hv, DV), dtype=torch.int16, device=gpu)
    pool.decode(0, _ids([2]), dev(x), dev(ab), dev(p["A_log"]), dev(p["dt_bias"]),
                dev(p["conv_w"]), y)
    gs = torch.empty((1, Hv, DV, DK), dtype=torch.float32, device=gpu)
    gc = torch.empty((1, K - 1, D), dtype=torch.int16, device=gpu)
    pool.read(0, _ids([2]), gs, gc)
    yr, cr, sr = O.decode(conv, state, x, ab, p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
    assert np.array_equal(host(gc), cr)           # rolling conv state: bit-exact shift
    dy = float(np.max(np.abs(O.bf16_to_f32(host(y)) - O.bf16_to_f32(yr))))
    ds = rel_l2(host(gs), sr)
    say("gdn_decode config0 |dy|", dy, "state relL2", ds)
    assert dy <= Y_TOL and ds <= STATE_TOL
    assert pool.check() == 0


@pytest.mark.parametrize("Hk,Hv", [(4, 4), (4, 16)])
def test_decode_fused_other_head_ratios(gpu, Hk, Hv):
    import torch
    say("gdn_decode", f"Hk={Hk} Hv={Hv} B=5")
    rng = np.random.default_rng(310 + Hv)
    B = 5
    D = conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    st, cs = gen_states(rng, B, Hk, Hv)
    x, ab = gen_tokens(rng, B, Hk, Hv)
    pool = _pool(1, 9, Hk, Hv)
    slots = [8, 1, 4, 0, 6]
    pool.write(0, _ids(slots), dev(st), dev(cs))
    y = torch.zeros((B, Hv, DV), dtype=torch.int16, device=gpu)
    pool.decode(0, _ids(slots), dev(x), dev(ab), dev(p["A_log"]), dev(p["dt_bias"]),
                dev(p["conv_w"]), y)
    gs = torch.empty((B, Hv, DV, DK), dtype=torch.float32, device=gpu)
    gc = torch.empty((B, K - 1, D), dtype=torch.int16, device=gpu)
    pool.read(0, _ids(slots), gs, gc)
    yr, cr, sr = O.decode(cs, st, x, ab, p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
    assert np.array_equal(host(gc), cr)
    dy = float(np.max(np.abs(O.bf16_to_f32(host(y)) - O.bf16_to_f32(yr))))
    ds = rel_l2(host(gs), sr)
    say("gdn_decode worst |dy|", dy, "state relL2", ds)
    assert dy <= Y_TOL and ds <= STATE_TOL


def test_decode_chained_config1(gpu):
    """30 layers x 256-slot pools, B=8 at scattered slots, 64 chained steps;
    every layer's y checked each step, states after the run, untouched slots
    bit-exact."""
    import torch
    L, S, B, steps, Hk, Hv = 30, 256, 8, 64, 16, 32
    D = conv_dim(Hk, Hv)
    say("gdn_decode chained", f"config1 L={L} S={S} B={B} steps={steps}")
    rng = np.random.default_rng(400)
    slots = np.sort(rng.choice(S, B, replace=False)).astype(np.int32)
    rng.shuffle(slots)
    assert np.any(np.diff(np.sort(slots)) > 1)
    pool = _pool(L, S)
    params = [gen_layer_params(rng, Hk, Hv) for _ in range(L)]
    dparams = [{k: dev(v) for k, v in p.items()} for p in params]
    # every slot of every layer starts from a seeded random state (device-side)
    gen = torch.Generator(device=gpu).manual_seed(401)
    snap = []
    ids_all = _ids(np.arange(S))
    for l in range(L):
        s0 = torch.randn((S, Hv, DV, DK), generator=gen, device=gpu) * 0.01
        c0 = (torch.randn((S, K - 1, D), generator=gen, device=gpu)).to(torch.bfloat16).view(torch.int16)
        pool.write(l, ids_all, s0, c0)
        snap.append((s0, c0))
    st = [host(snap[l][0][torch.from_numpy(slots).long().to(gpu)]) for l in range(L)]
    cs = [host(snap[l][1][torch.from_numpy(slots).long().to(gpu)]) for l in range(L)]
    d_ids = _ids(slots)
    y = torch.zeros((B, Hv, DV), dtype=torch.int16, device=gpu)
    worst_y = 0.0
    for step in range(steps):
        for l in range(L):
            x, ab = gen_tokens(rng, B, Hk, Hv)
            pool.decode(l, d_ids, dev(x), dev(ab), dparams[l]["A_log"], dparams[l]["dt_bias"],
                        dparams[l]["conv_w"], y)
            yr, cs[l], st[l] = O.decode(cs[l], st[l], x, ab, params[l]["A_log"],
                                        params[l]["dt_bias"], params[l]["conv_w"], Hk, Hv)
            worst_y = max(worst_y, float(np.max(np.abs(O.bf16_to_f32(host(y)) - O.bf16_to_f32(yr)))))
    assert worst_y <= Y_TOL
    out_s = torch.empty((S, Hv, DV, DK), dtype=torch.float32, device=gpu)
    out_c = torch.empty((S, K - 1, D), dtype=torch.int16, device=gpu)
    untouched = torch.from_numpy(np.setdiff1d(np.arange(S), slots)).long().to(gpu)
    worst_s = 0.0
    for l in range(L):
        pool.read(l, ids_all, out_s, out_c)
        assert torch.equal(out_s[untouched], snap[l][0][untouched])
        assert torch.equal(out_c[untouched], snap[l][1][untouched])
        sl = torch.from_numpy(slots).long().to(gpu)
        assert np.array_equal(host(out_c[sl]), cs[l])
        worst_s = max(worst_s, rel_l2(host(out_s[sl]), st[l]))
    assert worst_s <= STATE_TOL
    say("config1 worst |dy|", worst_y, "worst state relL2", worst_s)
    assert pool.check() == 0


@pytest.mark.parametrize("Hk,Hv,B", [(16, 32, 1), (16, 32, 6), (4, 16, 5)])
def test_decode_gated_matches_oracle_and_plain_decode(gpu, Hk, Hv, B):
    """gdn_decode_gated on merged qkvz rows (with padding columns after z):
    out = silu(z) * rms_norm(y, w, eps) against the oracle; state, conv window
    and y bit-identical to gdn_decode on a twin pool; y may be omitted."""
    import torch
    say("gdn_decode_gated", f"Hk={Hk} Hv={Hv} B={B}")
    rng = np.random.default_rng(900 + Hk + Hv + B)
    D = conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    st, cs = gen_states(rng, B, Hk, Hv)
    x, ab = gen_tokens(rng, B, Hk, Hv)
    z = O.f32_to_bf16(rng.standard_normal((B, Hv * DV)).astype(np.float32))
    norm_w = O.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(DV)).astype(np.float32))
    eps = 1e-6
    pad = 24
    qkvz = np.zeros((B, D + Hv * DV + pad), np.uint16)
    qkvz[:, :D] = x
    qkvz[:, D:D + Hv * DV] = z
    qkvz[:, D + Hv * DV:] = O.f32_to_bf16(np.full((B, pad), 7.0, np.float32))
    slots = [int(s) for s in rng.choice(2 * B + 2, B, replace=False)]
    ids = _ids(slots)
    pa, pb = _pool(1, 2 * B + 2, Hk, Hv), _pool(1, 2 * B + 2, Hk, Hv)
    for pool in (pa, pb):
        pool.write(0, ids, dev(st), dev(cs))
    args = (dev(ab), dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]))
    y_plain = torch.zeros((B, Hv, DV), dtype=torch.int16, device=gpu)
    pa.decode(0, ids, dev(x), *args, y_plain)
    y_g = torch.zeros((B, Hv, DV), dtype=torch.int16, device=gpu)
    out = torch.zeros((B, Hv, DV), dtype=torch.int16, device=gpu)
    pb.decode_gated(0, ids, dev(qkvz), *args, dev(norm_w), eps, out, y_g)
    sa = torch.empty((B, Hv, DV, DK), dtype=torch.float32, device=gpu)
    sb = torch.empty_like(sa)
    ca = torch.empty((B, K - 1, D), dtype=torch.int16, device=gpu)
    cb = torch.empty_like(ca)
    pa.read(0, ids, sa, ca)
    pb.read(0, ids, sb, cb)
    assert torch.equal(sa, sb) and torch.equal(ca, cb) and torch.equal(y_plain, y_g)
    yr, _, _ = O.decode(cs, st, x, ab, p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
    ref = O.norm_gate(yr, z.reshape(B, Hv, DV), norm_w, eps)
    do = float(np.max(np.abs(O.bf16_to_f32(host(out)) - O.bf16_to_f32(ref))))
    # the same epilogue on the GPU's own y isolates the epilogue's rounding
    ref_own = O.norm_gate(host(y_g), z.reshape(B, Hv, DV), norm_w, eps)
    do_own = float(np.max(np.abs(O.bf16_to_f32(host(out)) - O.bf16_to_f32(ref_own))))
    say("gdn_decode_gated |d out| vs oracle", do, "vs epilogue on own y", do_own,
        "max |out|", float(np.max(np.abs(O.bf16_to_f32(ref)))))
    assert do <= Y_TOL and do_own <= Y_TOL
    # y omitted: same out
    out2 = torch.zeros_like(out)
    pc = _pool(1, 2 * B + 2, Hk, Hv)
    pc.write(0, ids, dev(st), dev(cs))
    pc.decode_gated(0, ids, dev(qkvz), *args, dev(norm_w), eps, out2)
    assert torch.equal(out, out2)
    for pool in (pa, pb, pc):
        assert pool.check() == 0
