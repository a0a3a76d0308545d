"""GPU parity of the varlen prefill (gdn_prefill_varlen) against the oracle's
sequential per-sequence prefill (the reference prefills one sequence at a
time with one T-long recurrence launch), including the hand-off of final
recurrent and conv states into slots for later decode steps."""
import numpy as np
import pytest

from gdn_testlib import (O, DK, DV, K, conv_dim, dev, gen_layer_params, gen_states, gen_tokens,
                         host, rel_l2, say)

pytestmark = pytest.mark.gpu

Y_TOL = 2e-2
STATE_TOL = 1e-3
OUT_REL_TOL = 1e-2


def _ids(lst):
    return dev(np.asarray(lst, np.int32))


def _run_prefill(pool, layer, slots, lens, mixed, ab, p, gpu):
    import torch
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total = int(cu[-1])
    Hv = pool.Hv
    y = torch.zeros((max(total, 1), Hv, DV), dtype=torch.int16, device=gpu)
    pool.prefill(layer, _ids(slots), dev(cu), total, dev(mixed) if total else None,
                 dev(ab) if total else None, dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]),
                 y if total else None)
    return host(y)[:total], cu


def _read(pool, layer, slots, gpu):
    import torch
    n = len(slots)
    s = torch.empty((n, pool.Hv, DV, DK), dtype=torch.float32, device=gpu)
    c = torch.empty((n, K - 1, pool.D), dtype=torch.int16, device=gpu)
    pool.read(layer, _ids(slots), s, c)
    return host(s), host(c)


@pytest.fixture
def prefill_waves(monkeypatch):
    """Force the prefill's path: GDN_PREFILL_WAVES = 8 (fused chunk kernel),
    4 or 2 (split path: prefill_form_kernel, then 2 or 4 groups per head);
    0 leaves the choice to the library."""
    def force(w):
        if w:
            monkeypatch.setenv("GDN_PREFILL_WAVES", str(w))
        else:
            monkeypatch.delenv("GDN_PREFILL_WAVES", raising=False)
    return force


@pytest.mark.parametrize("waves", [0, 4])
def test_prefill_mixed_batch_config3(gpu, prefill_waves, waves):
    """4 prefills {128, 512, 1000, 2048} (the 1000 one ends in a partial
    64-token chunk) + 28 single-token decodes in one layer, then 3 decode
    steps for all 32 sequences from the handed-off states; with the library's
    choice of schedule and with the split schedule forced."""
    import gdn_amd
    import torch
    prefill_waves(waves)
    Hk, Hv = 16, 32
    lens = [128, 512, 1000, 2048]
    say("gdn_prefill_varlen", f"config3 lens={lens} + 28 decode, seed=500")
    rng = np.random.default_rng(500)
    pool = gdn_amd.Pool(1, 48, Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    slots = rng.permutation(48)[:32].astype(np.int32)
    pre_slots, dec_slots = slots[:4], slots[4:]
    # decode sequences carry random states; prefill slots are admitted (zeroed)
    dst, dcs = gen_states(rng, 28, Hk, Hv)
    pool.write(0, _ids(dec_slots), dev(dst), dev(dcs))
    pool.zero(0, _ids(pre_slots))
    mixed, ab = gen_tokens(rng, sum(lens), Hk, Hv)
    y, cu = _run_prefill(pool, 0, pre_slots, lens, mixed, ab, p, gpu)
    xd, abd = gen_tokens(rng, 28, Hk, Hv)
    yd = torch.zeros((28, Hv, DV), dtype=torch.int16, device=gpu)
    pool.decode(0, _ids(dec_slots), dev(xd), dev(abd), dev(p["A_log"]), dev(p["dt_bias"]),
                dev(p["conv_w"]), yd)
    # oracle: sequential prefill per sequence from zero state
    D = conv_dim(Hk, Hv)
    st_ref = np.zeros((32, Hv, DV, DK), np.float32)
    cs_ref = np.zeros((32, K - 1, D), np.uint16)
    worst_y = 0.0
    for i, L in enumerate(lens):
        a, b = cu[i], cu[i + 1]
        yr, cs_ref[i], st_ref[i] = O.prefill(np.zeros((K - 1, D), np.uint16),
                                             np.zeros((Hv, DV, DK), np.float32), mixed[a:b],
                                             ab[a:b], p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
        worst_y = max(worst_y, float(np.max(np.abs(O.bf16_to_f32(y[a:b]) - O.bf16_to_f32(yr)))))
    ydr, cs_ref[4:], st_ref[4:] = O.decode(dcs, dst, xd, abd, p["A_log"], p["dt_bias"],
                                           p["conv_w"], Hk, Hv)
    worst_y = max(worst_y, float(np.max(np.abs(O.bf16_to_f32(host(yd)) - O.bf16_to_f32(ydr)))))
    gs, gc = _read(pool, 0, slots, gpu)
    assert np.array_equal(gc, cs_ref)
    worst_s = max(rel_l2(gs[i], st_ref[i]) for i in range(32))
    say("config3 after prefill: worst |dy|", worst_y, "worst state relL2", worst_s)
    assert worst_y <= Y_TOL and worst_s <= STATE_TOL
    # hand-off: 3 decode steps over all 32 sequences
    ydec = torch.zeros((32, Hv, DV), dtype=torch.int16, device=gpu)
    for step in range(3):
        x, abx = gen_tokens(rng, 32, Hk, Hv)
        pool.decode(0, _ids(slots), dev(x), dev(abx), dev(p["A_log"]), dev(p["dt_bias"]),
                    dev(p["conv_w"]), ydec)
        yr, cs_ref, st_ref = O.decode(cs_ref, st_ref, x, abx, p["A_log"], p["dt_bias"],
                                      p["conv_w"], Hk, Hv)
        assert np.max(np.abs(O.bf16_to_f32(host(ydec)) - O.bf16_to_f32(yr))) <= Y_TOL
    gs, gc = _read(pool, 0, slots, gpu)
    assert np.array_equal(gc, cs_ref)
    assert max(rel_l2(gs[i], st_ref[i]) for i in range(32)) <= STATE_TOL
    assert pool.check() == 0


@pytest.mark.parametrize("Hk,Hv", [(16, 32), (2, 8), (4, 4)])
def test_prefill_edge_lengths_from_nonzero_state(gpu, Hk, Hv):
    """Lengths 1, 2, 3 (conv state mixes old rows), 0 (empty sequence: slot
    untouched), 63/64/65 around a chunk boundary; sequences continue from a
    nonzero state (prefill of a prompt continuation)."""
    import gdn_amd
    lens = [1, 2, 0, 3, 64, 65, 63]
    say("gdn_prefill_varlen", f"edge lens={lens} Hk={Hk} Hv={Hv}")
    rng = np.random.default_rng(510 + Hv)
    n = len(lens)
    pool = gdn_amd.Pool(1, n + 2, Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    slots = rng.permutation(n + 2)[:n].astype(np.int32)
    st0, cs0 = gen_states(rng, n, Hk, Hv, state_std=0.05)
    pool.write(0, _ids(slots), dev(st0), dev(cs0))
    mixed, ab = gen_tokens(rng, sum(lens), Hk, Hv)
    y, cu = _run_prefill(pool, 0, slots, lens, mixed, ab, p, gpu)
    gs, gc = _read(pool, 0, slots, gpu)
    for i, L in enumerate(lens):
        a, b = cu[i], cu[i + 1]
        if L == 0:
            assert np.array_equal(gs[i], st0[i]) and np.array_equal(gc[i], cs0[i])
            continue
        yr, csr, sr = O.prefill(cs0[i], st0[i], mixed[a:b], ab[a:b], p["A_log"], p["dt_bias"],
                                p["conv_w"], Hk, Hv)
        assert np.array_equal(gc[i], csr)
        assert np.max(np.abs(O.bf16_to_f32(y[a:b]) - O.bf16_to_f32(yr))) <= Y_TOL
        assert rel_l2(gs[i], sr) <= STATE_TOL
    assert pool.check() == 0


@pytest.mark.parametrize("waves", [8, 2])
def test_prefill_bad_cu_seqlens_are_flagged_and_clamped(gpu, prefill_waves, waves):
    """cu_seqlens must start at 0, not decrease and end at total_tokens; each
    violation latches GDN_FLAG_BAD_SEQLENS while the kernels clamp the bounds,
    so nothing outside the inputs or the named slots is touched. Both
    schedules (waves = 8: fused chunk kernel; 2: chunk records, then the split
    chunk kernel, whose record slots come from the clamped bounds)."""
    import torch
    import gdn_amd
    prefill_waves(waves)
    Hk, Hv = 2, 4
    D = conv_dim(Hk, Hv)
    rng = np.random.default_rng(620)
    p = gen_layer_params(rng, Hk, Hv)
    T = 12
    mixed, ab = gen_tokens(rng, T, Hk, Hv)
    pool = gdn_amd.Pool(1, 6, Hk, Hv)
    st, cs = gen_states(rng, 6, Hk, Hv)
    pool.write(0, _ids(list(range(6))), dev(st), dev(cs))
    args = (dev(mixed), dev(ab), dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]))
    y = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
    cases = {"decreasing": [0, 10, 4], "nonzero start": [2, 7, 12], "short end": [0, 4, 8],
             "past end": [0, 6, 20]}
    for name, cu in cases.items():
        say("bad cu_seqlens", name, cu)
        pool.prefill(0, _ids([1, 3]), dev(np.asarray(cu, np.int32)), T, *args, y)
        assert pool.check() == gdn_amd.GDN_FLAG_BAD_SEQLENS, name
    # slots never named keep their bytes
    gs = torch.empty((4, Hv, DV, DK), dtype=torch.float32, device=gpu)
    gc = torch.empty((4, K - 1, D), dtype=torch.int16, device=gpu)
    pool.read(0, _ids([0, 2, 4, 5]), gs, gc)
    assert np.array_equal(host(gs), st[[0, 2, 4, 5]])
    assert np.array_equal(host(gc), cs[[0, 2, 4, 5]])
    # a well-formed list raises nothing
    pool.prefill(0, _ids([1, 3]), dev(np.asarray([0, 5, 12], np.int32)), T, *args, y)
    assert pool.check() == 0


@pytest.mark.parametrize("Hk,Hv", [(16, 32), (4, 16)])
def test_prefill_gated_matches_oracle_and_plain_prefill(gpu, Hk, Hv):
    """gdn_prefill_varlen_gated on merged qkvz rows (padding columns after z)
    and ab rows read through a stride: out = silu(z) * rms_norm(y, w, eps)
    against the oracle; state, conv window and y bit-identical to
    gdn_prefill_varlen on a twin pool (the same kernels up to the epilogue);
    y may be omitted."""
    import gdn_amd
    import torch
    lens = [1, 3, 0, 64, 65, 200]
    say("gdn_prefill_varlen_gated", f"lens={lens} Hk={Hk} Hv={Hv}")
    rng = np.random.default_rng(530 + Hk + Hv)
    n, D = len(lens), conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    st0, cs0 = gen_states(rng, n, Hk, Hv, state_std=0.05)
    T = sum(lens)
    mixed, ab = gen_tokens(rng, T, Hk, Hv)
    z = O.f32_to_bf16(rng.standard_normal((T, Hv * DV)).astype(np.float32))
    norm_w = O.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(DV)).astype(np.float32))
    eps = 1e-6
    pad = 8
    qkvz = np.zeros((T, D + Hv * DV + pad), np.uint16)
    qkvz[:, :D] = mixed
    qkvz[:, D:D + Hv * DV] = z
    qkvz[:, D + Hv * DV:] = O.f32_to_bf16(np.full((T, pad), 5.0, np.float32))
    abw = np.zeros((T, 2 * Hv + 6), np.uint16)
    abw[:, :2 * Hv] = ab
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    slots = rng.permutation(n + 3)[:n].astype(np.int32)
    ids = _ids(slots)
    pools = [gdn_amd.Pool(1, n + 3, Hk, Hv) for _ in range(3)]
    for pool in pools:
        pool.write(0, ids, dev(st0), dev(cs0))
    args = (dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]))
    y_plain = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
    pools[0].prefill(0, ids, dev(cu), T, dev(mixed), dev(ab), *args, y_plain)
    y_g = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
    out = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
    pools[1].prefill_gated(0, ids, dev(cu), T, dev(qkvz), dev(abw)[:, :2 * Hv], *args,
                           dev(norm_w), eps, out, y_g)
    out2 = torch.zeros_like(out)
    pools[2].prefill_gated(0, ids, dev(cu), T, dev(qkvz), dev(abw)[:, :2 * Hv], *args,
                           dev(norm_w), eps, out2)
    sa, ca = _read(pools[0], 0, slots, gpu)
    for pool in pools[1:]:
        sb, cb = _read(pool, 0, slots, gpu)
        assert np.array_equal(sa, sb) and np.array_equal(ca, cb)
    assert torch.equal(y_plain, y_g) and torch.equal(out, out2)
    yo, oo = host(y_g), host(out)
    worst, worst_own = 0.0, 0.0
    for i, L in enumerate(lens):
        a, b = cu[i], cu[i + 1]
        if L == 0:
            continue
        yr, _, _ = O.prefill(cs0[i], st0[i], mixed[a:b], ab[a:b], p["A_log"], p["dt_bias"],
                             p["conv_w"], Hk, Hv)
        zr = z[a:b].reshape(L, Hv, DV)
        ref = O.norm_gate(yr, zr, norm_w, eps)
        # rms_norm divides by the head's rms of y, so y's absolute tolerance
        # turns into a relative one on out: bar on the relative L2 error
        worst = max(worst, rel_l2(O.bf16_to_f32(oo[a:b]), O.bf16_to_f32(ref)))
        # the same epilogue on the GPU's own y isolates the epilogue's rounding
        own = O.norm_gate(yo[a:b], zr, norm_w, eps)
        worst_own = max(worst_own,
                        float(np.max(np.abs(O.bf16_to_f32(oo[a:b]) - O.bf16_to_f32(own)))))
    say("gated prefill out relL2 vs oracle", worst, "|d out| vs epilogue on own y", worst_own)
    assert worst <= OUT_REL_TOL and worst_own <= Y_TOL
    for pool in pools:
        assert pool.check() == 0


@pytest.mark.parametrize("Hk,Hv", [(16, 32), (4, 16), (2, 8), (4, 4)])
def test_prefill_split_path_matches_fused(gpu, prefill_waves, Hk, Hv):
    """The split path (chunk records formed by prefill_form_kernel for all
    chunks at once, then 2 or 4 groups of 4 or 2 waves per head running only
    the state products, and for the gated call the separate epilogue) gives
    the same bits as the fused chunk kernel: the same products in the same
    order. Lengths cover partial chunks, an empty sequence, a chunk boundary
    and sequences that start mid-way through a 64-token slot; states start
    nonzero. Also the split path against the oracle."""
    import gdn_amd
    import torch
    lens = [700, 0, 1, 64, 129, 333]
    say("gdn_prefill_varlen split vs fused", f"lens={lens} Hk={Hk} Hv={Hv}")
    rng = np.random.default_rng(560 + Hk + Hv)
    n, D = len(lens), conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    st0, cs0 = gen_states(rng, n, Hk, Hv, state_std=0.05)
    T = sum(lens)
    mixed, ab = gen_tokens(rng, T, Hk, Hv)
    z = O.f32_to_bf16(rng.standard_normal((T, Hv * DV)).astype(np.float32))
    norm_w = O.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(DV)).astype(np.float32))
    qkvz = np.zeros((T, D + Hv * DV), np.uint16)
    qkvz[:, :D] = mixed
    qkvz[:, D:] = z
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    slots = rng.permutation(n + 2)[:n].astype(np.int32)
    ids = _ids(slots)
    args = (dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]))
    res = {}
    for w in (8, 4, 2):
        prefill_waves(w)
        pool = gdn_amd.Pool(1, n + 2, Hk, Hv)
        pool.write(0, ids, dev(st0), dev(cs0))
        y = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
        pool.prefill(0, ids, dev(cu), T, dev(mixed), dev(ab), *args, y)
        s, c = _read(pool, 0, slots, gpu)
        gpool = gdn_amd.Pool(1, n + 2, Hk, Hv)
        gpool.write(0, ids, dev(st0), dev(cs0))
        out = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
        gpool.prefill_gated(0, ids, dev(cu), T, dev(qkvz), dev(ab), *args, dev(norm_w), 1e-6, out)
        gs, gc = _read(gpool, 0, slots, gpu)
        assert pool.check() == 0 and gpool.check() == 0
        assert np.array_equal(s, gs) and np.array_equal(c, gc)
        res[w] = (host(y), s, c, host(out))
        pool.close()
        gpool.close()
    for w in (4, 2):
        for a, b, what in zip(res[8], res[w], ("y", "state", "conv", "gated out")):
            assert np.array_equal(a, b), f"W={w}: {what} differs from the fused path"
    y2, s2 = res[2][0], res[2][1]
    worst_y, worst_s = 0.0, 0.0
    for i, L in enumerate(lens):
        a, b = cu[i], cu[i + 1]
        yr, _, sr = O.prefill(cs0[i], st0[i], mixed[a:b], ab[a:b], p["A_log"], p["dt_bias"],
                              p["conv_w"], Hk, Hv)
        if L:
            worst_y = max(worst_y, float(np.max(np.abs(O.bf16_to_f32(y2[a:b]) - O.bf16_to_f32(yr)))))
        worst_s = max(worst_s, rel_l2(s2[i], sr))
    say("split path |dy|", worst_y, "state relL2", worst_s)
    assert worst_y <= Y_TOL and worst_s <= STATE_TOL


@pytest.fixture
def prefill_segments(monkeypatch):
    """Force the split path's pipeline: GDN_PREFILL_SEGMENTS = n segments (1:
    one pass); 0 leaves the choice to the library."""
    def force(n):
        if n:
            monkeypatch.setenv("GDN_PREFILL_SEGMENTS", str(n))
        else:
            monkeypatch.delenv("GDN_PREFILL_SEGMENTS", raising=False)
    return force


@pytest.mark.parametrize("Hk,Hv", [(16, 32), (4, 16), (4, 4)])
@pytest.mark.parametrize("waves", [2, 4])
def test_prefill_pipelined_segments_match_one_pass(gpu, prefill_waves, prefill_segments, Hk, Hv,
                                                   waves):
    """The split path run as a pipeline of token segments (qkv and form
    kernels of segment j + 1 on a second stream beside the chunk kernel of
    segment j, the state carried through the slot between the chunk kernel's
    launches) gives the bits of the one-pass call and of the fused path: y,
    state, conv window and the gated output. Segment counts 3 and 8 over
    sequences that start and end mid-way through 64-token tiles, an empty
    and a one-token sequence; states start nonzero."""
    import gdn_amd
    import torch
    lens = [700, 0, 1, 64, 129, 333, 5000]
    say("gdn_prefill_varlen pipelined", f"lens={lens} Hk={Hk} Hv={Hv} waves={waves}")
    rng = np.random.default_rng(590 + Hk + Hv + waves)
    n, D = len(lens), conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    st0, cs0 = gen_states(rng, n, Hk, Hv, state_std=0.05)
    T = sum(lens)
    mixed, ab = gen_tokens(rng, T, Hk, Hv)
    z = O.f32_to_bf16(rng.standard_normal((T, Hv * DV)).astype(np.float32))
    norm_w = O.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(DV)).astype(np.float32))
    qkvz = np.zeros((T, D + Hv * DV), np.uint16)
    qkvz[:, :D] = mixed
    qkvz[:, D:] = z
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    slots = rng.permutation(n + 2)[:n].astype(np.int32)
    ids = _ids(slots)
    args = (dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]))
    res = {}
    for w, segs in ((8, 1), (waves, 1), (waves, 3), (waves, 8)):
        prefill_waves(w)
        prefill_segments(segs)
        pool = gdn_amd.Pool(1, n + 2, Hk, Hv)
        pool.write(0, ids, dev(st0), dev(cs0))
        y = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
        pool.prefill(0, ids, dev(cu), T, dev(mixed), dev(ab), *args, y)
        s, c = _read(pool, 0, slots, gpu)
        gpool = gdn_amd.Pool(1, n + 2, Hk, Hv)
        gpool.write(0, ids, dev(st0), dev(cs0))
        out = torch.zeros((T, Hv, DV), dtype=torch.int16, device=gpu)
        gpool.prefill_gated(0, ids, dev(cu), T, dev(qkvz), dev(ab), *args, dev(norm_w), 1e-6, out)
        gs, gc = _read(gpool, 0, slots, gpu)
        assert pool.check() == 0 and gpool.check() == 0
        assert np.array_equal(s, gs) and np.array_equal(c, gc)
        res[(w, segs)] = (host(y), s, c, host(out))
        pool.close()
        gpool.close()
    ref = res[(8, 1)]
    for key, got in res.items():
        for a, b, what in zip(ref, got, ("y", "state", "conv", "gated out")):
            assert np.array_equal(a, b), f"waves, segments = {key}: {what} differs from the fused path"


def test_prefill_one_long_prompt_pipelined_matches_one_pass(gpu, prefill_segments):
    """One 16,384-token prompt takes the split path in 4 segments by default;
    its y, state and conv window equal the one-pass call's bit for bit, and a
    second call on the same pool (reusing its stream and events) gives the
    same bits again."""
    import gdn_amd
    import torch
    Hk, Hv, L = 16, 32, 16384
    say("gdn_prefill_varlen one long prompt, pipelined", f"L={L}")
    rng = np.random.default_rng(620)
    p = gen_layer_params(rng, Hk, Hv)
    st0, cs0 = gen_states(rng, 1, Hk, Hv, state_std=0.05)
    mixed, ab = gen_tokens(rng, L, Hk, Hv)
    cu = dev(np.asarray([0, L], np.int32))
    ids = _ids([1])
    args = (dev(mixed), dev(ab), dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]))
    res = []
    for segs in (1, 0, 0):
        prefill_segments(segs)
        pool = gdn_amd.Pool(1, 2, Hk, Hv)
        for _ in range(2 if segs == 0 else 1):
            pool.write(0, ids, dev(st0), dev(cs0))
            y = torch.zeros((L, Hv, DV), dtype=torch.int16, device=gpu)
            pool.prefill(0, ids, cu, L, *args, y)
            s, c = _read(pool, 0, [1], gpu)
            res.append((host(y), s, c))
        assert pool.check() == 0
        pool.close()
    for got in res[1:]:
        for a, b, what in zip(res[0], got, ("y", "state", "conv")):
            assert np.array_equal(a, b), f"pipelined call: {what} differs from one pass"
