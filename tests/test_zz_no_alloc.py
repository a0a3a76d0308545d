"""GPU test of gdn_prefill_varlen_noalloc (the prefill with a fixed per-device
scratch workspace) against gdn_prefill_varlen on twin pools: outputs and the
slots' recurrent and conv states bit-identical, over two calls in a row, the
second smaller, and a 2,048-token prompt on the split schedule; oversized calls
are refused on the host. The same call
captured in a HIP graph and replayed gives the eager call's results, and an
eager call leaves the device's free memory unchanged."""
import numpy as np
import pytest

from gdn_testlib import DK, DV, K, dev, gen_layer_params, gen_states, gen_tokens, host, say

pytestmark = pytest.mark.gpu

HK, HV = 16, 32


def _ids(lst):
    return dev(np.asarray(lst, np.int32))


def _call(pool, noalloc, slots, lens, x, ab, p, gpu):
    import torch
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total = int(cu[-1])
    y = torch.zeros((total, HV, DV), dtype=torch.int16, device=gpu)
    fn = pool.prefill_noalloc if noalloc else pool.prefill
    fn(0, _ids(slots), dev(cu), total, dev(x), dev(ab), dev(p["A_log"]), dev(p["dt_bias"]),
       dev(p["conv_w"]), y)
    s = torch.empty((len(slots), HV, DV, DK), dtype=torch.float32, device=gpu)
    c = torch.empty((len(slots), K - 1, pool.D), dtype=torch.int16, device=gpu)
    pool.read(0, _ids(slots), s, c)
    torch.cuda.synchronize()
    return host(y), host(s), host(c)


def test_noalloc_prefill_matches_prefill(gpu):
    import torch
    import gdn_amd
    rng = np.random.default_rng(1400)
    p = gen_layer_params(rng, HK, HV)
    pools = [gdn_amd.Pool(1, 12, HK, HV) for _ in range(2)]
    slots = [9, 2, 5, 11]
    st, cs = gen_states(rng, len(slots), HK, HV)
    for pool in pools:
        pool.write(0, _ids(slots), dev(st), dev(cs))
    # two calls in a row on the same slots, the second smaller; then one prompt
    # of 2,048 tokens alone, which takes the split schedule (its records fit the
    # scratch), continuing slot 9
    for sl, lens in ((slots, [70, 300, 5, 129]), (slots, [33, 2, 64, 1]), ([9], [2048])):
        say("gdn_prefill_varlen_noalloc", f"slots={sl} lens={lens}")
        x, ab = gen_tokens(rng, int(sum(lens)), HK, HV)
        ya, sa, ca = _call(pools[0], False, sl, lens, x, ab, p, gpu)
        yb, sb, cb = _call(pools[1], True, sl, lens, x, ab, p, gpu)
        assert np.array_equal(ya, yb)
        assert np.array_equal(sa, sb)
        assert np.array_equal(ca, cb)
    s0 = torch.empty((len(slots), HV, DV, DK), dtype=torch.float32, device=gpu)
    c0 = torch.empty((len(slots), K - 1, pools[1].D), dtype=torch.int16, device=gpu)
    pools[1].read(0, _ids(slots), s0, c0)
    torch.cuda.synchronize()
    sb, cb = host(s0), host(c0)
    # a call beyond the fixed scratch (64 MiB: 4,048 tokens at 16/32 heads on the
    # fused schedule) fails before any launch, changing nothing
    big = 4049
    x, ab = gen_tokens(rng, big, HK, HV)
    ybig = torch.zeros((big, HV, DV), dtype=torch.int16, device=gpu)
    with pytest.raises(gdn_amd.GdnError, match="scratch"):
        pools[1].prefill_noalloc(0, _ids([3]), dev(np.array([0, big], np.int32)), big, dev(x),
                                 dev(ab), dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]),
                                 ybig)
    s = torch.empty((len(slots), HV, DV, DK), dtype=torch.float32, device=gpu)
    c = torch.empty((len(slots), K - 1, pools[1].D), dtype=torch.int16, device=gpu)
    pools[1].read(0, _ids(slots), s, c)
    torch.cuda.synchronize()
    assert np.array_equal(host(s), sb) and np.array_equal(host(c), cb)
    for pool in pools:
        assert pool.check() == 0
        pool.close()


def test_noalloc_prefill_in_hip_graph(gpu):
    """gdn_prefill_varlen_noalloc captured in a HIP graph (torch.cuda.graph on
    the stream the binding passes) and replayed three times, the slots' state
    restored by eager writes between replays: every replay's y, recurrent and
    conv state bit-identical to the eager call's. Device memory in use is the
    same before and after an eager call (hipMemGetInfo)."""
    import torch
    import gdn_amd
    rng = np.random.default_rng(1500)
    p = gen_layer_params(rng, HK, HV)
    pools = [gdn_amd.Pool(1, 12, HK, HV) for _ in range(2)]
    slots = [4, 10, 0, 7]
    lens = [70, 300, 5, 129]
    st, cs = gen_states(rng, len(slots), HK, HV)
    x, ab = gen_tokens(rng, int(sum(lens)), HK, HV)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total = int(cu[-1])
    d_ids, d_cu, d_x, d_ab = _ids(slots), dev(cu), dev(x), dev(ab)
    d_al, d_dt, d_cw = dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"])
    d_st, d_cs = dev(st), dev(cs)
    for pool in pools:
        pool.write(0, d_ids, d_st, d_cs)
    torch.cuda.synchronize()
    # the eager reference on pool 0, free device memory around it
    ya = torch.zeros((total, HV, DV), dtype=torch.int16, device=gpu)
    free0 = torch.cuda.mem_get_info()[0]
    pools[0].prefill_noalloc(0, d_ids, d_cu, total, d_x, d_ab, d_al, d_dt, d_cw, ya)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    say("noalloc eager call", f"free device memory before {free0} after {free1}")
    assert free1 == free0, "the no-allocation prefill changed device memory in use"
    s = torch.empty((len(slots), HV, DV, DK), dtype=torch.float32, device=gpu)
    c = torch.empty((len(slots), K - 1, pools[0].D), dtype=torch.int16, device=gpu)
    pools[0].read(0, d_ids, s, c)
    torch.cuda.synchronize()
    ref = (host(ya), host(s), host(c))
    # captured on pool 1 (an eager call first sets the device's scratch address up)
    yb = torch.zeros((total, HV, DV), dtype=torch.int16, device=gpu)
    pools[1].prefill_noalloc(0, d_ids, d_cu, total, d_x, d_ab, d_al, d_dt, d_cw, yb)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pools[1].prefill_noalloc(0, d_ids, d_cu, total, d_x, d_ab, d_al, d_dt, d_cw, yb)
    for rep in range(3):
        pools[1].write(0, d_ids, d_st, d_cs)
        yb.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        pools[1].read(0, d_ids, s, c)
        torch.cuda.synchronize()
        say("noalloc graph replay", rep)
        assert np.array_equal(host(yb), ref[0]), rep
        assert np.array_equal(host(s), ref[1]), rep
        assert np.array_equal(host(c), ref[2]), rep
    del graph
    for pool in pools:
        assert pool.check() == 0
        pool.close()
