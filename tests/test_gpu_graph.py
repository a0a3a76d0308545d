"""The decode path under HIP graph capture.

gdn_decode and gdn_layer_decode launch kernels only (no memset nodes, no
allocation once the pool's buffers are reserved), so a caller can capture a
whole decode step -- every layer -- in one graph and replay it. Each replay
here is checked bit for bit against the same step run eagerly on a twin pool,
with new inputs copied into the graph's static buffers and unrelated eager work
between replays.
"""
import numpy as np
import pytest

from gdn_testlib import DK, DV, K, O, conv_dim, dev, gen_layer_params, gen_states, gen_tokens, say

pytestmark = pytest.mark.gpu


def _read_all(pool, layers, ids, B, gpu):
    import torch
    out = []
    for l in range(layers):
        s = torch.empty((B, pool.Hv, DV, DK), dtype=torch.float32, device=gpu)
        c = torch.empty((B, K - 1, pool.D), dtype=torch.int16, device=gpu)
        pool.read(l, ids, s, c)
        out.append((s, c))
    return out


def test_decode_step_graph_replays_match_eager(gpu):
    """Three layers of gdn_decode for B=6 scattered slots captured once and
    replayed for 5 steps."""
    import torch

    import gdn_amd
    Hk, Hv, B, L, S = 16, 32, 6, 3, 24
    say("graph: gdn_decode", f"B={B} layers={L}")
    rng = np.random.default_rng(1300)
    params = [gen_layer_params(rng, Hk, Hv) for _ in range(L)]
    slots = rng.permutation(S)[:B].astype(np.int32)
    ids = dev(slots)
    st, cs = gen_states(rng, B, Hk, Hv)
    pe, pg = gdn_amd.Pool(L, S, Hk, Hv), gdn_amd.Pool(L, S, Hk, Hv)
    for pool in (pe, pg):
        for l in range(L):
            pool.write(l, ids, dev(st), dev(cs))
    w = [(dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"])) for p in params]
    x_static = torch.zeros((B, conv_dim(Hk, Hv)), dtype=torch.int16, device=gpu)
    ab_static = torch.zeros((B, 2 * Hv), dtype=torch.int16, device=gpu)
    y_static = torch.zeros((L, B, Hv, DV), dtype=torch.int16, device=gpu)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for l in range(L):
                pg.decode(l, ids, x_static, ab_static, *w[l], y_static[l])
    torch.cuda.synchronize()
    # capture recorded the launches without running them: pool g is untouched
    for (s0, c0), (s1, c1) in zip(_read_all(pe, L, ids, B, gpu), _read_all(pg, L, ids, B, gpu)):
        assert torch.equal(s0, s1) and torch.equal(c0, c1)
    y_eager = torch.zeros_like(y_static)
    for step in range(5):
        x, ab = gen_tokens(rng, B, Hk, Hv)
        xd, abd = dev(x), dev(ab)
        for l in range(L):
            pe.decode(l, ids, xd, abd, *w[l], y_eager[l])
        x_static.copy_(xd)
        ab_static.copy_(abd)
        graph.replay()
        junk = torch.randn(1 << 20, device=gpu).sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(y_eager, y_static), step
        for l, ((s0, c0), (s1, c1)) in enumerate(zip(_read_all(pe, L, ids, B, gpu),
                                                     _read_all(pg, L, ids, B, gpu))):
            assert torch.equal(s0, s1) and torch.equal(c0, c1), (step, l)
    assert pe.check() == 0 and pg.check() == 0


def test_layer_decode_graph_replays_match_eager(gpu):
    """Two whole GDN layers (in_proj, fused decode + norm-gate, K-split out_proj)
    of B=4 sequences captured once after gdn_pool_reserve, replayed 4 times."""
    import torch

    import gdn_amd
    from gdn_testlib import quantize_w4
    Hk, Hv, hidden, B, L, S = 4, 16, 1024, 4, 2, 8
    say("graph: gdn_layer_decode", f"B={B} layers={L} hidden={hidden}")
    rng = np.random.default_rng(1310)
    D = conv_dim(Hk, Hv)
    pools = [gdn_amd.Pool(L, S, Hk, Hv), gdn_amd.Pool(L, S, Hk, Hv)]
    slots = rng.permutation(S)[:B].astype(np.int32)
    ids = dev(slots)
    st, cs = gen_states(rng, B, Hk, Hv)
    for pool in pools:
        for l in range(L):
            pool.write(l, ids, dev(st), dev(cs))
        pool.reserve(B)
    keep, layers = [], [[], []]
    for l in range(L):
        ip = gdn_amd.QLinear(hidden, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in
                                      [quantize_w4(rng.standard_normal((n, hidden)) * 0.03)
                                       for n in (D, Hv * DV, Hv, Hv)]])
        w, s, b = quantize_w4(rng.standard_normal((hidden, Hv * DV)) * 0.03)
        op = gdn_amd.QLinear(Hv * DV, [(dev(w.view(np.int32)), dev(s), dev(b))])
        p = gen_layer_params(rng, Hk, Hv)
        nw = dev(O.f32_to_bf16((1 + 0.1 * rng.standard_normal(DV)).astype(np.float32)))
        t = (dev(p["A_log"]), dev(p["dt_bias"]), dev(p["conv_w"]), nw)
        keep += [ip, op, t]
        for k in range(2):
            layers[k].append(gdn_amd.Layer(pools[k], l, ip, op, t[0], t[1], t[2], t[3], 1e-6))
    x_static = torch.zeros((B, hidden), dtype=torch.int16, device=gpu)
    h_static = [torch.zeros((B, hidden), dtype=torch.int16, device=gpu) for _ in range(L)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            inp = x_static
            for l in range(L):
                layers[1][l].decode(ids, inp, h_static[l])
                inp = h_static[l]
    torch.cuda.synchronize()
    for step in range(4):
        x = dev(O.f32_to_bf16(rng.standard_normal((B, hidden)).astype(np.float32)))
        inp = x
        h_eager = []
        for l in range(L):
            o = torch.empty((B, hidden), dtype=torch.int16, device=gpu)
            layers[0][l].decode(ids, inp, o)
            h_eager.append(o)
            inp = o
        x_static.copy_(x)
        graph.replay()
        junk = torch.randn(1 << 20, device=gpu).sum()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for l in range(L):
            assert torch.equal(h_eager[l], h_static[l]), (step, l)
        for l, ((s0, c0), (s1, c1)) in enumerate(zip(_read_all(pools[0], L, ids, B, gpu),
                                                     _read_all(pools[1], L, ids, B, gpu))):
            assert torch.equal(s0, s1) and torch.equal(c0, c1), (step, l)
    for pool in pools:
        assert pool.check() == 0
    for k in range(2):
        for layer in layers[k]:
            layer.close()
