"""GPU parity of the whole GatedDeltaNet layer (gdn_layer_decode /
gdn_layer_prefill: GatedDeltaNet::forward_with_cache, qwen3_5.rs:558-668):

  * bit-identical to the chain of the separately tested entry points
    (gdn_qlinear_forward -> gdn_decode_gated / gdn_prefill_varlen_gated ->
    gdn_qlinear_forward) on a twin pool, outputs and slot states;
  * against the oracle's composition of the same steps (quantized_matmul,
    decode / prefill, norm_gate, quantized_matmul), end to end: the bf16
    roundings of three stages stack up, so the bar is a relative L2 error of
    the layer output plus the per-stage tolerances of the chain's own tests.
"""
import numpy as np
import pytest

from gdn_testlib import (O, DK, DV, K, conv_dim, dev, gen_layer_params, gen_states, host,
                         quantize_w4, rel_l2, say)

pytestmark = pytest.mark.gpu

OUT_REL_TOL = 1e-2
STATE_TOL = 1e-3


def _weights(rng, Hk, Hv, hidden):
    D = conv_dim(Hk, Hv)
    rows = [D, Hv * DV, Hv, Hv]  # q|k|v, z, b, a
    in_parts = [quantize_w4(rng.standard_normal((n, hidden)) * 0.02) for n in rows]
    out_part = quantize_w4(rng.standard_normal((hidden, Hv * DV)) * 0.02)
    p = gen_layer_params(rng, Hk, Hv)
    p["norm_w"] = O.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(DV)).astype(np.float32))
    return in_parts, out_part, p


def _merged(parts):
    return tuple(np.concatenate([q[i] for q in parts]) for i in range(3))


def _qlinear(K_, parts):
    import gdn_amd
    return gdn_amd.QLinear(K_, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in parts])


class _Model:
    """Device weights of one layer, a gdn_amd.Layer on `pool`, and the oracle chain."""

    def __init__(self, rng, Hk, Hv, hidden, eps=1e-6):
        self.Hk, self.Hv, self.hidden, self.eps = Hk, Hv, hidden, eps
        self.D = conv_dim(Hk, Hv)
        self.in_parts, self.out_part, self.p = _weights(rng, Hk, Hv, hidden)
        self.in_proj = _qlinear(hidden, self.in_parts)
        self.out_proj = _qlinear(Hv * DV, [self.out_part])
        self.dA, self.ddt = dev(self.p["A_log"]), dev(self.p["dt_bias"])
        self.dcw, self.dnw = dev(self.p["conv_w"]), dev(self.p["norm_w"])

    def layer(self, pool):
        import gdn_amd
        return gdn_amd.Layer(pool, 0, self.in_proj, self.out_proj, self.dA, self.ddt, self.dcw,
                             self.dnw, self.eps)

    def split(self, proj):
        D, HvDv = self.D, self.Hv * DV
        return proj[:, :D], proj[:, D:D + HvDv], proj[:, D + HvDv:]

    def project(self, x, gpu):
        """The GPU's projection of x (the kernel's rows are independent, so the
        layer's internal projection of the same rows has the same bits)."""
        import torch
        proj = torch.empty((len(x), self.in_proj.N), dtype=torch.int16, device=gpu)
        self.in_proj.forward(dev(x), proj)
        return proj

    # The oracle chain. With proj given (the GPU's projection bits) the conv
    # windows it returns are the exact expectation of the layer's; without, the
    # whole layer is the oracle's.
    def oracle_decode(self, x, cs, st, proj=None):
        if proj is None:
            proj, _, _ = O.qmatmul_w4(x, *_merged(self.in_parts))
        qkv, z, ab = self.split(proj)
        y, cs2, st2 = O.decode(cs, st, qkv, ab, self.p["A_log"], self.p["dt_bias"],
                               self.p["conv_w"], self.Hk, self.Hv)
        g = O.norm_gate(y, z.reshape(y.shape), self.p["norm_w"], self.eps)
        out, _, _ = O.qmatmul_w4(g.reshape(len(x), -1), *self.out_part)
        return out, cs2, st2

    def oracle_prefill(self, x, cs, st, proj=None):
        if proj is None:
            proj, _, _ = O.qmatmul_w4(x, *_merged(self.in_parts))
        qkv, z, ab = self.split(proj)
        y, cs2, st2 = O.prefill(cs, st, qkv, ab, self.p["A_log"], self.p["dt_bias"],
                                self.p["conv_w"], self.Hk, self.Hv)
        g = O.norm_gate(y, z.reshape(y.shape), self.p["norm_w"], self.eps)
        out, _, _ = O.qmatmul_w4(g.reshape(len(x), -1), *self.out_part)
        return out, cs2, st2


def _read(pool, slots, gpu):
    import torch
    n = len(slots)
    s = torch.empty((n, pool.Hv, DV, DK), dtype=torch.float32, device=gpu)
    c = torch.empty((n, K - 1, pool.D), dtype=torch.int16, device=gpu)
    pool.read(0, dev(np.asarray(slots, np.int32)), s, c)
    return host(s), host(c)


def _out_check(got, ref, what):
    r = rel_l2(O.bf16_to_f32(got), O.bf16_to_f32(ref))
    say(what, "out relL2 vs oracle", r)
    assert r <= OUT_REL_TOL, (what, r)


@pytest.mark.parametrize("Hk,Hv,hidden,B", [(16, 32, 2048, 8), (4, 16, 1024, 3)])
def test_layer_decode_matches_chain_and_oracle(gpu, Hk, Hv, hidden, B):
    import gdn_amd
    import torch
    say("gdn_layer_decode", f"Hk={Hk} Hv={Hv} hidden={hidden} B={B}")
    rng = np.random.default_rng(1100 + Hk + B)
    m = _Model(rng, Hk, Hv, hidden)
    nslots = 2 * B + 1
    slots = rng.permutation(nslots)[:B].astype(np.int32)
    ids = dev(slots)
    st, cs = gen_states(rng, B, Hk, Hv)
    pa, pb = gdn_amd.Pool(1, nslots, Hk, Hv), gdn_amd.Pool(1, nslots, Hk, Hv)
    for pool in (pa, pb):
        pool.write(0, ids, dev(st), dev(cs))
    layer = m.layer(pa)
    x = O.f32_to_bf16(rng.standard_normal((B, hidden)).astype(np.float32))
    xpad = np.zeros((B, hidden + 8), np.uint16)
    xpad[:, :hidden] = x
    out = torch.full((B, hidden + 4), -1, dtype=torch.int16, device=gpu)
    layer.decode(ids, dev(xpad)[:, :hidden], out[:, :hidden])
    # the chain on pool b
    proj = m.project(x, gpu)
    gated = torch.empty((B, Hv, DV), dtype=torch.int16, device=gpu)
    D, HvDv = m.D, Hv * DV
    pb.decode_gated(0, ids, proj[:, :D + HvDv], proj[:, D + HvDv:], m.dA, m.ddt, m.dcw, m.dnw,
                    m.eps, gated)
    out_c = torch.empty((B, hidden), dtype=torch.int16, device=gpu)
    m.out_proj.forward(gated.view(B, HvDv), out_c)
    torch.cuda.synchronize()
    oh = host(out)
    assert np.all(oh[:, hidden:] == 0xFFFF), "columns past hidden were written"
    assert np.array_equal(oh[:, :hidden], host(out_c))
    sa, ca = _read(pa, slots, gpu)
    sb, cb = _read(pb, slots, gpu)
    assert np.array_equal(sa, sb) and np.array_equal(ca, cb)
    ref, _, st_ref = m.oracle_decode(x, cs, st)
    _out_check(oh[:, :hidden], ref, "layer decode")
    ref_p, cs_ref, st_ref_p = m.oracle_decode(x, cs, st, host(proj))
    _out_check(oh[:, :hidden], ref_p, "layer decode (oracle on the GPU projection)")
    assert np.array_equal(ca, cs_ref)
    assert max(rel_l2(sa[i], st_ref[i]) for i in range(B)) <= STATE_TOL
    assert max(rel_l2(sa[i], st_ref_p[i]) for i in range(B)) <= STATE_TOL
    assert pa.check() == 0 and pb.check() == 0
    layer.close()


def test_layer_prefill_then_decode_matches_chain_and_oracle(gpu):
    """Packed prefill of lengths {1, 5, 0, 64, 130} from zeroed and nonzero
    slots, then two decode steps of all sequences from the handed-off states."""
    import gdn_amd
    import torch
    Hk, Hv, hidden = 4, 16, 1024
    lens = [1, 5, 0, 64, 130]
    say("gdn_layer_prefill", f"Hk={Hk} Hv={Hv} hidden={hidden} lens={lens}")
    rng = np.random.default_rng(1150)
    m = _Model(rng, Hk, Hv, hidden)
    n, T = len(lens), sum(lens)
    slots = rng.permutation(n + 2)[:n].astype(np.int32)
    ids = dev(slots)
    st, cs = gen_states(rng, n, Hk, Hv, state_std=0.05)
    st[:2] = 0.0
    cs[:2] = 0
    pa, pb = gdn_amd.Pool(1, n + 2, Hk, Hv), gdn_amd.Pool(1, n + 2, Hk, Hv)
    for pool in (pa, pb):
        pool.write(0, ids, dev(st), dev(cs))
    pa.reserve(T)
    layer = m.layer(pa)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = O.f32_to_bf16(rng.standard_normal((T, hidden)).astype(np.float32))
    out = torch.empty((T, hidden), dtype=torch.int16, device=gpu)
    layer.prefill(ids, dev(cu), T, dev(x), out)
    proj = m.project(x, gpu)
    gated = torch.empty((T, Hv, DV), dtype=torch.int16, device=gpu)
    D, HvDv = m.D, Hv * DV
    pb.prefill_gated(0, ids, dev(cu), T, proj[:, :D + HvDv], proj[:, D + HvDv:], m.dA, m.ddt,
                     m.dcw, m.dnw, m.eps, gated)
    out_c = torch.empty((T, hidden), dtype=torch.int16, device=gpu)
    m.out_proj.forward(gated.view(T, HvDv), out_c)
    torch.cuda.synchronize()
    assert torch.equal(out, out_c)
    sa, ca = _read(pa, slots, gpu)
    sb, cb = _read(pb, slots, gpu)
    assert np.array_equal(sa, sb) and np.array_equal(ca, cb)
    oh, ph = host(out), host(proj)
    cs_ref, st_ref = cs.copy(), st.copy()
    for i, L in enumerate(lens):
        if L == 0:
            assert np.array_equal(sa[i], st[i]) and np.array_equal(ca[i], cs[i])
            continue
        a, b = cu[i], cu[i + 1]
        ref, _, st_pure = m.oracle_prefill(x[a:b], cs[i], st[i])
        _out_check(oh[a:b], ref, f"layer prefill seq {i} len {L}")
        assert rel_l2(sa[i], st_pure) <= STATE_TOL
        ref, cs_ref[i], st_ref[i] = m.oracle_prefill(x[a:b], cs[i], st[i], ph[a:b])
        _out_check(oh[a:b], ref, f"layer prefill seq {i} len {L} (oracle on the GPU projection)")
        assert np.array_equal(ca[i], cs_ref[i])
        assert rel_l2(sa[i], st_ref[i]) <= STATE_TOL
    for step in range(2):
        xd = O.f32_to_bf16(rng.standard_normal((n, hidden)).astype(np.float32))
        od = torch.empty((n, hidden), dtype=torch.int16, device=gpu)
        layer.decode(ids, dev(xd), od)
        pd = host(m.project(xd, gpu))
        ref, cs_ref, st_ref = m.oracle_decode(xd, cs_ref, st_ref, pd)
        _out_check(host(od), ref, f"layer decode after prefill, step {step}")
    sa, ca = _read(pa, slots, gpu)
    assert np.array_equal(ca, cs_ref)
    assert max(rel_l2(sa[i], st_ref[i]) for i in range(n)) <= STATE_TOL
    assert pa.check() == 0 and pb.check() == 0
    layer.close()


def test_layer_argument_checks(gpu):
    import gdn_amd
    import torch
    rng = np.random.default_rng(1160)
    Hk, Hv, hidden = 4, 16, 512
    m = _Model(rng, Hk, Hv, hidden)
    pool = gdn_amd.Pool(1, 4, Hk, Hv)
    with pytest.raises(gdn_amd.GdnError):  # projections swapped
        gdn_amd.Layer(pool, 0, m.out_proj, m.in_proj, m.dA, m.ddt, m.dcw, m.dnw, 1e-6)
    with pytest.raises(gdn_amd.GdnError):  # layer index outside the pool
        gdn_amd.Layer(pool, 1, m.in_proj, m.out_proj, m.dA, m.ddt, m.dcw, m.dnw, 1e-6)
    other = gdn_amd.Pool(1, 4, 2, 8)
    with pytest.raises(gdn_amd.GdnError):  # in_proj width does not match the pool's heads
        gdn_amd.Layer(other, 0, m.in_proj, m.out_proj, m.dA, m.ddt, m.dcw, m.dnw, 1e-6)
    layer = m.layer(pool)
    ids = dev(np.array([0, 1], np.int32))
    x = torch.zeros((2, hidden + 8), dtype=torch.int16, device=gpu)
    out = torch.zeros((2, hidden), dtype=torch.int16, device=gpu)
    with pytest.raises(gdn_amd.GdnError):  # misaligned input rows
        layer.decode(ids, x[:, 4:hidden + 4], out)
    layer.decode(ids[:0], x[:0, :hidden], out[:0])  # B = 0 is a no-op
    assert pool.check() == 0
    layer.close()
