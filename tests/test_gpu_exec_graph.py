"""The executor's decode steps replayed from HIP graphs (one set of segments
per batch size, attention calls between them run eagerly) against the same
steps run launch by launch (GDN_EXEC_GRAPHS=0 at create): twin executors on
twin pools and caches, sharing the weights, fed the same requests. Every
step's tokens and logits must be bit-identical, through batch-size changes,
releases and admissions, submit/collect pipelining, and for the GatedDeltaNet-
only and the hybrid stack (attention layer at position 2)."""
import os

import numpy as np
import pytest

from gdn_testlib import O, DV, conv_dim, dev, quantize_w4

pytestmark = pytest.mark.gpu

HK, HV, HIDDEN, VOCAB = 8, 16, 512, 2048
HQ, HKV, THETA, ROT, EPS = 8, 2, 1.0e7, 64, 1e-6


def _bfw(rng, n, s=0.1):
    return O.f32_to_bf16((1 + s * rng.standard_normal(n)).astype(np.float32))


def _weights(rng, hybrid):
    D = conv_dim(HK, HV)
    layers = []
    for _ in range(2):
        layers.append(dict(
            in_parts=[quantize_w4(rng.standard_normal((n, HIDDEN)) * 0.05)
                      for n in (D, HV * DV, HV, HV)],
            out=quantize_w4(rng.standard_normal((HIDDEN, HV * DV)) * 0.03),
            A_log=rng.uniform(0.0, np.log(16.0), HV).astype(np.float32),
            dt_bias=(rng.standard_normal(HV) * 0.1).astype(np.float32),
            conv_w=O.f32_to_bf16((rng.standard_normal((D, 4)) * 0.25).astype(np.float32)),
            norm_w=_bfw(rng, DV), in_norm=_bfw(rng, HIDDEN)))
    nqkv = HQ * 512 + 2 * HKV * 256
    attn = dict(qkv=quantize_w4(rng.standard_normal((nqkv, HIDDEN)) * 0.05),
                o=quantize_w4(rng.standard_normal((HIDDEN, HQ * 256)) * 0.03),
                qn=_bfw(rng, 256), kn=_bfw(rng, 256), in_norm=_bfw(rng, HIDDEN))
    return dict(layers=layers, attn=attn if hybrid else None, final=_bfw(rng, HIDDEN),
                embed=O.f32_to_bf16(rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32)),
                head=quantize_w4(rng.standard_normal((VOCAB, HIDDEN)) * 0.05))


def _executor(W, graphs):
    import gdn_amd

    def ql(K_, parts):
        return gdn_amd.QLinear(K_, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in parts])

    pool = gdn_amd.Pool(2, 6, HK, HV)
    layers = [gdn_amd.Layer(pool, i, ql(HIDDEN, L["in_parts"]), ql(HV * DV, [L["out"]]),
                            dev(L["A_log"]), dev(L["dt_bias"]), dev(L["conv_w"]),
                            dev(L["norm_w"]), EPS) for i, L in enumerate(W["layers"])]
    norms = [dev(L["in_norm"]) for L in W["layers"]]
    kv, attn_dev = None, []
    if W["attn"] is not None:
        a = W["attn"]
        kv = gdn_amd.KVCache(1, 6, 48, 8, HQ, HKV, max_step_tokens=256)
        attn_dev = [(2, ql(HIDDEN, [a["qkv"]]), ql(HQ * 256, [a["o"]]), dev(a["qn"]), dev(a["kn"]))]
        norms.append(dev(a["in_norm"]))
    old = os.environ.get("GDN_EXEC_GRAPHS")
    if graphs:
        os.environ.pop("GDN_EXEC_GRAPHS", None)
    else:
        os.environ["GDN_EXEC_GRAPHS"] = "0"
    try:
        ex = gdn_amd.Executor(pool, layers, norms, dev(W["final"]), dev(W["embed"]),
                              ql(HIDDEN, [W["head"]]), EPS, 6, 256, attn_layers=attn_dev, kv=kv,
                              rope_theta=THETA, rotary_dim=ROT)
    finally:
        if old is None:
            os.environ.pop("GDN_EXEC_GRAPHS", None)
        else:
            os.environ["GDN_EXEC_GRAPHS"] = old
    return ex


@pytest.mark.parametrize("hybrid", [False, True], ids=["gdn_only", "hybrid"])
def test_graph_replay_matches_eager(gpu, hybrid):
    W = _weights(np.random.default_rng(2600 + hybrid), hybrid)
    eager, graph = _executor(W, False), _executor(W, True)
    rng = np.random.default_rng(7)
    prompts = {s: list(rng.integers(0, VOCAB, n)) for s, n in ((1, 9), (2, 40), (3, 5), (4, 17))}
    cur = {}

    def both(fn):
        a, b = fn(eager), fn(graph)
        assert a == b
        return a

    def logits_equal(tag):
        le = eager.logits().cpu().numpy()
        lg = graph.logits().cpu().numpy()
        assert le.shape == lg.shape and np.array_equal(le, lg), tag

    firsts = both(lambda ex: ex.prefill_batch([1, 2], [prompts[1], prompts[2]]))
    cur.update({1: firsts[0], 2: firsts[1]})
    cur[3] = both(lambda ex: ex.prefill(3, prompts[3]))

    def step(ids, tag, pipelined=False):
        toks = [cur[i] for i in ids]
        if pipelined:
            nxt = both(lambda ex: (ex.submit_batch(ids, toks), ex.collect_batch(len(ids)))[1])
        else:
            nxt = both(lambda ex: ex.decode_batch(ids, toks))
        logits_equal(tag)
        cur.update(dict(zip(ids, nxt)))

    for k in range(5):
        step([1, 2, 3], f"B3 step {k}")
    step([3, 1], "B2 step")                      # a second batch size
    for ex in (eager, graph):
        ex.release(2)
    cur[4] = both(lambda ex: ex.prefill(4, prompts[4]))
    for k in range(3):
        step([4, 1, 3], f"B3 after admit {k}", pipelined=k % 2 == 1)
    step([1], "B1 step")
    for k in range(2):
        step([3, 4, 1], f"B3 again {k}")
    eager.close()
    graph.close()


@pytest.mark.parametrize("hybrid", [False, True], ids=["gdn_only", "hybrid"])
def test_chained_steps_match_host_fed(gpu, hybrid):
    """gdn_exec_submit_next: steps fed their predecessor's picks on the device,
    one queued ahead of each collect, against the same steps fed from the host
    (launched kernel by kernel): the tokens of every step and the last step's
    logits are identical, also after a batch-size change; a release ends the
    chain."""
    import gdn_amd

    W = _weights(np.random.default_rng(2700 + hybrid), hybrid)
    fed, chained = _executor(W, False), _executor(W, True)
    rng = np.random.default_rng(11)
    prompts = [list(rng.integers(0, VOCAB, n)) for n in (12, 33, 7)]
    ids = [1, 2, 3]
    first = fed.prefill_batch(ids, prompts)
    assert chained.prefill_batch(ids, prompts) == first

    def host_fed(ids_, cur, n):
        out = []
        for _ in range(n):
            cur = fed.decode_batch(ids_, cur)
            out.append(cur)
        return out

    def run_chained(ids_, cur, n):
        B = len(ids_)
        chained.submit_batch(ids_, cur)
        out = []
        for _ in range(n - 1):
            chained.submit_next(B)
            out.append(chained.collect_batch(B))
        out.append(chained.collect_batch(B))
        return out

    ref = host_fed(ids, first, 7)
    assert run_chained(ids, first, 7) == ref
    assert np.array_equal(fed.logits().cpu().numpy(), chained.logits().cpu().numpy())
    cur = dict(zip(ids, ref[-1]))
    sub = [3, 1]
    ref2 = host_fed(sub, [cur[i] for i in sub], 4)
    assert run_chained(sub, [cur[i] for i in sub], 4) == ref2
    assert np.array_equal(fed.logits().cpu().numpy(), chained.logits().cpu().numpy())
    chained.release(2)
    with pytest.raises(gdn_amd.GdnError):
        chained.submit_next(2)
    fed.close()
    chained.close()


def test_wide_head_pick_matches_host_argmax(gpu):
    """An lm_head wide enough (131,136 columns, over 131,072; its last 128-column
    tile part padding) to take the wide projection (x copied into LDS by DMA,
    three waves per SIMD): every decode step's tokens equal the argmax of that
    step's bf16 logits read back (first index of the maximum), on the
    graph-replaying and the eager executor alike."""
    V = 131136
    rng = np.random.default_rng(2800)
    W = _weights(rng, False)
    W["embed"] = O.f32_to_bf16(rng.standard_normal((V, HIDDEN)).astype(np.float32))
    W["head"] = quantize_w4(rng.standard_normal((V, HIDDEN)) * 0.05)
    eager, graph = _executor(W, False), _executor(W, True)
    ids = [1, 2, 3]
    prompts = [list(rng.integers(0, V, n)) for n in (7, 19, 3)]
    cur = graph.prefill_batch(ids, prompts)
    assert eager.prefill_batch(ids, prompts) == cur
    for step in range(4):
        nxt = graph.decode_batch(ids, cur)
        assert eager.decode_batch(ids, cur) == nxt, step
        lg = O.bf16_to_f32(graph.logits().cpu().numpy().view(np.uint16))
        assert lg.shape == (3, V)
        assert [int(i) for i in np.argmax(lg, axis=1)] == nxt, step
        cur = nxt
    eager.close()
    graph.close()
