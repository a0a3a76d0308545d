"""GPU tests of the executor over the hybrid decoder stack: GatedDeltaNet
layers and attention layers (Qwen35Attention::forward_with_cache,
qwen3_5.rs:377-455) interleaved, the attention layers' KV cache keyed by the
pool's slot ids (gdn_exec_desc.attn_layers / kv).

The stack here is [GDN, attention, GDN, attention] at hidden 1024 with
Qwen's attention heads (16 query heads with output gates, 2 kv heads, head
dim 256, RoPE over 64 dimensions, base 1e7). Attention results do not depend
on what else runs in a step, so the executor keeps its defining property:
every sequence's tokens equal its solo run bit for bit, under both scheduler
loops of the reference. The logits of one sequence are also compared with a
composition of separately tested calls (gdn_amd.Layer, QLinear, KVCache on
twins, torch float32 for the body's norms and residual).
"""
import numpy as np
import pytest

from gdn_testlib import O, DV, dev, quantize_w4, rel_l2, say
from test_gpu_exec import (EPS, HIDDEN, HK, HV, VOCAB, _qlinear, _ref_norm, _requests,
                           _serve_loop, _solo, _step_loop)

pytestmark = pytest.mark.gpu

HQ, HKV, HD, THETA, ROT = 16, 2, 256, 1.0e7, 64
NQKV = HQ * 2 * HD + 2 * HKV * HD  # q|gate per head, then k, then v
POS = (1, 3)                        # attention positions; GDN at 0 and 2


def _bf(a):
    return O.f32_to_bf16(np.asarray(a, np.float32))


class _Hybrid:
    def __init__(self, seed):
        rng = np.random.default_rng(seed)
        D = 2 * HK * 128 + HV * DV
        self.gdn = []
        for _ in range(2):
            in_parts = [quantize_w4(rng.standard_normal((n, HIDDEN)) * 0.03)
                        for n in (D, HV * DV, HV, HV)]
            self.gdn.append(dict(
                in_proj=_qlinear(HIDDEN, in_parts),
                out_proj=_qlinear(HV * DV, [quantize_w4(rng.standard_normal((HIDDEN, HV * DV)) * 0.03)]),
                A_log=dev(rng.uniform(0.0, np.log(16.0), HV).astype(np.float32)),
                dt_bias=dev((rng.standard_normal(HV) * 0.1).astype(np.float32)),
                conv_w=dev(_bf(rng.standard_normal((D, 4)) * 0.25)),
                norm_w=dev(_bf(1 + 0.1 * rng.standard_normal(DV)))))
        self.attn = [dict(qkv=_qlinear(HIDDEN, [quantize_w4(rng.standard_normal((NQKV, HIDDEN)) * 0.03)]),
                          o=_qlinear(HQ * HD, [quantize_w4(rng.standard_normal((HIDDEN, HQ * HD)) * 0.03)]),
                          qn=dev(_bf(1 + 0.1 * rng.standard_normal(HD))),
                          kn=dev(_bf(1 + 0.1 * rng.standard_normal(HD)))) for _ in range(2)]
        self.in_norm = [_bf(1 + 0.1 * rng.standard_normal(HIDDEN)) for _ in range(4)]
        self.final_norm = _bf(1 + 0.1 * rng.standard_normal(HIDDEN))
        self.embed = _bf(rng.standard_normal((VOCAB, HIDDEN)))
        self.head = _qlinear(HIDDEN, [quantize_w4(rng.standard_normal((VOCAB, HIDDEN)) * 0.03)])

    def gdn_layers(self, pool):
        import gdn_amd
        return [gdn_amd.Layer(pool, i, L["in_proj"], L["out_proj"], L["A_log"], L["dt_bias"],
                              L["conv_w"], L["norm_w"], EPS) for i, L in enumerate(self.gdn)]

    def executor(self, slots, max_batch=8, max_prompt=160, pages=64):
        import gdn_amd
        pool = gdn_amd.Pool(2, slots, HK, HV)
        kv = gdn_amd.KVCache(2, slots, pages, 8, HQ, HKV, max_step_tokens=max(max_batch, max_prompt))
        attn = [(p, a["qkv"], a["o"], a["qn"], a["kn"]) for p, a in zip(POS, self.attn)]
        ex = gdn_amd.Executor(pool, self.gdn_layers(pool), [dev(w) for w in self.in_norm],
                              dev(self.final_norm), dev(self.embed), self.head, EPS, max_batch,
                              max_prompt, attn_layers=attn, kv=kv, rope_theta=THETA,
                              rotary_dim=ROT)
        return pool, kv, ex


@pytest.fixture(scope="module")
def hybrid(gpu):
    return _Hybrid(1250)


@pytest.mark.parametrize("loop", ["step", "serve"])
def test_hybrid_tokens_do_not_depend_on_batching(hybrid, loop):
    """12 requests (prompts 1..128 tokens) through a 6-slot pool in batches of
    up to 4, slots and KV pages reused as sequences finish: each sequence's
    tokens equal its solo run bit for bit, and every page comes back."""
    say("gdn_exec hybrid", f"{loop} loop, 12 requests, 6 slots, max_batch 4")
    eos = {5}
    pool, kv, ex = hybrid.executor(6, max_batch=4)
    reqs = _requests(1251, 12)
    run = _step_loop if loop == "step" else _serve_loop
    finished = run(ex, reqs, 4, 2, [6], eos)
    assert sorted(s.id for s in finished) == sorted(r.id for r in reqs)
    assert pool.slots_in_use() == 0 and kv.free_pages() == 64
    for s in finished:
        solo = _solo(ex, s, eos)
        assert s.out == solo, (s.id, s.out, solo)
    assert pool.check() == 0 and kv.free_pages() == 64
    say("gdn_exec hybrid tokens", {s.id: len(s.out) for s in finished})
    ex.close()


def test_hybrid_logits_match_composition(hybrid):
    """Prefill of a 70-token prompt (two KV pages) then 4 decode steps of one
    sequence; after each forward the executor's logits are compared with the
    same stack built from separately tested calls on twins (relative L2
    1e-2: the composition's norms are torch float32, not the executor's
    kernel)."""
    import torch

    import gdn_amd
    say("gdn_exec hybrid", "logits vs composition, 1 sequence")
    pool, kv, ex = hybrid.executor(3, max_batch=2)
    twin = gdn_amd.Pool(2, 3, HK, HV)
    tkv = gdn_amd.KVCache(2, 3, 64, 8, HQ, HKV, max_step_tokens=160)
    layers = hybrid.gdn_layers(twin)
    emb = dev(hybrid.embed).view(torch.bfloat16)
    fin = dev(hybrid.final_norm).view(torch.bfloat16)
    norms = [dev(w).view(torch.bfloat16) for w in hybrid.in_norm]
    prompt = [int(t) for t in np.random.default_rng(1252).integers(0, VOCAB, 70)]
    tok = ex.prefill(88, prompt)
    sl = ex.slot(88)
    slot = dev(np.array([sl], np.int32))
    twin.zero(-1, slot)
    q0 = HQ * 2 * HD

    def forward(tokens, prefill):
        h = emb[torch.tensor(tokens, device="cuda:0")]
        n = h.shape[0]
        tkv.step([sl], [n])
        gi = ai = 0
        for p in range(4):
            hn = _ref_norm(h, norms[p]).view(torch.int16)
            out = torch.empty((n, HIDDEN), dtype=torch.int16, device="cuda:0")
            if p in POS:
                a = hybrid.attn[ai]
                qkv = torch.empty((n, NQKV), dtype=torch.int16, device="cuda:0")
                a["qkv"].forward(hn, qkv)
                att = torch.empty((n, HQ * HD), dtype=torch.int16, device="cuda:0")
                tkv.forward(ai, qkv[:, :q0], qkv[:, q0:q0 + HKV * HD], qkv[:, q0 + HKV * HD:],
                            a["qn"], a["kn"], EPS, THETA, ROT, att)
                a["o"].forward(att, out)
                ai += 1
            else:
                if prefill:
                    layers[gi].prefill(slot, dev(np.array([0, n], np.int32)), n, hn, out)
                else:
                    layers[gi].decode(slot, hn, out)
                gi += 1
            h = (h.float() + out.view(torch.bfloat16).float()).bfloat16()
        hn = _ref_norm(h[-1:], fin)
        logits = torch.empty((1, VOCAB), dtype=torch.int16, device="cuda:0")
        hybrid.head.forward(hn.view(torch.int16), logits)
        return logits.view(torch.bfloat16).float()

    ref = forward(prompt, True)
    got = ex.logits()[-1:].view(torch.bfloat16).float()
    worst = rel_l2(got.cpu().numpy(), ref.cpu().numpy())
    assert int(torch.argmax(got)) == tok
    for step in range(4):
        nxt = ex.decode_batch([88], [tok])[0]
        got = ex.logits()[:1].view(torch.bfloat16).float()
        ref = forward([tok], False)
        worst = max(worst, rel_l2(got.cpu().numpy(), ref.cpu().numpy()))
        assert int(torch.argmax(got)) == nxt
        tok = nxt
    say("gdn_exec hybrid logits relL2 vs composition", worst)
    assert worst <= 1e-2
    # the executor's KV cache holds what the composition's does. The first
    # attention layer's rows are bit-identical; later ones can carry the
    # composition's float32 torch norms (rsqrt, mean order), which flip a
    # bf16 rounding of the normed input now and then.
    for layer in range(2):
        for x, y in zip(kv.read(layer, sl), tkv.read(layer, sl)):
            a = O.bf16_to_f32(x.cpu().numpy().view(np.uint16))
            b = O.bf16_to_f32(y.cpu().numpy().view(np.uint16))
            say(f"kv layer {layer}", f"{int(np.sum(a != b))} of {a.size} differ, "
                                     f"relL2 {rel_l2(a, b):.2e}")
            if layer == 0:
                assert np.array_equal(a, b)
            assert rel_l2(a, b) <= 1e-2, layer
    ex.release(88)
    assert kv.length(sl) == 0
    for layer in layers:
        layer.close()
    tkv.close()
    ex.close()


def test_hybrid_kv_pages_run_out(hybrid):
    """A 4-page cache: a prompt needing more pages than are free is refused
    before anything changes (the new sequence is not admitted); a decode step
    that needs a page no one can give fails the same way; releasing frees
    pages for both."""
    import gdn_amd
    say("gdn_exec hybrid", "KV pages run out")
    pool, kv, ex = hybrid.executor(4, max_batch=4, pages=4)
    t1 = ex.prefill(1, list(range(1, 129)))      # 128 tokens: 2 pages
    with pytest.raises(gdn_amd.GdnError):
        ex.prefill(2, list(range(1, 200)))      # 199 tokens: 4 pages, 2 free
    assert pool.slots_in_use() == 1 and kv.free_pages() == 2
    t2 = ex.prefill(2, list(range(1, 129)))     # 2 pages: now full
    assert kv.free_pages() == 0
    with pytest.raises(gdn_amd.GdnError):       # position 128 needs a third page each
        ex.decode_batch([1, 2], [t1, t2])
    assert kv.length(ex.slot(1)) == 128 and kv.length(ex.slot(2)) == 128
    ex.release(2)
    assert kv.free_pages() == 2
    assert len(ex.decode_batch([1], [t1])) == 1
    assert kv.free_pages() == 1 and kv.length(ex.slot(1)) == 129
    ex.close()
    assert pool.slots_in_use() == 0


def test_hybrid_descriptor_checks(hybrid):
    """gdn_exec_create refuses attention layers that do not fit: positions
    out of order or past the stack, projections of the wrong shape, a KV cache
    with fewer slots than the pool or too few step tokens."""
    import gdn_amd
    pool = gdn_amd.Pool(2, 4, HK, HV)
    layers = hybrid.gdn_layers(pool)
    norms = [dev(w) for w in hybrid.in_norm]
    a0, a1 = hybrid.attn

    def make(attn, kv, max_prompt=64):
        return gdn_amd.Executor(pool, layers, norms, dev(hybrid.final_norm), dev(hybrid.embed),
                                hybrid.head, EPS, 4, max_prompt, attn_layers=attn, kv=kv)

    def spec(p, a):
        return (p, a["qkv"], a["o"], a["qn"], a["kn"])

    kv = gdn_amd.KVCache(2, 4, 16, 4, HQ, HKV, max_step_tokens=64)
    for bad in ([spec(3, a0), spec(1, a1)],                       # not increasing
                [spec(1, a0), spec(4, a1)],                       # past the 4-layer stack
                [spec(1, a0), (3, a1["o"], a1["qkv"], a1["qn"], a1["kn"])]):  # swapped projections
        with pytest.raises(gdn_amd.GdnError):
            make(bad, kv)
    with pytest.raises(gdn_amd.GdnError):                        # 2 slots < the pool's 4
        make([spec(1, a0), spec(3, a1)], gdn_amd.KVCache(2, 2, 16, 4, HQ, HKV, max_step_tokens=64))
    with pytest.raises(gdn_amd.GdnError):                        # 32 step tokens < 64 rows
        make([spec(1, a0), spec(3, a1)], gdn_amd.KVCache(2, 4, 16, 4, HQ, HKV, max_step_tokens=32))
    with pytest.raises(gdn_amd.GdnError):                        # one kv layer for two
        make([spec(1, a0), spec(3, a1)], gdn_amd.KVCache(1, 4, 16, 4, HQ, HKV, max_step_tokens=64))
    ex = make([spec(1, a0), spec(3, a1)], kv)
    assert ex.prefill(1, [1, 2, 3]) >= 0
    ex.close()
    for layer in layers:
        layer.close()


def test_hybrid_failed_restart_changes_nothing(hybrid):
    """A restart (prefill of a known sequence) that the KV cache cannot hold
    fails before anything changes: the sequence keeps its slot, pages and
    state, and decodes on exactly as in a twin run without the failed call.
    An executor whose max_prompt exceeds one slot's KV pages is refused."""
    import gdn_amd
    say("gdn_exec hybrid", "failed restart, max_prompt vs pages per slot")
    pool = gdn_amd.Pool(2, 4, HK, HV)
    kv = gdn_amd.KVCache(2, 4, 16, 2, HQ, HKV, max_step_tokens=200)  # 128 tokens per slot
    attn = [(p, a["qkv"], a["o"], a["qn"], a["kn"]) for p, a in zip(POS, hybrid.attn)]
    with pytest.raises(gdn_amd.GdnError):
        gdn_amd.Executor(pool, hybrid.gdn_layers(pool), [dev(w) for w in hybrid.in_norm],
                         dev(hybrid.final_norm), dev(hybrid.embed), hybrid.head, EPS, 2, 200,
                         attn_layers=attn, kv=kv, rope_theta=THETA, rotary_dim=ROT)
    rng = np.random.default_rng(1260)
    pa = [int(t) for t in rng.integers(0, VOCAB, 100)]   # 2 pages
    pb = [int(t) for t in rng.integers(0, VOCAB, 150)]   # 3 pages
    long_prompt = [int(t) for t in rng.integers(0, VOCAB, 160)]
    runs = []
    for fail in (False, True):
        pool, kv, ex = hybrid.executor(4, max_batch=2, max_prompt=160, pages=5)
        toks = [ex.prefill(1, pa), ex.prefill(2, pb)]
        out = []
        for _ in range(8):
            toks = ex.decode_batch([1, 2], toks)
            out.append(tuple(toks))
        slot_a = ex.slot(1)
        if fail:
            # needs 3 pages; free 0 + the 2 sequence 1 gives back
            with pytest.raises(gdn_amd.GdnError):
                ex.prefill(1, long_prompt)
            assert ex.slot(1) == slot_a and pool.slots_in_use() == 2 and kv.free_pages() == 0
        for _ in range(8):
            toks = ex.decode_batch([1, 2], toks)
            out.append(tuple(toks))
        assert pool.check() == 0
        runs.append(out)
        ex.close()
    assert runs[0] == runs[1]
