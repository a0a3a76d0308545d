"""GPU tests of the executor (gdn_exec_*: ModelExecutor, executor.rs:21-49, over
pool slots).

The executor's defining property is that a sequence's tokens do not depend on
what else runs: every kernel of a step works on its rows / slots alone, so a
sequence decoded in any batch, next to sequences admitted and retired around
it, in pipelined submit / collect, gives bit-for-bit the tokens it gives when
run alone. The scheduler loops here restate the reference's callers:
TokenScheduler::step (scheduler.rs:96-174: prefill budget, round-robin batch,
requeue unfinished) and the pipelined serve loop of qwen_mlx_serve.rs:110-177
(collect -> prefill waiting -> submit). One sequence is also followed step by
step against a composition of separately tested pieces (gdn_amd.Layer on a twin
pool, torch float32 for the body's embedding / norm / head), comparing logits.
"""
from collections import deque

import numpy as np
import pytest

from gdn_testlib import O, DV, dev, quantize_w4, rel_l2, say

pytestmark = pytest.mark.gpu

HK, HV, HIDDEN, VOCAB, LAYERS = 4, 16, 1024, 10240, 3  # vocab: two greedy-pick chunks
EPS = 1e-6


def _qlinear(K_, parts):
    import gdn_amd
    return gdn_amd.QLinear(K_, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in parts])


class _Weights:
    def __init__(self, seed):
        rng = np.random.default_rng(seed)
        D = 2 * HK * 128 + HV * DV
        self.layers = []
        for _ in range(LAYERS):
            in_parts = [quantize_w4(rng.standard_normal((n, HIDDEN)) * 0.03)
                        for n in (D, HV * DV, HV, HV)]
            out_part = quantize_w4(rng.standard_normal((HIDDEN, HV * DV)) * 0.03)
            self.layers.append(dict(
                in_proj=_qlinear(HIDDEN, in_parts), out_proj=_qlinear(HV * DV, [out_part]),
                A_log=dev(rng.uniform(0.0, np.log(16.0), HV).astype(np.float32)),
                dt_bias=dev((rng.standard_normal(HV) * 0.1).astype(np.float32)),
                conv_w=dev(O.f32_to_bf16((rng.standard_normal((D, 4)) * 0.25).astype(np.float32))),
                norm_w=dev(O.f32_to_bf16((1 + 0.1 * rng.standard_normal(DV)).astype(np.float32))),
                in_norm=O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32))))
        self.final_norm = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32))
        self.embed = O.f32_to_bf16(rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32))
        self.head = _qlinear(HIDDEN, [quantize_w4(rng.standard_normal((VOCAB, HIDDEN)) * 0.03)])

    def gdn_layers(self, pool):
        import gdn_amd
        return [gdn_amd.Layer(pool, i, L["in_proj"], L["out_proj"], L["A_log"], L["dt_bias"],
                              L["conv_w"], L["norm_w"], EPS) for i, L in enumerate(self.layers)]

    def executor(self, slots, max_batch=8, max_prompt=160):
        import gdn_amd
        pool = gdn_amd.Pool(LAYERS, slots, HK, HV)
        ex = gdn_amd.Executor(pool, self.gdn_layers(pool),
                              [dev(L["in_norm"]) for L in self.layers], dev(self.final_norm),
                              dev(self.embed), self.head, EPS, max_batch, max_prompt)
        return pool, ex


@pytest.fixture(scope="module")
def weights(gpu):
    return _Weights(1200)


class _Seq:
    def __init__(self, sid, prompt, max_tokens):
        self.id, self.prompt, self.max_tokens = sid, prompt, max_tokens
        self.out, self.cur = [], None

    def push(self, tok, eos):
        self.out.append(tok)
        self.cur = tok
        return tok in eos or len(self.out) >= self.max_tokens  # should_stop, sequence.rs:131-134


def _requests(seed, n):
    rng = np.random.default_rng(seed)
    lens = [1, 7, 33, 64, 65, 100, 3, 20, 50, 128, 2, 90][:n]
    return [_Seq(100 + i, [int(t) for t in rng.integers(0, VOCAB, L)], int(rng.integers(3, 14)))
            for i, L in enumerate(lens)]


def _solo(ex, seq, eos):
    s = _Seq(seq.id, seq.prompt, seq.max_tokens)
    done = s.push(ex.prefill(s.id, s.prompt), eos)
    while not done:
        done = s.push(ex.decode_batch([s.id], [s.cur])[0], eos)
    ex.release(s.id)
    return s.out


def _step_loop(ex, reqs, max_batch, budget, free_slots, eos):
    """TokenScheduler::step (scheduler.rs:96-174) driven to completion; a
    sequence is admitted only while the pool has a free slot."""
    waiting, active, finished = deque(reqs), deque(), []
    while waiting or active:
        for _ in range(min(budget, len(waiting))):
            if free_slots[0] == 0:
                break
            s = waiting.popleft()
            free_slots[0] -= 1
            if s.push(ex.prefill(s.id, s.prompt), eos):
                ex.release(s.id)
                free_slots[0] += 1
                finished.append(s)
            else:
                active.append(s)
        B = min(max_batch, len(active))
        if B == 0:
            continue
        batch = [active.popleft() for _ in range(B)]
        toks = ex.decode_batch([s.id for s in batch], [s.cur for s in batch])
        for s, t in zip(batch, toks):
            if s.push(t, eos):
                ex.release(s.id)
                free_slots[0] += 1
                finished.append(s)
            else:
                active.append(s)
    return finished


def _serve_loop(ex, reqs, max_batch, budget, free_slots, eos):
    """run_scheduler_loop of qwen_mlx_serve.rs:110-177: collect the batch in
    flight, prefill waiting sequences (while the GPU still works on nothing),
    submit the next batch, and do host work before the next collect."""
    waiting, active, finished = deque(reqs), deque(), []
    inflight = []
    while waiting or active or inflight:
        if inflight:
            toks = ex.collect_batch(len(inflight))
            for s, t in zip(inflight, toks):
                if s.push(t, eos):
                    ex.release(s.id)
                    free_slots[0] += 1
                    finished.append(s)
                else:
                    active.append(s)
            inflight = []
        for _ in range(min(budget, len(waiting))):
            if free_slots[0] == 0:
                break
            s = waiting.popleft()
            free_slots[0] -= 1
            if s.push(ex.prefill(s.id, s.prompt), eos):
                ex.release(s.id)
                free_slots[0] += 1
                finished.append(s)
            else:
                active.append(s)
        B = min(max_batch, len(active))
        if B:
            inflight = [active.popleft() for _ in range(B)]
            ex.submit_batch([s.id for s in inflight], [s.cur for s in inflight])
    return finished


@pytest.mark.parametrize("loop", ["step", "serve"])
def test_executor_tokens_do_not_depend_on_batching(weights, loop):
    """12 requests (prompts 1..128 tokens, 3..13 new tokens, one EOS id) through
    a 6-slot pool with batches of up to 4: slots are reused as sequences
    finish. Each sequence's tokens equal its solo run, bit for bit."""
    say("gdn_exec", f"{loop} loop, 12 requests, 6 slots, max_batch 4")
    eos = {5}
    pool, ex = weights.executor(6, max_batch=4)
    reqs = _requests(1201, 12)
    run = _step_loop if loop == "step" else _serve_loop
    finished = run(ex, reqs, 4, 2, [6], eos)
    assert sorted(s.id for s in finished) == sorted(r.id for r in reqs)
    assert pool.slots_in_use() == 0
    assert pool.check() == 0
    for s in finished:
        solo = _solo(ex, s, eos)
        assert s.out == solo, (s.id, s.out, solo)
    say("gdn_exec tokens", {s.id: len(s.out) for s in finished})
    ex.close()


def test_executor_mirrors_reference_scheduler_tests(weights):
    """scheduler.rs:271-345 with the real executor: a single sequence runs to
    max_tokens; three interleaved sequences of max_tokens 3 count 6 decode
    tokens; with batch 1 two sequences alternate (round-robin)."""
    say("gdn_exec", "reference scheduler cases")
    pool, ex = weights.executor(4, max_batch=4)
    s = _Seq(1, [1, 2, 3], 5)
    out = _step_loop(ex, [s], 4, 1, [4], set())
    assert len(out[0].out) == 5
    reqs = [_Seq(10 + i, [i + 1], 3) for i in range(3)]
    decoded = []
    waiting, active = deque(reqs), deque()
    while waiting or active:
        if waiting:
            q = waiting.popleft()
            q.push(ex.prefill(q.id, q.prompt), set())
            active.append(q)
        batch = [active.popleft() for _ in range(min(4, len(active)))]
        for q, t in zip(batch, ex.decode_batch([q.id for q in batch], [q.cur for q in batch])):
            decoded.append(t)
            if q.push(t, set()):
                ex.release(q.id)
            else:
                active.append(q)
    assert len(decoded) == 6
    a, b = _Seq(20, [1], 100), _Seq(21, [2], 100)
    for q in (a, b):
        q.push(ex.prefill(q.id, q.prompt), set())
    order = deque([a, b])
    seen = []
    for _ in range(4):
        q = order.popleft()
        q.push(ex.decode_batch([q.id], [q.cur])[0], set())
        seen.append(q.id)
        order.append(q)
    assert seen == [20, 21, 20, 21]
    ex.release(20)
    ex.release(21)
    assert pool.slots_in_use() == 0
    ex.close()


def _ref_norm(h, w):
    """The body's residual-stream rms-norm in float32 torch: bf16(w * bf16(h * rn))."""
    import torch
    hf = h.float()
    rn = torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + EPS)
    return (w.float() * (hf * rn).bfloat16().float()).bfloat16()


def test_executor_logits_match_composition(weights):
    """Prefill then 4 decode steps of one sequence; after each forward the
    executor's logits are compared with the same model built from gdn_amd.Layer
    calls on a twin pool plus torch float32 embedding / norm / residual / head
    (the head through the same QLinear), fed the executor's tokens."""
    import gdn_amd
    import torch
    say("gdn_exec", "logits vs composition, 1 sequence")
    pool, ex = weights.executor(3, max_batch=2)
    twin = gdn_amd.Pool(LAYERS, 3, HK, HV)
    layers = weights.gdn_layers(twin)
    emb = dev(weights.embed).view(torch.bfloat16)
    fin = dev(weights.final_norm).view(torch.bfloat16)
    norms = [dev(L["in_norm"]).view(torch.bfloat16) for L in weights.layers]
    prompt = [int(t) for t in np.random.default_rng(1202).integers(0, VOCAB, 40)]
    tok = ex.prefill(77, prompt)
    slot = dev(np.array([ex.slot(77)], np.int32))
    twin.zero(-1, slot)

    def forward(tokens, prefill):
        h = emb[torch.tensor(tokens, device="cuda:0")]
        n = h.shape[0]
        for L, w, layer in zip(weights.layers, norms, layers):
            hn = _ref_norm(h, w)
            out = torch.empty((n, HIDDEN), dtype=torch.int16, device="cuda:0")
            if prefill:
                cu = dev(np.array([0, n], np.int32))
                layer.prefill(slot, cu, n, hn.view(torch.int16), out)
            else:
                layer.decode(slot, hn.view(torch.int16), out)
            h = (h.float() + out.view(torch.bfloat16).float()).bfloat16()
        hn = _ref_norm(h[-1:], fin)
        logits = torch.empty((1, VOCAB), dtype=torch.int16, device="cuda:0")
        weights.head.forward(hn.view(torch.int16), logits)
        return logits.view(torch.bfloat16).float()

    worst = 0.0
    ref = forward(prompt, True)
    got = ex.logits()[-1:].view(torch.bfloat16).float()
    worst = max(worst, rel_l2(got.cpu().numpy(), ref.cpu().numpy()))
    assert int(torch.argmax(got)) == tok
    for step in range(4):
        nxt = ex.decode_batch([77], [tok])[0]
        got = ex.logits()[:1].view(torch.bfloat16).float()
        ref = forward([tok], False)
        worst = max(worst, rel_l2(got.cpu().numpy(), ref.cpu().numpy()))
        assert int(torch.argmax(got)) == nxt
        tok = nxt
    say("gdn_exec logits relL2 vs composition", worst)
    assert worst <= 1e-2
    ex.release(77)
    assert pool.check() == 0 and twin.check() == 0
    for layer in layers:
        layer.close()
    ex.close()


def test_executor_errors_and_slots(weights):
    import gdn_amd
    say("gdn_exec", "argument errors, slot accounting")
    pool, ex = weights.executor(2, max_batch=2)
    assert ex.max_batch_size() == 2 and ex.supports_pipeline()
    t1 = ex.prefill(1, [3, 4])
    t2 = ex.prefill(2, [5])
    assert pool.slots_in_use() == 2
    with pytest.raises(gdn_amd.GdnError):  # pool full
        ex.prefill(3, [1])
    with pytest.raises(gdn_amd.GdnError):  # unknown sequence
        ex.decode_batch([1, 9], [t1, 0])
    with pytest.raises(gdn_amd.GdnError):  # the same sequence twice
        ex.decode_batch([1, 1], [t1, t1])
    with pytest.raises(gdn_amd.GdnError):  # token outside the vocabulary
        ex.decode_batch([1], [VOCAB])
    with pytest.raises(gdn_amd.GdnError):  # above max_batch
        ex.decode_batch([1, 2, 1], [t1, t2, t1])
    with pytest.raises(gdn_amd.GdnError):  # prompt token outside the vocabulary
        ex.prefill(1, [VOCAB + 1])
    with pytest.raises(gdn_amd.GdnError):  # collect before submit
        ex.collect_batch(1)
    ex.submit_batch([1, 2], [t1, t2])
    with pytest.raises(gdn_amd.GdnError):  # second submit before collect
        ex.submit_batch([1], [t1])
    # a prefill of a known sequence between submit and collect restarts it
    # (same slot, zeroed) after the batch in flight
    s1 = ex.slot(1)
    r1 = ex.prefill(1, [3, 4])
    assert ex.slot(1) == s1 and r1 == t1
    ex.collect_batch(2)
    ex.release(1)
    with pytest.raises(gdn_amd.GdnError):
        ex.release(1)
    assert pool.slots_in_use() == 1
    ex.prefill(3, [1])
    assert pool.slots_in_use() == 2
    ex.close()
    assert pool.slots_in_use() == 0
    assert pool.check() == 0


def test_executor_batched_prefill(weights):
    """gdn_exec_prefill_batch against separate prefills on a twin executor:
    bit-identical while the packed rows stay within the decode-sized projection
    path (64 rows), within the projections' rounding beyond it; then decode
    steps from the handed-off states. A batch that runs out of slots admits
    none of its new sequences."""
    import torch

    import gdn_amd
    say("gdn_exec", "batched prefill vs separate prefills")
    rng = np.random.default_rng(1203)

    def logits_rows(ex, n):
        return ex.logits()[:n].view(torch.bfloat16).float().cpu().numpy()

    for lens, exact in (([3, 20, 41], True), ([5, 40, 100, 1], False)):
        prompts = [[int(t) for t in rng.integers(0, VOCAB, L)] for L in lens]
        ids = [300 + i for i in range(len(lens))]
        _, ea = weights.executor(8, max_batch=4, max_prompt=160)
        _, eb = weights.executor(8, max_batch=4, max_prompt=160)
        ta = ea.prefill_batch(ids, prompts)
        la = logits_rows(ea, len(lens))
        for i, (sid, p) in enumerate(zip(ids, prompts)):
            tb = eb.prefill(sid, p)
            lb = logits_rows(eb, 1)[0]
            if exact:
                assert tb == ta[i] and np.array_equal(la[i], lb), (lens, i)
            else:
                assert rel_l2(la[i], lb) <= 1e-2, (lens, i)
            assert int(np.argmax(la[i])) == ta[i]
        cur = ta
        for step in range(3):
            na = ea.decode_batch(ids, cur)
            ga = logits_rows(ea, len(lens))
            nb = eb.decode_batch(ids, cur)
            gb = logits_rows(eb, len(lens))
            if exact:
                assert na == nb and np.array_equal(ga, gb), (lens, step)
            else:
                assert max(rel_l2(ga[i], gb[i]) for i in range(len(lens))) <= 1e-2, (lens, step)
            cur = na
        ea.close()
        eb.close()
    # out of slots: 3-slot pool, one sequence admitted, a batch of three new ones fails
    pool, ex = weights.executor(3, max_batch=4)
    ex.prefill(1, [1, 2])
    with pytest.raises(gdn_amd.GdnError):
        ex.prefill_batch([2, 3, 4], [[1], [2], [3]])
    assert pool.slots_in_use() == 1
    with pytest.raises(gdn_amd.GdnError):  # a sequence twice in one batch
        ex.prefill_batch([2, 2], [[1], [2]])
    t = ex.prefill_batch([1, 2], [[1, 2], [7]])  # a known sequence starts over, one new
    assert t[0] == ex.prefill(1, [1, 2]) and pool.slots_in_use() == 2
    ex.close()
    assert pool.slots_in_use() == 0
