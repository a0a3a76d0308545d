"""GPU parity of the attention layers' step on the paged KV cache
(gdn_kv_step + gdn_attn_forward: Qwen35Attention::forward_with_cache,
qwen3_5.rs:377-455) against the oracle's per-sequence restatement.

Bars: gated outputs within 2e-2 (absolute below 1, relative above) and 1e-2
relative L2 of the oracle (float32 softmax and accumulation against float64);
cached values bit-exact; cached keys (norm and RoPE in float32) within one
bf16 ulp of the key plus one of its RoPE pair's magnitude. A token's work
reads only its own sequence and its keys are cut into partials at fixed
points, so a batched step equals the same sequences stepped alone bit for bit
-- the property the reference's padded, unmasked, single-offset batching
(mlx_executor.rs:57-88, qwen3_5.rs:410,443-447) lacks -- and a prompt
processed in one step equals the same tokens spread over several.
"""
import numpy as np
import pytest

from gdn_testlib import O, dev, host, rel_l2, say

pytestmark = pytest.mark.gpu

HD, EPS, THETA, ROT = 256, 1e-6, 1.0e7, 64


class _Seqs:
    """Random q/k/v rows per sequence, the oracle's caches per layer."""

    def __init__(self, rng, Hq, Hkv, layers):
        self.rng, self.Hq, self.Hkv, self.layers = rng, Hq, Hkv, layers
        self.w = [(O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)),
                   O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)))
                  for _ in range(layers)]
        self.cache = {}

    def rows(self, n):
        r = self.rng
        q = O.f32_to_bf16(r.standard_normal((n, self.Hq * 2 * HD)).astype(np.float32))
        k = O.f32_to_bf16(r.standard_normal((n, self.Hkv * HD)).astype(np.float32))
        v = O.f32_to_bf16(r.standard_normal((n, self.Hkv * HD)).astype(np.float32))
        return q, k, v

    def oracle(self, layer, slot, q, k, v):
        empty = np.zeros((self.Hkv, 0, HD), np.uint16)
        ck, cv = self.cache.get((layer, slot), (empty, empty))
        out, ck, cv = O.attention_step(q, k, v, *self.w[layer], EPS, THETA, ROT, ck, cv, self.Hq,
                                       self.Hkv)
        self.cache[(layer, slot)] = (ck, cv)
        return out


def _run_step(kv, seqs, slots, ntok, gpu, check=True, label=""):
    """One planned step over `slots` (ntok rows each) through every layer;
    returns the GPU outputs per layer and checks them against the oracle."""
    import torch
    T = sum(ntok)
    kv.step(slots, ntok)
    q, k, v = seqs.rows(T)
    qd, kd, vd = dev(q), dev(k), dev(v)
    outs = []
    for layer in range(seqs.layers):
        out = torch.empty((T, seqs.Hq * HD), dtype=torch.int16, device=gpu)
        kv.forward(layer, qd, kd, vd, dev(seqs.w[layer][0]), dev(seqs.w[layer][1]), EPS, THETA,
                   ROT, out)
        outs.append(host(out))
    torch.cuda.synchronize()
    if check:
        worst_abs, worst_rel = 0.0, 0.0
        for layer in range(seqs.layers):
            r0 = 0
            for s, n in zip(slots, ntok):
                ref = seqs.oracle(layer, s, q[r0:r0 + n], k[r0:r0 + n], v[r0:r0 + n])
                g = O.bf16_to_f32(outs[layer][r0:r0 + n])
                rf = O.bf16_to_f32(ref)
                worst_abs = max(worst_abs, float(np.max(np.abs(g - rf) / np.maximum(1.0, np.abs(rf)))))
                worst_rel = max(worst_rel, rel_l2(g, rf))
                r0 += n
        say(label, f"|d out| {worst_abs:.2e} relL2 {worst_rel:.2e}")
        assert worst_abs <= 2e-2 and worst_rel <= 1e-2, (label, worst_abs, worst_rel)
    return outs


def _ulp(x):
    return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 1e-30))) - 7)


def _key_tolerance(ck):
    """Per-element bound on |GPU key - oracle key| for cached keys ck (bf16
    bits [Hkv, L, 256]): one bf16 ulp of the element for its final rounding
    plus one ulp of the RoPE pair's magnitude for the float32 norm scale,
    angle and rotation (a pair (i, i + ROT/2) keeps its length under the turn,
    so a small rotated value can carry the error of its large partner). Past
    ROT the pair is the element itself."""
    b = O.bf16_to_f32(ck).astype(np.float64)
    mag = np.abs(b)
    h = ROT // 2
    pair = np.sqrt(b[..., :h] ** 2 + b[..., h:ROT] ** 2)
    mag[..., :h] = pair
    mag[..., h:ROT] = pair
    return _ulp(b) + _ulp(mag)


def _check_cache(kv, seqs, slots, gpu):
    for layer in range(seqs.layers):
        for s in slots:
            kg, vg = kv.read(layer, s)
            ck, cv = seqs.cache[(layer, s)]
            assert kv.length(s) == ck.shape[1]
            assert np.array_equal(host(vg), cv)
            a, b = O.bf16_to_f32(host(kg)).astype(np.float64), O.bf16_to_f32(ck).astype(np.float64)
            err = np.abs(a - b) / _key_tolerance(ck)
            say("cached keys", f"layer {layer} slot {s}: worst |d| / bound {err.max():.2f}")
            assert np.all(err <= 1.0), (layer, s)


@pytest.mark.parametrize("Hq,Hkv", [(16, 2), (8, 2)])
def test_attention_prefill_then_decode_matches_oracle(gpu, Hq, Hkv):
    """Prompts of 1, 63, 64 and 130 tokens packed in one step, three decode
    steps of all four, then a step mixing a new 5-token prompt with decodes."""
    import gdn_amd
    say("gdn_attn_forward", f"Hq={Hq} Hkv={Hkv}")
    rng = np.random.default_rng(1400 + Hq)
    kv = gdn_amd.KVCache(2, 8, 64, 8, Hq, Hkv, max_step_tokens=512)
    seqs = _Seqs(rng, Hq, Hkv, 2)
    slots = [5, 0, 7, 2]
    _run_step(kv, seqs, slots, [1, 63, 64, 130], gpu, label="prefill step")
    for step in range(3):
        _run_step(kv, seqs, slots, [1, 1, 1, 1], gpu, label=f"decode step {step}")
    _run_step(kv, seqs, [0, 3, 2], [1, 5, 1], gpu, label="mixed step")
    _check_cache(kv, seqs, slots + [3], gpu)
    assert kv.free_pages() == 64 - (1 + 2 + 2 + 3 + 1)
    kv.close()


def test_attention_batched_step_equals_sequences_alone(gpu):
    """Three sequences of different lengths stepped together and, on a twin
    cache, each alone: outputs and caches bit-identical."""
    import torch

    import gdn_amd
    say("gdn_attn_forward", "batched vs alone")
    rng = np.random.default_rng(1410)
    Hq, Hkv = 16, 2
    ka, kb = (gdn_amd.KVCache(1, 4, 32, 8, Hq, Hkv, max_step_tokens=256) for _ in range(2))
    w = (dev(O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))),
         dev(O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))))
    slots = [1, 3, 0]
    for ntok in ([20, 3, 90], [1, 1, 1], [2, 1, 1]):
        T = sum(ntok)
        q = dev(O.f32_to_bf16(rng.standard_normal((T, Hq * 2 * HD)).astype(np.float32)))
        k = dev(O.f32_to_bf16(rng.standard_normal((T, Hkv * HD)).astype(np.float32)))
        v = dev(O.f32_to_bf16(rng.standard_normal((T, Hkv * HD)).astype(np.float32)))
        oa = torch.empty((T, Hq * HD), dtype=torch.int16, device=gpu)
        ka.step(slots, ntok)
        ka.forward(0, q, k, v, *w, EPS, THETA, ROT, oa)
        ob = torch.empty_like(oa)
        r0 = 0
        for s, n in zip(slots, ntok):
            kb.step([s], [n])
            kb.forward(0, q[r0:r0 + n], k[r0:r0 + n], v[r0:r0 + n], *w, EPS, THETA, ROT,
                       ob[r0:r0 + n])
            r0 += n
        torch.cuda.synchronize()
        assert torch.equal(oa, ob), ntok
    for s in slots:
        for x, y in zip(ka.read(0, s), kb.read(0, s)):
            assert torch.equal(x, y)
    ka.close()
    kb.close()


def test_attention_prompt_split_over_steps_is_bit_identical(gpu):
    """A 600-token prompt in one step against the same rows in steps of 1, 5,
    331 and 263 tokens (other token groupings, other chunk owners, other
    step sizes), then two decode steps: outputs and caches bit-identical."""
    import torch

    import gdn_amd
    say("gdn_attn_forward", "prompt at once vs split over steps")
    rng = np.random.default_rng(1415)
    Hq, Hkv, n = 16, 2, 600
    ka, kb = (gdn_amd.KVCache(1, 2, 32, 16, Hq, Hkv, max_step_tokens=n) for _ in range(2))
    w = (dev(O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))),
         dev(O.f32_to_bf16((1 + 0.1 * rng.standard_normal(HD)).astype(np.float32))))
    q = dev(O.f32_to_bf16(rng.standard_normal((n + 2, Hq * 2 * HD)).astype(np.float32)))
    k = dev(O.f32_to_bf16(rng.standard_normal((n + 2, Hkv * HD)).astype(np.float32)))
    v = dev(O.f32_to_bf16(rng.standard_normal((n + 2, Hkv * HD)).astype(np.float32)))
    oa = torch.empty((n + 2, Hq * HD), dtype=torch.int16, device=gpu)
    ob = torch.empty_like(oa)
    ka.step([1], [n])
    ka.forward(0, q[:n], k[:n], v[:n], *w, EPS, THETA, ROT, oa[:n])
    r0 = 0
    for m in (1, 5, 331, 263):
        kb.step([1], [m])
        kb.forward(0, q[r0:r0 + m], k[r0:r0 + m], v[r0:r0 + m], *w, EPS, THETA, ROT, ob[r0:r0 + m])
        r0 += m
    for cache, out in ((ka, oa), (kb, ob)):
        for t in (n, n + 1):
            cache.step([1], [1])
            cache.forward(0, q[t:t + 1], k[t:t + 1], v[t:t + 1], *w, EPS, THETA, ROT, out[t:t + 1])
    torch.cuda.synchronize()
    diff = int((oa != ob).sum())
    say("prompt at once vs split", f"{diff} of {oa.numel()} outputs differ")
    assert diff == 0
    for x, y in zip(ka.read(0, 1), kb.read(0, 1)):
        assert torch.equal(x, y)
    ka.close()
    kb.close()


def test_attention_long_context_splits(gpu):
    """A 2,500-token context (three 1,024-key splits) built by prefill steps of
    1,000 and 1,500 tokens, then two decode steps, against the oracle."""
    import gdn_amd
    say("gdn_attn_forward", "long context, 3 splits")
    rng = np.random.default_rng(1420)
    Hq, Hkv = 16, 2
    kv = gdn_amd.KVCache(1, 2, 64, 48, Hq, Hkv, max_step_tokens=1500)
    seqs = _Seqs(rng, Hq, Hkv, 1)
    _run_step(kv, seqs, [1], [1000], gpu, check=False)
    _run_step(kv, seqs, [1], [1500], gpu, check=False)
    # the decode steps are checked against the oracle continuing from the
    # GPU's cache (keys within one ulp of the oracle's, values exact), which
    # isolates the split / combine path from the prefill's rounding
    kg, vg = kv.read(0, 1)
    seqs.cache[(0, 1)] = (host(kg), host(vg))
    for step in range(2):
        _run_step(kv, seqs, [1], [1], gpu, label=f"decode at {kv.length(1)} keys")
    assert kv.length(1) == 2502
    kv.close()


@pytest.mark.parametrize("workers", [1, 3])
def test_attention_few_workers(gpu, workers):
    """All of a step's key blocks on one or three workers: pieces run over
    many segments and past 64 pages (the page-id reload), then a mixed step
    of a 40-token prompt and a decode, against the oracle."""
    import gdn_amd
    say("gdn_attn_forward", f"max_workers={workers}")
    rng = np.random.default_rng(1430 + workers)
    Hq, Hkv = 16, 2
    kv = gdn_amd.KVCache(1, 2, 96, 96, Hq, Hkv, max_step_tokens=2500, max_workers=workers)
    seqs = _Seqs(rng, Hq, Hkv, 1)
    _run_step(kv, seqs, [0], [2500], gpu, check=False)
    _run_step(kv, seqs, [0], [2500], gpu, check=False)
    kg, vg = kv.read(0, 0)
    seqs.cache[(0, 0)] = (host(kg), host(vg))
    _run_step(kv, seqs, [0], [1], gpu, label=f"decode at {kv.length(0)} keys")
    _run_step(kv, seqs, [1, 0], [40, 1], gpu, label="40-token prompt + decode")
    _check_cache(kv, seqs, [1], gpu)
    kv.close()


def test_kv_pages_and_errors(gpu):
    import torch

    import gdn_amd
    kv = gdn_amd.KVCache(1, 3, 4, 2, 16, 2, max_step_tokens=200)
    q = torch.zeros((1, 16 * 2 * HD), dtype=torch.int16, device=gpu)
    k = torch.zeros((1, 2 * HD), dtype=torch.int16, device=gpu)
    w = torch.zeros(HD, dtype=torch.int16, device=gpu)
    out = torch.empty((1, 16 * HD), dtype=torch.int16, device=gpu)
    with pytest.raises(gdn_amd.GdnError):  # nothing planned yet
        kv.forward(0, q, k, k, w, w, EPS, THETA, ROT, out)
    kv.step([0], [100])                     # two pages
    assert kv.free_pages() == 2 and kv.length(0) == 100
    with pytest.raises(gdn_amd.GdnError):  # 129 tokens > 2 pages per slot
        kv.step([0], [29])
    with pytest.raises(gdn_amd.GdnError):  # a slot twice
        kv.step([1, 1], [1, 1])
    with pytest.raises(gdn_amd.GdnError):  # more tokens than one step holds
        kv.step([1], [201])
    kv.step([1], [64])
    with pytest.raises(gdn_amd.GdnError):  # out of pages: nothing changes
        kv.step([2, 1], [64, 1])
    assert kv.free_pages() == 1 and kv.length(2) == 0 and kv.length(1) == 64
    kv.release(0)
    assert kv.free_pages() == 3 and kv.length(0) == 0
    kv.step([2, 1], [64, 1])
    assert kv.free_pages() == 1
    kv.close()
