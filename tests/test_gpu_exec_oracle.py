"""GPU parity of the executor (gdn_exec_*) against the oracle's forward of
the same decoder stack (O.StackForward: embedding, per layer rms-norm + mixer
+ residual, final norm, lm_head; qwen3_5.rs:723-743,826-880), composed from
the oracle's pinned pieces. Every call's logits are compared (relative L2),
and every greedy token where the oracle's top-two margin is clear of the
logits' error. The stack is small: hidden 512, two GatedDeltaNet layers
(8 key / 16 value heads), then, in the hybrid form, one attention layer (8
query / 2 kv heads of 256); vocabulary 2048, random 4-bit weights; three sequences with ragged
prompts (a packed two-prompt prefill and a single one), then decode steps at
B = 3 fed the executor's own tokens."""
import numpy as np
import pytest

from gdn_testlib import O, DV, conv_dim, dev, quantize_w4, say

pytestmark = pytest.mark.gpu

HK, HV, HIDDEN, VOCAB = 8, 16, 512, 2048
HQ, HKV, THETA, ROT, EPS = 8, 2, 1.0e7, 64, 1e-6
LOGIT_TOL = 2e-2


def _bfw(rng, n, s=0.1):
    return O.f32_to_bf16((1 + s * rng.standard_normal(n)).astype(np.float32))


@pytest.fixture(scope="module", params=["hybrid", "gdn_only"])
def stack(gpu, request):
    import gdn_amd
    hybrid = request.param == "hybrid"
    rng = np.random.default_rng(1500)
    D = conv_dim(HK, HV)
    host_layers, gdn_dev = [], []
    for _ in range(2):
        in_parts = [quantize_w4(rng.standard_normal((n, HIDDEN)) * 0.05)
                    for n in (D, HV * DV, HV, HV)]
        out = quantize_w4(rng.standard_normal((HIDDEN, HV * DV)) * 0.03)
        L = dict(in_parts=in_parts, out=out,
                 A_log=rng.uniform(0.0, np.log(16.0), HV).astype(np.float32),
                 dt_bias=(rng.standard_normal(HV) * 0.1).astype(np.float32),
                 conv_w=O.f32_to_bf16((rng.standard_normal((D, 4)) * 0.25).astype(np.float32)),
                 norm_w=_bfw(rng, DV), in_norm=_bfw(rng, HIDDEN))
        host_layers.append(L)
    nqkv = HQ * 512 + 2 * HKV * 256
    attn = dict(qkv=quantize_w4(rng.standard_normal((nqkv, HIDDEN)) * 0.05),
                o=quantize_w4(rng.standard_normal((HIDDEN, HQ * 256)) * 0.03),
                qn=_bfw(rng, 256), kn=_bfw(rng, 256), in_norm=_bfw(rng, HIDDEN))
    if hybrid:
        host_layers.append(attn)
    final_norm = _bfw(rng, HIDDEN)
    embed = O.f32_to_bf16(rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32))
    head = quantize_w4(rng.standard_normal((VOCAB, HIDDEN)) * 0.05)

    def ql(K_, parts):
        return gdn_amd.QLinear(K_, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in parts])

    pool = gdn_amd.Pool(2, 4, HK, HV)
    layers = [gdn_amd.Layer(pool, i, ql(HIDDEN, L["in_parts"]), ql(HV * DV, [L["out"]]),
                            dev(L["A_log"]), dev(L["dt_bias"]), dev(L["conv_w"]),
                            dev(L["norm_w"]), EPS) for i, L in enumerate(host_layers[:2])]
    kv, attn_dev = None, []
    if hybrid:
        kv = gdn_amd.KVCache(1, 4, 32, 8, HQ, HKV, max_step_tokens=256)
        attn_dev = [(2, ql(HIDDEN, [attn["qkv"]]), ql(HQ * 256, [attn["o"]]), dev(attn["qn"]),
                     dev(attn["kn"]))]
    ex = gdn_amd.Executor(pool, layers, [dev(L["in_norm"]) for L in host_layers],
                          dev(final_norm), dev(embed), ql(HIDDEN, [head]), EPS, 4, 256,
                          attn_layers=attn_dev, kv=kv, rope_theta=THETA, rotary_dim=ROT)
    orc = O.StackForward(host_layers, final_norm, embed, head, EPS, HK, HV, Hq=HQ, Hkv=HKV,
                         theta=THETA, rot_dim=ROT)
    yield ex, orc, pool
    ex.close()


def _check(ex_logits, ex_tokens, oracle_rows, tag, worst):
    """Compare one call: logits by relative L2 per row, tokens where clear."""
    got = O.bf16_to_f32(ex_logits).astype(np.float64)
    checked = 0
    for i, (yb, ye) in enumerate(oracle_rows):
        err = float(np.linalg.norm(got[i] - ye) / np.linalg.norm(ye))
        worst[0] = max(worst[0], err)
        assert err <= LOGIT_TOL, (tag, i, err)
        top2 = np.sort(ye)[-2:]
        margin = top2[1] - top2[0]
        if margin > 4 * float(np.max(np.abs(got[i] - ye))):
            assert ex_tokens[i] == int(np.argmax(ye)), (tag, i)
            checked += 1
    return checked


def test_executor_matches_oracle_stack_forward(stack):
    ex, orc, pool = stack
    say("gdn_exec vs oracle stack", f"hidden 512, {len(orc.layers)} layers, 3 ragged sequences")
    rng = np.random.default_rng(1501)
    prompts = {1: rng.integers(0, VOCAB, 5), 2: rng.integers(0, VOCAB, 70),
               3: rng.integers(0, VOCAB, 130)}
    prompts = {k: [int(t) for t in v] for k, v in prompts.items()}
    worst, checked = [0.0], 0
    # packed prefill of two prompts, then a single prefill
    first = ex.prefill_batch([1, 2], [prompts[1], prompts[2]])
    lg = ex.logits().cpu().numpy().view(np.uint16)
    rows = [orc.forward(1, prompts[1], fresh=True), orc.forward(2, prompts[2], fresh=True)]
    checked += _check(lg, first, rows, "prefill_batch", worst)
    t3 = ex.prefill(3, prompts[3])
    checked += _check(ex.logits().cpu().numpy().view(np.uint16), [t3],
                      [orc.forward(3, prompts[3], fresh=True)], "prefill", worst)
    ids, toks = [1, 2, 3], first + [t3]
    for step in range(8):
        nxt = ex.decode_batch(ids, toks)
        rows = [orc.forward(s, [t]) for s, t in zip(ids, toks)]
        checked += _check(ex.logits().cpu().numpy().view(np.uint16), nxt, rows,
                          f"decode {step}", worst)
        toks = nxt
    say("worst logits relL2", worst[0], "greedy tokens compared", checked, "of", 3 + 24)
    assert checked >= 27 // 2  # most picks have a clear margin; those are compared
    assert pool.check() == 0
