"""GPU parity of the executor against the oracle's stack forward (O.StackForward)
at Qwen3.5-35B-A3B's layer width: hidden 2048, 16 key / 32 value heads, so that
the merged in_proj (2048 -> 12,352) takes the whole-K decode projection that
reads the group sums of its rows from the residual norm (launch_add_norm's
split sums) instead of forming them. One GatedDeltaNet layer, vocabulary 2048,
random 4-bit weights; two sequences prefilled, then decode steps at B = 2 fed
the executor's own tokens. Logits by relative L2 per row; greedy tokens where
the oracle's top-two margin is clear of the logits' error."""
import numpy as np
import pytest

from gdn_testlib import O, DV, conv_dim, dev, quantize_w4, say

pytestmark = pytest.mark.gpu

HK, HV, HIDDEN, VOCAB, EPS = 16, 32, 2048, 2048, 1e-6
LOGIT_TOL = 2e-2


def _bfw(rng, n, s=0.1):
    return O.f32_to_bf16((1 + s * rng.standard_normal(n)).astype(np.float32))


def test_executor_full_width_matches_oracle(gpu):
    import gdn_amd
    rng = np.random.default_rng(1700)
    D = conv_dim(HK, HV)
    L = dict(in_parts=[quantize_w4(rng.standard_normal((n, HIDDEN)) * 0.03)
                       for n in (D, HV * DV, HV, HV)],
             out=quantize_w4(rng.standard_normal((HIDDEN, HV * DV)) * 0.02),
             A_log=rng.uniform(0.0, np.log(16.0), HV).astype(np.float32),
             dt_bias=(rng.standard_normal(HV) * 0.1).astype(np.float32),
             conv_w=O.f32_to_bf16((rng.standard_normal((D, 4)) * 0.25).astype(np.float32)),
             norm_w=_bfw(rng, DV), in_norm=_bfw(rng, HIDDEN))
    final_norm = _bfw(rng, HIDDEN)
    embed = O.f32_to_bf16(rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32))
    head = quantize_w4(rng.standard_normal((VOCAB, HIDDEN)) * 0.05)

    def ql(K_, parts):
        return gdn_amd.QLinear(K_, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in parts])

    pool = gdn_amd.Pool(1, 4, HK, HV)
    layer = gdn_amd.Layer(pool, 0, ql(HIDDEN, L["in_parts"]), ql(HV * DV, [L["out"]]),
                          dev(L["A_log"]), dev(L["dt_bias"]), dev(L["conv_w"]), dev(L["norm_w"]),
                          EPS)
    ex = gdn_amd.Executor(pool, [layer], [dev(L["in_norm"])], dev(final_norm), dev(embed),
                          ql(HIDDEN, [head]), EPS, 4, 64)
    orc = O.StackForward([L], final_norm, embed, head, EPS, HK, HV)
    say("gdn_exec vs oracle stack", "hidden 2048, 16/32 heads, 1 layer")
    prompts = {1: [int(t) for t in rng.integers(0, VOCAB, 6)],
               2: [int(t) for t in rng.integers(0, VOCAB, 11)]}
    worst, checked = 0.0, 0

    def check(tokens, rows, tag):
        nonlocal worst, checked
        got = O.bf16_to_f32(ex.logits().cpu().numpy().view(np.uint16)).astype(np.float64)
        for i, ye in enumerate(rows):
            err = float(np.linalg.norm(got[i] - ye) / np.linalg.norm(ye))
            worst = max(worst, err)
            assert err <= LOGIT_TOL, (tag, i, err)
            top2 = np.sort(ye)[-2:]
            if top2[1] - top2[0] > 4 * float(np.max(np.abs(got[i] - ye))):
                assert tokens[i] == int(np.argmax(ye)), (tag, i)
                checked += 1

    toks = ex.prefill_batch([1, 2], [prompts[1], prompts[2]])
    check(toks, [orc.forward(1, prompts[1], fresh=True)[1], orc.forward(2, prompts[2], fresh=True)[1]],
          "prefill")
    for step in range(4):
        nxt = ex.decode_batch([1, 2], toks)
        check(nxt, [orc.forward(s, [t])[1] for s, t in zip([1, 2], toks)], f"decode {step}")
        toks = nxt
    say("worst logits relL2", worst, "greedy tokens compared", checked, "of", 10)
    assert checked >= 5
    assert pool.check() == 0
    ex.close()
