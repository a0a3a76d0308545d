"""The executor's decode step with the in_proj group sums taken from the
residual norm (the default: gdn_add_rms_norm -> gdn_qlinear_forward_sums)
against the same executor forming them in the projection
(GDN_EXEC_SPLIT_SUMS=0), at Qwen3.5-35B-A3B's layer width (hidden 2048, 16 key
/ 32 value heads, so the merged in_proj 2048 -> 12,352 takes the whole-K decode
tiles) with B = 48 sequences, two GDN layers, random 4-bit weights.

Both executors get the same prompts and, every step, the same tokens (those of
the default path), so their steps see identical inputs. The two in_proj paths
add the same f32 products in a different order: an output differs by one bf16
ulp where the exact value sits near a rounding boundary (3 in 100,000 outputs at
M = 64 in test_gpu_qlinear_sums.py), and such a difference runs on through the
recurrent state, out_proj and lm_head of that sequence, step after step. Bar
per step: every logit within 2 bf16 ulps of the row's largest logit of the
default path (measured: at most 1 ulp over the 5 steps, with 95-99% of the
logits bit-identical), every row within relative L2 1e-2 (measured: 4.6e-3),
and the greedy tokens equal wherever the default path's top-two margin exceeds
twice the row's largest logit difference (at least 80% of the rows)."""
import os

import numpy as np
import pytest

from gdn_testlib import O, DV, conv_dim, dev, quantize_w4, say

pytestmark = pytest.mark.gpu

HK, HV, HIDDEN, VOCAB, EPS, NL, B = 16, 32, 2048, 2048, 1e-6, 2, 48


def _bfw(rng, n, s=0.1):
    return O.f32_to_bf16((1 + s * rng.standard_normal(n)).astype(np.float32))


def _executor(W, split_sums):
    import gdn_amd

    def ql(K_, parts):
        return gdn_amd.QLinear(K_, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in parts])

    pool = gdn_amd.Pool(NL, B + 4, HK, HV)
    layers = [gdn_amd.Layer(pool, i, ql(HIDDEN, L["in_parts"]), ql(HV * DV, [L["out"]]),
                            dev(L["A_log"]), dev(L["dt_bias"]), dev(L["conv_w"]), dev(L["norm_w"]),
                            EPS) for i, L in enumerate(W["layers"])]
    old = os.environ.get("GDN_EXEC_SPLIT_SUMS")
    os.environ["GDN_EXEC_SPLIT_SUMS"] = "1" if split_sums else "0"
    try:
        ex = gdn_amd.Executor(pool, layers, [dev(L["in_norm"]) for L in W["layers"]],
                              dev(W["final_norm"]), dev(W["embed"]), ql(HIDDEN, [W["head"]]), EPS,
                              64, 1024)
    finally:
        if old is None:
            del os.environ["GDN_EXEC_SPLIT_SUMS"]
        else:
            os.environ["GDN_EXEC_SPLIT_SUMS"] = old
    return pool, ex


def test_split_sums_on_off_agree(gpu):
    rng = np.random.default_rng(4300)
    D = conv_dim(HK, HV)
    W = dict(layers=[dict(in_parts=[quantize_w4(rng.standard_normal((n, HIDDEN)) * 0.03)
                                    for n in (D, HV * DV, HV, HV)],
                          out=quantize_w4(rng.standard_normal((HIDDEN, HV * DV)) * 0.02),
                          A_log=rng.uniform(0.0, np.log(16.0), HV).astype(np.float32),
                          dt_bias=(rng.standard_normal(HV) * 0.1).astype(np.float32),
                          conv_w=O.f32_to_bf16((rng.standard_normal((D, 4)) * 0.25).astype(np.float32)),
                          norm_w=_bfw(rng, DV), in_norm=_bfw(rng, HIDDEN)) for _ in range(NL)],
             final_norm=_bfw(rng, HIDDEN),
             embed=O.f32_to_bf16(rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32)),
             head=quantize_w4(rng.standard_normal((VOCAB, HIDDEN)) * 0.05))
    pa, ea = _executor(W, True)
    pb, eb = _executor(W, False)
    try:
        seqs = list(range(1, B + 1))
        prompts = [[int(t) for t in rng.integers(0, VOCAB, int(n))] for n in rng.integers(3, 12, B)]
        ta = ea.prefill_batch(seqs, prompts)
        tb = eb.prefill_batch(seqs, prompts)
        assert ta == tb, "prefill tokens differ (the prefill path is the same in both)"
        toks = ta
        worst_ulps, worst_rel, margin_checked = 0.0, 0.0, 0
        same_by_step = []
        for step in range(5):
            na = ea.decode_batch(seqs, toks)
            la = O.bf16_to_f32(ea.logits().cpu().numpy().view(np.uint16)).astype(np.float64)[:B]
            nb = eb.decode_batch(seqs, toks)
            lb = O.bf16_to_f32(eb.logits().cpu().numpy().view(np.uint16)).astype(np.float64)[:B]
            same_by_step.append(round(float(np.mean(la == lb)), 5))
            rel = np.linalg.norm(la - lb, axis=1) / np.linalg.norm(la, axis=1)
            rowmax = np.max(np.abs(la), axis=1)
            ulp = 2.0 ** (np.floor(np.log2(rowmax)) - 7)
            dmax = np.max(np.abs(la - lb), axis=1)
            worst_ulps = max(worst_ulps, float(np.max(dmax / ulp)))
            worst_rel = max(worst_rel, float(np.max(rel)))
            checked = 0
            for i in range(B):
                top2 = np.sort(la[i])[-2:]
                if top2[1] - top2[0] > 2 * dmax[i]:
                    assert na[i] == nb[i], (step, i)
                    checked += 1
            assert checked >= 0.8 * B, (step, checked)
            margin_checked += checked
            toks = na
        say("split sums on/off", f"bit-identical logits by step {same_by_step}, worst row relL2 "
            f"{worst_rel:.2e}, worst {worst_ulps:.2f} ulps of the row max, tokens compared "
            f"{margin_checked} of {5 * B}")
        assert worst_rel <= 1e-2, worst_rel
        assert worst_ulps <= 2.0, worst_ulps
        assert pa.check() == 0 and pb.check() == 0
    finally:
        ea.close()
        eb.close()


def test_pool_closed_before_its_executor(gpu):
    """Closing a pool while an executor on it is still open destroys the
    executor first (its slots go back to the live pool); the executor's own
    close afterwards is a no-op."""
    import gdn_amd
    rng = np.random.default_rng(4400)
    D = conv_dim(HK, HV)
    W = dict(layers=[dict(in_parts=[quantize_w4(rng.standard_normal((n, HIDDEN)) * 0.03)
                                    for n in (D, HV * DV, HV, HV)],
                          out=quantize_w4(rng.standard_normal((HIDDEN, HV * DV)) * 0.02),
                          A_log=rng.uniform(0.0, np.log(16.0), HV).astype(np.float32),
                          dt_bias=(rng.standard_normal(HV) * 0.1).astype(np.float32),
                          conv_w=O.f32_to_bf16((rng.standard_normal((D, 4)) * 0.25).astype(np.float32)),
                          norm_w=_bfw(rng, DV), in_norm=_bfw(rng, HIDDEN)) for _ in range(NL)],
             final_norm=_bfw(rng, HIDDEN),
             embed=O.f32_to_bf16(rng.standard_normal((VOCAB, HIDDEN)).astype(np.float32)),
             head=quantize_w4(rng.standard_normal((VOCAB, HIDDEN)) * 0.05))
    pool, ex = _executor(W, True)
    ex.prefill_batch([1, 2], [[5, 6, 7], [8, 9]])
    assert ex.handle is not None
    pool.close()
    assert ex.handle is None and pool.handle is None
    ex.close()
