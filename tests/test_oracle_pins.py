"""Pins the CPU oracle (oracle/gdn_oracle.c) without the reference.

The reference ships no tests or fixtures for any GDN numerics, so each oracle
function is held to something independent of its own code: a closed form,
an invariant of the recurrence, brute force on tiny inputs, or the float64
restatement in another state layout (tests/gdn_testlib.py). Each check is
chosen so that a plausible slip (swapped a/b halves, reversed conv taps, a
transposed state, a dropped delta term, a wrong GQA map) fails it.
"""
import math

import numpy as np
import pytest

from gdn_testlib import (O, DK, DV, K, conv_dim, f64, gen_recurrent_inputs, gen_layer_params,
                         gen_states, gen_tokens, np_chunked_one_head, np_conv_depthwise,
                         np_recurrent_dkdv, quantize_w4, rel_l2, unpack_w4_bytes)


# ------------------------------------------------------------------ bf16 --

def test_bf16_rounding_is_rne():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, -2.5, 0.0, -0.0, np.inf], np.float32)
    got = O.bf16_to_f32(O.f32_to_bf16(x))
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even mantissa wins (1.0)
    exp = np.array([1.0, 1.0, 1.0 + 2 ** -7, -2.5, 0.0, -0.0, np.inf], np.float32)
    assert np.array_equal(got, exp)
    assert np.signbit(got[5])
    assert np.isnan(O.bf16_to_f32(O.f32_to_bf16(np.array([np.nan], np.float32))))[0]


# ----------------------------------------------------------------- gates --

def test_beta_g_closed_form():
    rng = np.random.default_rng(1)
    Hv = 32
    ab = O.f32_to_bf16(rng.standard_normal((64, 2 * Hv)).astype(np.float32) * 3)
    A_log = rng.uniform(0, np.log(16), Hv).astype(np.float32)
    dt = (rng.standard_normal(Hv) * 0.1).astype(np.float32)
    beta, g = O.beta_g(ab, A_log, dt)
    b = f64(ab[:, :Hv])
    a = f64(ab[:, Hv:])
    beta_ref = 1.0 / (1.0 + np.exp(-b))
    sp = np.log1p(np.exp(a + dt.astype(np.float64)))
    g_ref = np.exp(-np.exp(A_log.astype(np.float64)) * sp)
    # beta: f32 sigmoid rounded to bf16 -> within one bf16 ulp of the exact value
    assert np.all(np.abs(O.bf16_to_f32(beta) - beta_ref) <= 2 ** -8 * np.abs(beta_ref) + 1e-7)
    assert np.allclose(g, g_ref, rtol=2e-5, atol=1e-30)
    # the halves are not interchangeable: b drives beta, a drives g
    beta_sw, g_sw = O.beta_g(np.concatenate([ab[:, Hv:], ab[:, :Hv]], 1), A_log, dt)
    assert not np.array_equal(beta_sw, beta) and not np.allclose(g_sw, g)


def test_beta_g_special_values():
    Hv = 4
    one = O.f32_to_bf16(np.array([0.0, 0.0, 0.0, 0.0, 0.0, 100.0, -40.0, 0.0], np.float32))
    A_log = np.array([-np.inf, 0.0, 0.0, 0.0], np.float32)
    dt = np.zeros(Hv, np.float32)
    beta, g = O.beta_g(one[None, :], A_log, dt)
    beta, g = O.bf16_to_f32(beta)[0], g[0]
    assert np.all(beta == 0.5)                     # sigmoid(0)
    # a = ab[:, Hv:] = [0, 100, -40, 0]
    assert g[0] == 1.0                             # A_log = -inf: exp(-0*sp) = 1
    assert g[1] == 0.0                             # naive softplus overflows: log(inf) -> g = 0
    assert g[2] == 1.0                             # exp(-40)+1 == 1 in f32: softplus 0 -> g = 1
    assert g[3] == pytest.approx(0.5, rel=1e-6)    # a = 0, A_log = 0: exp(-log 2) = 1/2


# ------------------------------------------------------------------ conv --

def test_conv_update_one_hot_taps_pick_window_rows():
    rng = np.random.default_rng(2)
    B, D = 3, 256
    _, cs = gen_states(rng, B, 1, 1)  # shape [B,3,conv_dim(1,1)=384]
    cs = cs[:, :, :D].copy()
    x = O.f32_to_bf16(rng.standard_normal((B, D)).astype(np.float32))
    for tap in range(K):
        w = np.zeros((D, K), np.float32)
        w[:, tap] = 1.0
        new, out = O.conv_update(cs, x, O.f32_to_bf16(w))
        window = np.concatenate([cs, x[:, None, :]], 1)   # [s0 s1 s2 x], oldest first
        expect = O.bf16_to_f32(window[:, tap])
        expect_silu = O.round_bf16(expect * O.round_bf16(1.0 / (1.0 + np.exp(-expect.astype(np.float64)))))
        assert np.array_equal(new, window[:, 1:])        # bit-exact shift
        got = O.bf16_to_f32(out)
        assert np.allclose(got, expect_silu, rtol=2 ** -7, atol=1e-6)


def test_conv_update_closed_form_random_weights():
    rng = np.random.default_rng(3)
    B, Hk, Hv = 2, 1, 2
    D = conv_dim(Hk, Hv)
    _, cs = gen_states(rng, B, Hk, Hv)
    x, _ = gen_tokens(rng, B, Hk, Hv)
    w = gen_layer_params(rng, Hk, Hv)["conv_w"]
    _, out = O.conv_update(cs, x, w)
    win = f64(np.concatenate([cs, x[:, None, :]], 1))
    pre = np.einsum("bkd,dk->bd", win, f64(w))
    ref = pre / (1 + np.exp(-pre))
    assert np.max(np.abs(O.bf16_to_f32(out) - ref)) < 0.03 * max(1.0, np.abs(ref).max())


def test_conv_prefill_matches_textbook_conv_and_repeated_updates():
    rng = np.random.default_rng(4)
    Hk, Hv = 1, 2
    D = conv_dim(Hk, Hv)
    _, cs = gen_states(rng, 1, Hk, Hv)
    cs = cs[0]
    S = 9
    x, _ = gen_tokens(rng, S, Hk, Hv)
    w = gen_layer_params(rng, Hk, Hv)["conv_w"]
    new, out = O.conv_prefill(cs, x, w)
    padded = np.concatenate([cs, x], 0)
    assert np.array_equal(new, padded[-(K - 1):])
    pre = np_conv_depthwise(f64(padded), f64(w))
    ref = pre / (1 + np.exp(-pre))
    assert np.max(np.abs(O.bf16_to_f32(out) - ref)) < 0.03 * max(1.0, np.abs(ref).max())
    # With small-integer inputs and weights every product and sum is exact, so
    # the prefill conv must equal S single-token updates bit for bit.
    xi = O.f32_to_bf16(rng.integers(-3, 4, (S, D)).astype(np.float32))
    csi = O.f32_to_bf16(rng.integers(-3, 4, (K - 1, D)).astype(np.float32))
    wi = O.f32_to_bf16(rng.integers(-2, 3, (D, K)).astype(np.float32))
    new_p, out_p = O.conv_prefill(csi, xi, wi)
    st = csi[None]
    for t in range(S):
        st, o = O.conv_update(st, xi[t:t + 1], wi)
        assert np.array_equal(o[0], out_p[t])
    assert np.array_equal(st[0], new_p)


def test_conv_prefill_short_sequence_state_mixes_old_rows():
    rng = np.random.default_rng(5)
    D = 384
    cs = O.f32_to_bf16(rng.standard_normal((K - 1, D)).astype(np.float32))
    x = O.f32_to_bf16(rng.standard_normal((1, D)).astype(np.float32))
    w = O.f32_to_bf16(rng.standard_normal((D, K)).astype(np.float32))
    new, _ = O.conv_prefill(cs, x, w)
    assert np.array_equal(new, np.concatenate([cs[1:], x], 0))


# ------------------------------------------------------------------ norm --

def test_norm_weights_are_the_baked_bf16_values():
    assert O.q_norm_weight(128) == 0.0078125
    assert O.k_norm_weight(128) == 0.08837890625


def test_rms_norm_closed_form():
    rng = np.random.default_rng(6)
    x = O.f32_to_bf16(rng.standard_normal((50, DK)).astype(np.float32) * 2)
    xk = O.rms_norm(x, O.k_norm_weight(DK), 1e-6)
    xq = O.rms_norm(x, O.q_norm_weight(DK), 1e-6)
    xf = f64(x)
    base = xf / np.sqrt((xf ** 2).sum(-1, keepdims=True) + DK * 1e-6)
    assert np.allclose(f64(xk), base * 0.08837890625 * np.sqrt(DK), rtol=2 ** -7, atol=1e-6)
    assert np.allclose(f64(xq), base / np.sqrt(DK), rtol=2 ** -7, atol=1e-8)
    # |k| is 0.99989, not 1 (the bf16 weight), |q| is 1/sqrt(128)
    assert np.allclose(np.linalg.norm(f64(xk), axis=-1), 0.08837890625 * np.sqrt(DK), rtol=5e-3)
    # tiny inputs are dominated by eps (effective 128 * 1e-6 in sum-of-squares
    # space): |k| = sqrt(ss / (ss + 1.28e-4)) * 0.99989, about 0.0995 here
    tiny = O.f32_to_bf16(np.full((1, DK), 1e-4, np.float32))
    ss = float((f64(tiny) ** 2).sum())
    expect = math.sqrt(ss / (ss + DK * 1e-6)) * 0.08837890625 * math.sqrt(DK)
    got = np.linalg.norm(f64(O.rms_norm(tiny, O.k_norm_weight(DK), 1e-6)))
    assert got == pytest.approx(expect, rel=1e-2) and got < 0.11


def test_norm_gate_closed_form_and_special_values():
    """RMSNormGated out = silu(z) * rms_norm(y, w, eps) per row of Dv."""
    rng = np.random.default_rng(16)
    rows = 40
    y = O.f32_to_bf16(rng.standard_normal((rows, DV)).astype(np.float32) * 0.3)
    z = O.f32_to_bf16(rng.standard_normal((rows, DV)).astype(np.float32))
    w = O.f32_to_bf16((1.0 + 0.2 * rng.standard_normal(DV)).astype(np.float32))
    eps = 1e-6
    out = f64(O.norm_gate(y, z, w, eps))
    yf, zf, wf = f64(y), f64(z), f64(w)
    silu = zf / (1.0 + np.exp(-zf))
    expect = silu * wf * yf / np.sqrt((yf ** 2).mean(-1, keepdims=True) + eps)
    # three bf16 roundings on the way (y*r, w*., silu, product): a few ulps
    assert np.allclose(out, expect, rtol=2 ** -6, atol=1e-6)
    # the mean, not the sum, of squares: a dropped 1/Dv would scale by sqrt(Dv)
    assert np.abs(np.linalg.norm(out, axis=-1) / np.linalg.norm(expect, axis=-1) - 1).max() < 1e-2
    # z = 0 gates everything off exactly (to +-0)
    assert not f64(O.norm_gate(y, np.zeros_like(z), w, eps)).any()
    # rows are independent: permuting rows permutes outputs
    perm = rng.permutation(rows)
    assert np.array_equal(O.norm_gate(y[perm], z[perm], w, eps), O.norm_gate(y, z, w, eps)[perm])
    # z = 16: sigmoid rounds to 1.0 in bf16 and silu(z) = 16, so out/16 is
    # exactly the (already pinned) baked-weight rms_norm with a constant w
    c = O.f32_to_bf16(np.array([0.75], np.float32))[0]
    z16 = np.full_like(z, O.f32_to_bf16(np.float32(16.0)))
    wc = np.full(DV, c, np.uint16)
    got = f64(O.norm_gate(y, z16, wc, eps)) / 16.0
    assert np.array_equal(got, f64(O.rms_norm(y, float(O.bf16_to_f32(np.array([c]))[0]), eps)))
    # eps matters for tiny y: a row of 1e-4 normalises to ~0.1, not 1
    tiny = O.f32_to_bf16(np.full((1, DV), 1e-4, np.float32))
    got = f64(O.norm_gate(tiny, z16[:1], np.full(DV, O.f32_to_bf16(np.float32(1.0)), np.uint16),
                          eps)) / 16.0
    assert got.max() == pytest.approx(1e-4 / math.sqrt(1e-8 + eps), rel=1e-2)


# ------------------------------------------------------------ recurrence --

def _brute_recurrence(q, k, v, g, beta, S):
    """Scalar loops straight from the per-row description of the kernel."""
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    S = S.astype(np.float64).copy()
    y = np.zeros((B, T, Hv, Dv))
    for b in range(B):
        for h in range(Hv):
            hk = h // (Hv // Hk)
            for dv in range(Dv):
                s = S[b, h, dv]
                for t in range(T):
                    s = s * g[b, t, h]
                    kv = sum(s[i] * k[b, t, hk, i] for i in range(Dk))
                    d = (v[b, t, h, dv] - kv) * beta[b, t, h]
                    s = s + k[b, t, hk] * d
                    y[b, t, h, dv] = sum(s[i] * q[b, t, hk, i] for i in range(Dk))
                S[b, h, dv] = s
    return y, S


def test_recurrence_matches_brute_force_tiny():
    rng = np.random.default_rng(7)
    B, T, Hk, Hv, Dk, Dv = 1, 4, 2, 4, 32, 4
    inp = gen_recurrent_inputs(rng, B, T, Hk, Hv, Dk, Dv, state_std=0.3)
    y, st = O.recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"])
    yr, sr = _brute_recurrence(f64(inp["q"]), f64(inp["k"]), f64(inp["v"]),
                               inp["g"].astype(np.float64), f64(inp["beta"]), inp["state"])
    assert rel_l2(st, sr) < 1e-6
    assert np.max(np.abs(O.bf16_to_f32(y) - yr)) <= 2 ** -8 * np.abs(yr).max() + 1e-7


def test_recurrence_matches_dkdv_restatement_and_gqa_map():
    rng = np.random.default_rng(8)
    B, T, Hk, Hv = 2, 6, 2, 4
    inp = gen_recurrent_inputs(rng, B, T, Hk, Hv, state_std=0.05)
    y, st = O.recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"])
    o, s64 = np_recurrent_dkdv(f64(inp["q"]), f64(inp["k"]), f64(inp["v"]),
                               inp["g"].astype(np.float64), f64(inp["beta"]), inp["state"])
    assert rel_l2(st, s64) < 1e-6
    assert np.max(np.abs(O.bf16_to_f32(y) - o)) <= 2 ** -8 * np.abs(o).max()
    # a transposed state or a k<->q swap is caught by the same comparison
    o_t, _ = np_recurrent_dkdv(f64(inp["q"]), f64(inp["k"]), f64(inp["v"]),
                               inp["g"].astype(np.float64), f64(inp["beta"]),
                               np.swapaxes(inp["state"], -1, -2))
    assert rel_l2(O.bf16_to_f32(y), o_t) > 1e-2
    # GQA: value heads 2j and 2j+1 read key head j (hv // 2), not hv % Hk
    q2 = inp["q"].copy()
    q2[:, :, 1] = inp["q"][:, :, 0]
    k2 = inp["k"].copy()
    k2[:, :, 1] = inp["k"][:, :, 0]
    y2, _ = O.recurrent(q2, k2, inp["v"], inp["g"], inp["beta"], inp["state"])
    assert np.array_equal(y2[:, :, :2], y[:, :, :2])     # heads 0,1 use key head 0
    assert not np.array_equal(y2[:, :, 2:], y[:, :, 2:])  # heads 2,3 use key head 1


def test_recurrence_invariants():
    rng = np.random.default_rng(9)
    B, T, Hk, Hv = 1, 3, 1, 2
    inp = gen_recurrent_inputs(rng, B, T, Hk, Hv, state_std=0.1)
    q, k, v, st0 = inp["q"], inp["k"], inp["v"], inp["state"]
    zero_beta = np.zeros_like(inp["beta"])
    one_g = np.ones_like(inp["g"])
    # (i) beta = 0: pure decay, y_t = (prod g) S0 q_t
    y, st = O.recurrent(q, k, v, inp["g"], zero_beta, st0)
    gp = np.cumprod(inp["g"][0].astype(np.float64), axis=0)      # [T, Hv]
    for t in range(T):
        for h in range(Hv):
            ref = gp[t, h] * st0[0, h].astype(np.float64) @ f64(q[0, t, 0])
            assert np.allclose(f64(y[0, t, h]), ref, rtol=2 ** -7, atol=1e-7)
    assert np.allclose(st, st0 * gp[-1][None, :, None, None], rtol=1e-5)
    # (ii) g = 1, beta = 0: state bit-identical
    _, st = O.recurrent(q, k, v, one_g, zero_beta, st0)
    assert np.array_equal(st, st0)
    # (iii) delta-rule write: g = 1, beta = 1, k = e_j  =>  S_new[:, :, j] = v
    kj = np.zeros_like(k)
    kj[..., 5] = O.f32_to_bf16(np.float32(1.0))
    one_beta = O.f32_to_bf16(np.ones(inp["beta"].shape, np.float32))
    _, st = O.recurrent(q[:, :1], kj[:, :1], v[:, :1], one_g[:, :1], one_beta[:, :1], st0)
    assert np.allclose(st[0, :, :, 5], f64(v[0, 0]), rtol=0, atol=1e-6)
    others = [i for i in range(DK) if i != 5]
    assert np.array_equal(st[0][:, :, others], st0[0][:, :, others])


def test_recurrence_batch_permutation_equivariance():
    rng = np.random.default_rng(10)
    B, T, Hk, Hv = 4, 2, 2, 4
    inp = gen_recurrent_inputs(rng, B, T, Hk, Hv)
    y, st = O.recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"])
    p = rng.permutation(B)
    yp, stp = O.recurrent(inp["q"][p], inp["k"][p], inp["v"][p], inp["g"][p], inp["beta"][p],
                          inp["state"][p])
    assert np.array_equal(yp, y[p]) and np.array_equal(stp, st[p])


def test_recurrence_f32_tracks_f64_over_256_steps():
    rng = np.random.default_rng(11)
    B, T, Hk, Hv = 1, 256, 1, 2
    inp = gen_recurrent_inputs(rng, B, T, Hk, Hv)
    y, st = O.recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"])
    y64b, y64, st64 = O.recurrent_f64(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                      inp["state"])
    assert rel_l2(st, st64) < 1e-5
    assert np.max(np.abs(O.bf16_to_f32(y) - y64)) < 2e-2


# --------------------------------------------------------- chunked form --

@pytest.mark.parametrize("T", [1, 40, 64, 130])
def test_chunked_wy_form_equals_sequential_recurrence(T):
    """The chunked algorithm the prefill kernel implements reproduces the
    token-by-token recurrence, including a partial last chunk."""
    rng = np.random.default_rng(12 + T)
    inp = gen_recurrent_inputs(rng, 1, T, 1, 1, state_std=0.05)
    q, k, v = f64(inp["q"][0, :, 0]), f64(inp["k"][0, :, 0]), f64(inp["v"][0, :, 0])
    g = inp["g"][0, :, 0].astype(np.float64)
    beta = f64(inp["beta"][0, :, 0])
    S0 = inp["state"][0, 0].astype(np.float64)          # [Dv, Dk]
    o, S = np_chunked_one_head(q, k, v, np.log(g), beta, S0.T)
    y, st = O.recurrent(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], inp["state"])
    _, y64, st64 = O.recurrent_f64(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                   inp["state"])
    assert rel_l2(S.T, st64[0, 0]) < 1e-7        # st64 is stored rounded to f32
    assert np.max(np.abs(o - y64[0, :, 0])) < 1e-9
    assert np.max(np.abs(O.bf16_to_f32(y[0, :, 0]) - o)) < 2e-2


# ------------------------------------------------------- composed layer --

def test_decode_equals_composition_of_steps():
    rng = np.random.default_rng(13)
    B, Hk, Hv = 2, 2, 4
    D = conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    st, cs = gen_states(rng, B, Hk, Hv)
    x, ab = gen_tokens(rng, B, Hk, Hv)
    y, cs2, st2 = O.decode(cs, st, x, ab, p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
    cs_ref, xc = O.conv_update(cs, x, p["conv_w"])
    q, k, v = O.split_qkv(xc, Hk, Hv, DK, DV)
    q = O.rms_norm(q, O.q_norm_weight(DK))
    k = O.rms_norm(k, O.k_norm_weight(DK))
    beta, g = O.beta_g(ab, p["A_log"], p["dt_bias"])
    yr, str_ = O.recurrent(q[:, None], k[:, None], v[:, None], g[:, None], beta[:, None], st)
    assert np.array_equal(cs2, cs_ref)
    assert np.array_equal(y, yr[:, 0]) and np.array_equal(st2, str_)
    assert D == 1024


def test_prefill_equals_token_by_token_decode_within_rounding():
    """Prefill (conv1d, f32 accumulation) vs S decode steps (bf16 products):
    same mathematics, different MLX rounding, so equal to tolerance."""
    rng = np.random.default_rng(14)
    Hk, Hv, S = 1, 2, 12
    p = gen_layer_params(rng, Hk, Hv)
    st, cs = gen_states(rng, 1, Hk, Hv)
    x, ab = gen_tokens(rng, S, Hk, Hv)
    y, cs_p, st_p = O.prefill(cs[0], st[0], x, ab, p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
    cs_d, st_d = cs, st
    ys = []
    for t in range(S):
        yt, cs_d, st_d = O.decode(cs_d, st_d, x[t:t + 1], ab[t:t + 1], p["A_log"], p["dt_bias"],
                                  p["conv_w"], Hk, Hv)
        ys.append(yt[0])
    assert np.array_equal(cs_p, cs_d[0])
    assert np.max(np.abs(O.bf16_to_f32(y) - O.bf16_to_f32(np.stack(ys)))) < 2e-2
    assert rel_l2(st_p, st_d[0]) < 2e-2


def test_stack_unstack_are_gather_scatter():
    rng = np.random.default_rng(15)
    pool = rng.standard_normal((10, 3, 4)).astype(np.float32)
    ids = np.array([7, 2, 9], np.int32)
    batched = O.stack(pool, ids)
    assert np.array_equal(batched, pool[[7, 2, 9]])
    new = pool.copy()
    O.unstack(new, ids, batched * 2)
    assert np.array_equal(new[[7, 2, 9]], pool[[7, 2, 9]] * 2)
    untouched = [i for i in range(10) if i not in (7, 2, 9)]
    assert np.array_equal(new[untouched], pool[untouched])


# ------------------------------------------------ 4-bit quantized matmul --
# quantized_matmul(x, w, scales, biases, transpose, group 64, bits 4)
# (qwen3_5.rs:572-586). MLX is not importable here; the oracle's reading of
# the MLX storage format and of the operation is pinned below by hand-built
# words, a byte-wise re-reading of the nibbles, a quantize round trip and
# brute force, and its bf16 rounding by ties built to expose double rounding.

def _bf(v):
    return int(np.ravel(O.f32_to_bf16(np.array([v], np.float32)))[0])


def test_w4_dequant_known_words_and_affine_direction():
    w = np.array([[0x76543210, 0xFEDCBA98] * 4], np.uint32)  # K = 64: one group
    s = np.array([[_bf(2.0)]], np.uint16)
    b = np.array([[_bf(-3.0)]], np.uint16)
    d = O.dequant_w4(w, s, b)
    q = np.tile(np.arange(16), 4)
    assert np.array_equal(d[0], 2.0 * q - 3.0)  # scale * q + bias, element k at bits 4*(k%8)


def test_w4_dequant_matches_bytewise_unpack_and_group_indexing():
    rng = np.random.default_rng(40)
    N, Kd = 48, 512
    w = rng.integers(0, 2**32, (N, Kd // 8), dtype=np.uint64).astype(np.uint32)
    s = O.f32_to_bf16(rng.standard_normal((N, Kd // 64)).astype(np.float32))
    b = O.f32_to_bf16(rng.standard_normal((N, Kd // 64)).astype(np.float32))
    q = unpack_w4_bytes(w).astype(np.float64)
    sf = np.repeat(O.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bf = np.repeat(O.bf16_to_f32(b).astype(np.float64), 64, axis=1)
    assert np.array_equal(O.dequant_w4(w, s, b), sf * q + bf)


def test_w4_quantize_round_trip_within_half_step():
    rng = np.random.default_rng(41)
    wf = rng.standard_normal((32, 1024)) * 0.02
    w, s, b = quantize_w4(wf)
    d = O.dequant_w4(w, s, b)
    step = np.repeat(O.bf16_to_f32(s).astype(np.float64), 64, axis=1)
    # half a step from rounding q, plus the bf16 rounding of the group minimum
    # and of the step (at most 15 steps' worth of it)
    slack = np.repeat(np.abs(O.bf16_to_f32(b)).astype(np.float64), 64, axis=1) * 2.0**-8
    assert np.all(np.abs(d - wf) <= 0.5 * step + 15 * step * 2.0**-8 + slack)


def _rne_bf16_exact(v):
    """Independent nearest-even bf16 of a float64 (frexp arithmetic is exact)."""
    import math
    if v == 0.0:
        return 0x8000 if math.copysign(1.0, v) < 0 else 0
    m, e = math.frexp(abs(v))          # v = m 2^e, m in [0.5, 1)
    t = m * 256.0                      # 8 significant bits above the point
    f = math.floor(t)
    r = t - f
    if r > 0.5 or (r == 0.5 and f % 2 == 1):
        f += 1
    mag = f * 2.0 ** (e - 8)
    return _bf(math.copysign(mag, v))


def test_qmatmul_w4_brute_force_and_rounding():
    rng = np.random.default_rng(42)
    M, N, Kd = 5, 32, 512
    x = O.f32_to_bf16(rng.standard_normal((M, Kd)).astype(np.float32))
    w, s, b = quantize_w4(rng.standard_normal((N, Kd)) * 0.05)
    y, ye, mag = O.qmatmul_w4(x, w, s, b)
    W = (np.repeat(O.bf16_to_f32(s).astype(np.float64), 64, axis=1) * unpack_w4_bytes(w)
         + np.repeat(O.bf16_to_f32(b).astype(np.float64), 64, axis=1))
    ref = O.bf16_to_f32(x).astype(np.float64) @ W.T
    assert np.allclose(ye, ref, rtol=1e-12, atol=1e-12)
    assert all(int(y.flat[i]) == _rne_bf16_exact(float(ye.flat[i])) for i in range(y.size))
    assert np.all(mag >= np.abs(ye))


def test_qmatmul_w4_ties_round_once():
    """y = 1 + 2^-8 is a bf16 tie (to even: 1.0); 1 + 2^-8 + 2^-40 lies just
    above it (1 + 2^-7). Rounding to f32 first with round-to-nearest would give
    1.0 for both."""
    Kd = 128
    words = np.zeros((1, Kd // 8), np.uint32)
    words[0, 0] = 1                                   # q[0] = 1, every other q = 0
    s = np.array([[_bf(2.0**-8), 0]], np.uint16)      # group 0: w[0] = 2^-8, rest 0
    b = np.array([[0, _bf(1.0)]], np.uint16)          # group 1: w = 0 * q + 1 = 1
    x = np.zeros((2, Kd), np.uint16)
    x[:, 0] = _bf(1.0)
    x[:, 64] = _bf(1.0)
    x[1, 65] = _bf(2.0**-40)
    y, ye, _ = O.qmatmul_w4(x, words, s, b)
    assert ye[0, 0] == 1.0 + 2.0**-8 and int(y[0, 0]) == 0x3F80
    assert ye[1, 0] == 1.0 + 2.0**-8 + 2.0**-40 and int(y[1, 0]) == 0x3F81


# ------------------------------------------------------ attention layers --

def test_f64_to_bf16_array_is_correctly_rounded():
    """The one-step vectorised rounding equals the C oracle's scalar rounding,
    including exact ties and values one f64 ulp either side of a tie."""
    rng = np.random.default_rng(70)
    base = O.bf16_to_f32(rng.integers(0x0080, 0x7F00, 4000).astype(np.uint16)).astype(np.float64)
    half = np.ldexp(1.0, np.frexp(base)[1] - 9)  # half a bf16 ulp
    xs = np.concatenate([base + half, base - half, np.nextafter(base + half, np.inf),
                         np.nextafter(base + half, 0), -(base + half),
                         rng.standard_normal(2000) * np.exp(rng.uniform(-30, 30, 2000))])
    got = O.f64_to_bf16_array(xs)
    want = np.array([O.f64_to_bf16(v) for v in xs], np.uint16)
    assert np.array_equal(got, want)


def test_rope_half_closed_forms():
    """Rotate-half RoPE: position 0 is the identity; a unit vector in dimension
    i (i < rot/2) turns into (cos a, sin a) on dimensions (i, i + rot/2) with
    a = pos * theta^(-2i/rot), its partner into (-sin a, cos a); dimensions
    past rot_dim pass through; scores depend on the position difference only."""
    hd, rot, theta = 256, 64, 1.0e7
    rng = np.random.default_rng(71)
    x = O.f32_to_bf16(rng.standard_normal(hd).astype(np.float32))
    assert np.array_equal(O.rope_half_f64(x, 0, rot, theta), O.bf16_to_f32(x).astype(np.float64))
    h = rot // 2
    for i in (0, 5, h - 1):
        for p in (1, 37, 1000):
            a = p * theta ** (-2.0 * i / rot)
            e = np.zeros(hd, np.float32)
            e[i] = 1.0
            r = O.rope_half_f64(O.f32_to_bf16(e), p, rot, theta)
            want = np.zeros(hd)
            want[i], want[i + h] = np.cos(a), np.sin(a)
            assert np.allclose(r, want, atol=1e-12), (i, p)
            e2 = np.zeros(hd, np.float32)
            e2[i + h] = 1.0
            r2 = O.rope_half_f64(O.f32_to_bf16(e2), p, rot, theta)
            want2 = np.zeros(hd)
            want2[i], want2[i + h] = -np.sin(a), np.cos(a)
            assert np.allclose(r2, want2, atol=1e-12), (i, p)
    r = O.rope_half_f64(x, 123, rot, theta)
    assert np.array_equal(r[rot:], O.bf16_to_f32(x[rot:]).astype(np.float64))
    y = O.f32_to_bf16(rng.standard_normal(hd).astype(np.float32))
    d1 = O.rope_half_f64(x, 17, rot, theta) @ O.rope_half_f64(y, 9, rot, theta)
    d2 = O.rope_half_f64(x, 517, rot, theta) @ O.rope_half_f64(y, 509, rot, theta)
    assert abs(d1 - d2) <= 1e-9 * (1 + abs(d1))
    assert np.array_equal(O.rope_half_f64(x, 99, 0, theta), O.bf16_to_f32(x).astype(np.float64))


def test_rms_norm_w_agrees_with_the_pinned_scalar_norm():
    """With a constant weight the vector-weight norm equals the pinned
    orc_rms_norm bit for bit; a constant row of 2 with eps 0 normalises to w."""
    rng = np.random.default_rng(72)
    x = O.f32_to_bf16(rng.standard_normal((40, 256)).astype(np.float32))
    for w in (1.0, 0.08837890625, 0.5):
        wv = O.f32_to_bf16(np.full(256, w, np.float32))
        assert np.array_equal(O.rms_norm_w(x, wv, 1e-6), O.rms_norm(x, w, 1e-6))
    w = O.f32_to_bf16(rng.standard_normal(256).astype(np.float32))
    two = O.f32_to_bf16(np.full((1, 256), 2.0, np.float32))
    assert np.array_equal(O.rms_norm_w(two, w, 0.0)[0], w)


def _attn_inputs(rng, S, Hq, Hkv, hd=256):
    q = O.f32_to_bf16(rng.standard_normal((S, Hq * 2 * hd)).astype(np.float32))
    k = O.f32_to_bf16(rng.standard_normal((S, Hkv * hd)).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal((S, Hkv * hd)).astype(np.float32))
    qw = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    kw = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    return q, k, v, qw, kw


def test_attention_step_closed_forms_and_causality():
    """One token with an empty cache attends to itself only: out = bf16(v *
    bf16(sigmoid(gate))) exactly. Identical keys give the mean of the values.
    A prompt processed at once equals the same tokens processed one by one
    against the growing cache (positions and causal mask line up), and later
    tokens cannot change earlier outputs. Query head h reads kv head h // G."""
    rng = np.random.default_rng(73)
    Hq, Hkv, hd, eps, theta, rot = 8, 2, 256, 1e-6, 1.0e7, 64
    q, k, v, qw, kw = _attn_inputs(rng, 1, Hq, Hkv)
    empty = np.zeros((Hkv, 0, hd), np.uint16)
    out, ck, cv = O.attention_step(q, k, v, qw, kw, eps, theta, rot, empty, empty, Hq, Hkv)
    gate = O.bf16_to_f32(q.reshape(Hq, 2, hd)[:, 1]).astype(np.float64)
    sg = O.bf16_to_f32(O.f64_to_bf16_array(1 / (1 + np.exp(-gate))))
    vf = O.bf16_to_f32(v.reshape(Hkv, hd)).astype(np.float64)
    want = O.f64_to_bf16_array(np.stack([vf[h // (Hq // Hkv)] for h in range(Hq)]) * sg)
    assert np.array_equal(out.reshape(Hq, hd), want)
    assert ck.shape == (Hkv, 1, hd) and np.array_equal(cv[:, 0], v.reshape(Hkv, hd))
    # the first token sits at position 0, where RoPE is the identity: its
    # cached key is the normed key; the next one is rotated by position 1
    assert np.array_equal(ck[:, 0], O.rms_norm_w(k.reshape(Hkv, hd), kw, eps))
    q2, k2_, v2, _, _ = _attn_inputs(rng, 1, Hq, Hkv)
    _, ck2, _ = O.attention_step(q2, k2_, v2, qw, kw, eps, theta, rot, ck, cv, Hq, Hkv)
    kn2 = O.rms_norm_w(k2_.reshape(Hkv, hd), kw, eps)
    assert np.array_equal(ck2[:, 1], O.f64_to_bf16_array(O.rope_half_f64(kn2, 1, rot, theta)))
    # identical keys: uniform weights, the output is the mean of the values
    S = 6
    q, k, v, qw, kw = _attn_inputs(rng, S, Hq, Hkv)
    same = O.f32_to_bf16(np.zeros((Hkv, 3, hd), np.float32))
    vals = O.f32_to_bf16(rng.standard_normal((Hkv, 3, hd)).astype(np.float32))
    kz = O.f32_to_bf16(np.zeros((1, Hkv * hd), np.float32))
    o1, _, _ = O.attention_step(q[:1], kz, v[:1], qw, kw, eps, theta, rot, same, vals, Hq, Hkv)
    allv = np.concatenate([O.bf16_to_f32(vals).astype(np.float64),
                           O.bf16_to_f32(v[:1].reshape(Hkv, 1, hd)).astype(np.float64)], 1)
    gate = O.bf16_to_f32(q[:1].reshape(Hq, 2, hd)[:, 1]).astype(np.float64)
    sg = O.bf16_to_f32(O.f64_to_bf16_array(1 / (1 + np.exp(-gate))))
    mean = O.bf16_to_f32(O.f64_to_bf16_array(allv.mean(1))).astype(np.float64)
    want = O.f64_to_bf16_array(np.stack([mean[h // 4] for h in range(Hq)]) * sg)
    assert np.array_equal(o1.reshape(Hq, hd), want)
    # prompt at once == token by token; later tokens do not reach earlier outputs
    ca, va = empty, empty
    outs = []
    for i in range(S):
        o, ca, va = O.attention_step(q[i:i + 1], k[i:i + 1], v[i:i + 1], qw, kw, eps, theta, rot,
                                     ca, va, Hq, Hkv)
        outs.append(o)
    ob, cb, vb = O.attention_step(q, k, v, qw, kw, eps, theta, rot, empty, empty, Hq, Hkv)
    assert np.array_equal(np.concatenate(outs), ob) and np.array_equal(ca, cb)
    k2 = k.copy()
    k2[-1] ^= 0x0100
    ob2, _, _ = O.attention_step(q, k2, v, qw, kw, eps, theta, rot, empty, empty, Hq, Hkv)
    assert np.array_equal(ob2[:-1], ob[:-1]) and not np.array_equal(ob2[-1], ob[-1])


def test_attention_step_score_scale_and_softmax():
    """Scores are q.k / sqrt(256) under a softmax: with cached keys k1 =
    q_hat / 8 (q_hat the token's normed, rotated query, bf16) and k2 = 0, and
    a zero new key (its norm is 0), the weights are e^s, 1, 1 over e^s + 2
    with s = |q_hat|^2 / 128. A scale of 1 or 1/256 fails it."""
    rng = np.random.default_rng(74)
    Hq = Hkv = 1
    hd, eps, theta, rot = 256, 1e-6, 1.0e7, 64
    q, _, v, qw, kw = _attn_inputs(rng, 1, Hq, Hkv)
    kzero = O.f32_to_bf16(np.zeros((1, hd), np.float32))
    qn = O.rms_norm_w(q.reshape(1, 2, hd)[:, 0], qw, eps)
    qhat = O.bf16_to_f32(O.f64_to_bf16_array(O.rope_half_f64(qn, 2, rot, theta))).astype(np.float64)
    k1 = O.f64_to_bf16_array(qhat / 8.0)                      # exact: a power-of-two scale
    ck = np.stack([k1[0], O.f32_to_bf16(np.zeros(hd, np.float32))])[None]  # [1, 2, hd]
    cv = O.f32_to_bf16(rng.standard_normal((1, 2, hd)).astype(np.float32))
    out, _, _ = O.attention_step(q, kzero, v, qw, kw, eps, theta, rot, ck, cv, Hq, Hkv)
    s = float(np.sum(qhat ** 2)) / 128.0
    assert 1.0 < s < 4.0                                     # weights well inside (0, 1)
    vals = np.concatenate([O.bf16_to_f32(cv[0]).astype(np.float64),
                           O.bf16_to_f32(v.reshape(1, hd)).astype(np.float64)])
    w = np.array([np.exp(s), 1.0, 1.0]) / (np.exp(s) + 2.0)
    o = O.bf16_to_f32(O.f64_to_bf16_array(w @ vals)).astype(np.float64)
    gate = O.bf16_to_f32(q.reshape(1, 2, hd)[:, 1]).astype(np.float64)
    sg = O.bf16_to_f32(O.f64_to_bf16_array(1 / (1 + np.exp(-gate))))
    assert np.array_equal(out, O.f64_to_bf16_array(o * sg))


def _tiny_stack(rng, zero_mixers=False, hidden=128, vocab=256, Hk=1, Hv=2, Hq=2, Hkv=1):
    """A two-layer stack (GatedDeltaNet, attention) at tiny sizes for the
    composition pins of O.StackForward."""
    from gdn_testlib import quantize_w4

    def q4(n, k, scale=0.05):
        wf = rng.standard_normal((n, k)) * scale
        return quantize_w4(np.zeros_like(wf) if zero_mixers else wf)

    def bfw(n, s=0.1):
        return O.f32_to_bf16((1 + s * rng.standard_normal(n)).astype(np.float32))

    D = conv_dim(Hk, Hv)
    p = gen_layer_params(rng, Hk, Hv)
    gdn = dict(in_parts=[quantize_w4(rng.standard_normal((n, hidden)) * 0.05)
                         for n in (D, Hv * DV, Hv, Hv)],
               out=q4(hidden, Hv * DV), A_log=p["A_log"], dt_bias=p["dt_bias"],
               conv_w=p["conv_w"], norm_w=bfw(DV), in_norm=bfw(hidden))
    attn = dict(qkv=quantize_w4(rng.standard_normal((Hq * 512 + 2 * Hkv * 256, hidden)) * 0.05),
                o=q4(hidden, Hq * 256), qn=bfw(256), kn=bfw(256), in_norm=bfw(hidden))
    embed = O.f32_to_bf16(rng.standard_normal((vocab, hidden)).astype(np.float32))
    head = quantize_w4(rng.standard_normal((vocab, hidden)) * 0.05)
    return O.StackForward([gdn, attn], bfw(hidden), embed, head, 1e-6, Hk, Hv, Hq=Hq, Hkv=Hkv)


def test_stack_forward_with_zero_mixers_is_head_of_embedding():
    """Mixers whose output projections are zero add nothing to the residual
    stream: the logits are lm_head(rms_norm(embed[token])) of the last token,
    whatever the prompt before it."""
    rng = np.random.default_rng(80)
    st = _tiny_stack(rng, zero_mixers=True)
    toks = [int(t) for t in rng.integers(0, 256, 9)]
    y, ye = st.forward(1, toks, fresh=True)
    hn = O.rms_norm_w(np.asarray(st.embed)[toks[-1:]], st.final_norm_w, st.eps)
    y2, ye2, _ = O.qmatmul_w4(hn, *st.head)
    assert np.array_equal(y, y2[0]) and np.array_equal(ye, ye2[0])
    y3, _ = st.forward(1, toks[:1])   # one more token on the same sequence
    hn = O.rms_norm_w(np.asarray(st.embed)[toks[:1]], st.final_norm_w, st.eps)
    assert np.array_equal(y3, O.qmatmul_w4(hn, *st.head)[0][0])


def test_stack_forward_prefill_then_decode_continues_the_sequence():
    """A prompt of n tokens followed by one decode token leaves the same
    logits as one pass over the n + 1 tokens, up to the S=1 conv's bf16
    product rounding (the reference rounds each S=1 conv product, and not the
    S>1 conv's): recurrent state, conv window, attention positions and the
    growing K/V all carry over. A decode step that restarted the sequence, or
    an attention step at position 0, fails it."""
    rng = np.random.default_rng(81)
    st = _tiny_stack(rng)
    toks = [int(t) for t in rng.integers(0, 256, 21)]
    st.forward(1, toks[:-1], fresh=True)
    _, ye_a = st.forward(1, toks[-1:])
    _, ye_b = st.forward(2, toks, fresh=True)
    _, ye_c = st.forward(3, toks[-1:], fresh=True)   # the last token alone
    scale = np.linalg.norm(ye_b)
    assert np.linalg.norm(ye_a - ye_b) / scale < 1e-2
    assert np.linalg.norm(ye_c - ye_b) / scale > 1e-1
    # the states after both routes
    ga, gb = st.seqs[1][0], st.seqs[2][0]
    assert np.array_equal(ga[0], gb[0])   # conv window: the last 3 raw inputs
    assert np.linalg.norm(ga[1] - gb[1]) / np.linalg.norm(gb[1]) < 1e-2
    assert st.seqs[1][1][0].shape == st.seqs[2][1][0].shape == (1, 21, 256)
