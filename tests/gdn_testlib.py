"""Shared test helpers: seeded input generators and an independent float64
NumPy restatement of the GatedDeltaNet step in the [Dk, Dv] state layout.

The restatement here is written from the mathematics of the gated delta rule
(per token: S <- g S; d = beta (v - S^T k); S <- S + k d^T; o = S^T q, with S
indexed [dk, dv]) and of the chunked WY form, not from the oracle's C code, so
that a transposed operand, a dropped term or a wrong index in either one shows
up as a mismatch between the two.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "qwen-mlx_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import oracle as O  # noqa: E402

DK = DV = 128
K = 4


def conv_dim(Hk, Hv, Dk=DK, Dv=DV):
    return 2 * Hk * Dk + Hv * Dv


# ------------------------------------------------------------ generators --

def l2norm_rows(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def gen_recurrent_inputs(rng, B, T, Hk, Hv, Dk=DK, Dv=DV, state_std=0.01):
    """Recurrence-level inputs drawn as the single-layer decode workload: q, k
    ~N(0,1) L2-normalised per head (q also x 1/sqrt(Dk)), v ~N(0,1), all bf16;
    a, b bf16 ~N(0,1); A_log ~U(0, ln 16); dt_bias ~N(0, 0.1); g and beta from
    the gate formulas; state f32 ~N(0, state_std)."""
    q = l2norm_rows(rng.standard_normal((B, T, Hk, Dk))) / np.sqrt(Dk)
    k = l2norm_rows(rng.standard_normal((B, T, Hk, Dk)))
    v = rng.standard_normal((B, T, Hv, Dv))
    ab = O.f32_to_bf16(rng.standard_normal((B, T, 2 * Hv)).astype(np.float32))
    A_log = rng.uniform(0.0, np.log(16.0), Hv).astype(np.float32)
    dt_bias = (rng.standard_normal(Hv) * 0.1).astype(np.float32)
    beta, g = O.beta_g(ab, A_log, dt_bias)
    state = (rng.standard_normal((B, Hv, Dv, Dk)) * state_std).astype(np.float32)
    return dict(q=O.f32_to_bf16(q.astype(np.float32)), k=O.f32_to_bf16(k.astype(np.float32)),
                v=O.f32_to_bf16(v.astype(np.float32)), g=g, beta=beta, state=state, ab=ab,
                A_log=A_log, dt_bias=dt_bias)


def gen_layer_params(rng, Hk, Hv, Dk=DK, Dv=DV, w_std=0.25):
    """Per-layer constants: A_log ~U(0, ln 16), dt_bias ~N(0,0.1) f32, depthwise
    conv weight [D, K] bf16 ~N(0, w_std)."""
    D = conv_dim(Hk, Hv, Dk, Dv)
    A_log = rng.uniform(0.0, np.log(16.0), Hv).astype(np.float32)
    dt_bias = (rng.standard_normal(Hv) * 0.1).astype(np.float32)
    conv_w = O.f32_to_bf16((rng.standard_normal((D, K)) * w_std).astype(np.float32))
    return dict(A_log=A_log, dt_bias=dt_bias, conv_w=conv_w)


def gen_tokens(rng, n, Hk, Hv, Dk=DK, Dv=DV):
    """Projection outputs for n tokens: mixed qkv [n, D] and ab [n, 2Hv], bf16 ~N(0,1)."""
    D = conv_dim(Hk, Hv, Dk, Dv)
    mixed = O.f32_to_bf16(rng.standard_normal((n, D)).astype(np.float32))
    ab = O.f32_to_bf16(rng.standard_normal((n, 2 * Hv)).astype(np.float32))
    return mixed, ab


def gen_states(rng, n, Hk, Hv, Dk=DK, Dv=DV, state_std=0.01):
    """Per-sequence states: recurrent f32 [n,Hv,Dv,Dk] ~N(0,state_std), conv
    bf16 [n,K-1,D] ~N(0,1)."""
    D = conv_dim(Hk, Hv, Dk, Dv)
    st = (rng.standard_normal((n, Hv, Dv, Dk)) * state_std).astype(np.float32)
    cs = O.f32_to_bf16(rng.standard_normal((n, K - 1, D)).astype(np.float32))
    return st, cs


# ------------------------------------------- independent f64 restatement --

def f64(x_bf16):
    return O.bf16_to_f32(x_bf16).astype(np.float64)


def np_recurrent_dkdv(q, k, v, g, beta, state_dvdk):
    """Gated delta rule, f64, state in [B,Hv,Dk,Dv] (transposed w.r.t. the pool).
    q,k [B,T,Hk,Dk], v [B,T,Hv,Dv] (float64), g/beta [B,T,Hv] (float64).
    Returns (o [B,T,Hv,Dv], state back in [B,Hv,Dv,Dk])."""
    B, T, Hk, Dk = q.shape
    Hv = v.shape[2]
    rep = Hv // Hk
    qh = np.repeat(q, rep, axis=2)  # value head h uses key head h // rep
    kh = np.repeat(k, rep, axis=2)
    S = np.swapaxes(state_dvdk.astype(np.float64), -1, -2).copy()  # [B,Hv,Dk,Dv]
    o = np.zeros(v.shape, np.float64)
    for t in range(T):
        S *= g[:, t, :, None, None]
        kv = np.einsum("bhkv,bhk->bhv", S, kh[:, t])
        d = (v[:, t] - kv) * beta[:, t, :, None]
        S += kh[:, t, :, :, None] * d[:, :, None, :]
        o[:, t] = np.einsum("bhkv,bhk->bhv", S, qh[:, t])
    return o, np.swapaxes(S, -1, -2)


def np_chunked_one_head(q, k, v, lg, beta, S0, C=64):
    """Chunked WY form of the same recurrence for ONE head, f64.
    q, k [T, Dk]; v [T, Dv]; lg [T] = log of the decay multiplier; beta [T];
    S0 [Dk, Dv]. Per chunk with cumulative log-decay G (G_i = sum_{l<=i} lg_l):
      L_ij = beta_i (k_i . k_j) exp(G_i - G_j)            (j < i)
      Tm   = (I + L)^-1
      U    = Tm (beta v),  W = Tm (beta exp(G) k)
      V'   = U - W S0
      o_i  = exp(G_i) q_i S0 + sum_{j<=i} (q_i . k_j) exp(G_i - G_j) V'_j
      S    = exp(G_C) S0 + sum_j exp(G_C - G_j) k_j V'_j^T
    Returns (o [T, Dv], S [Dk, Dv])."""
    T = q.shape[0]
    S = S0.astype(np.float64).copy()
    o = np.zeros((T, v.shape[1]))
    for c0 in range(0, T, C):
        c1 = min(T, c0 + C)
        qc, kc, vc, bc = q[c0:c1], k[c0:c1], v[c0:c1], beta[c0:c1]
        G = np.cumsum(lg[c0:c1])
        n = c1 - c0
        dec = np.exp(np.minimum(G[:, None] - G[None, :], 0.0))
        tri = np.tril(np.ones((n, n)), -1)
        L = (bc[:, None] * (kc @ kc.T)) * dec * tri
        Tm = np.linalg.inv(np.eye(n) + L)
        U = Tm @ (bc[:, None] * vc)
        W = Tm @ (bc[:, None] * np.exp(G)[:, None] * kc)
        Vp = U - W @ S
        A = (qc @ kc.T) * dec * np.tril(np.ones((n, n)))
        o[c0:c1] = (np.exp(G)[:, None] * qc) @ S + A @ Vp
        S = np.exp(G[-1]) * S + (np.exp(G[-1] - G)[:, None] * kc).T @ Vp
    return o, S


def np_conv_depthwise(padded, w):
    """Textbook depthwise causal conv: out[t,c] = sum_k padded[t+k,c] w[c,k], f64."""
    P, D = padded.shape
    Kw = w.shape[1]
    out = np.zeros((P - Kw + 1, D))
    for kk in range(Kw):
        out += padded[kk:P - Kw + 1 + kk] * w[:, kk][None, :]
    return out


def quantize_w4(wf):
    """Test-data generator: affine 4-bit quantization of float weights [N, K] in
    groups of 64 into MLX's storage format. Per group scale = (max - min) / 15
    and bias = min, both rounded to bf16; q = clip(rint((w - bias) / scale), 0,
    15); eight nibbles per uint32 with element k at bits 4*(k % 8). Returns
    (w uint32 [N, K/8], scales uint16 [N, K/64], biases uint16 [N, K/64])."""
    wf = np.asarray(wf, np.float64)
    N, Kd = wf.shape
    g = wf.reshape(N, Kd // 64, 64)
    lo, hi = g.min(-1), g.max(-1)
    s = O.f32_to_bf16(((hi - lo) / 15.0).astype(np.float32))
    b = O.f32_to_bf16(lo.astype(np.float32))
    sf = O.bf16_to_f32(s).astype(np.float64)
    bf = O.bf16_to_f32(b).astype(np.float64)
    q = np.clip(np.rint((g - bf[..., None]) / np.where(sf == 0, 1.0, sf)[..., None]), 0, 15)
    q = q.astype(np.uint32).reshape(N, Kd // 8, 8)
    w = np.bitwise_or.reduce(q << (4 * np.arange(8, dtype=np.uint32)), axis=-1).astype(np.uint32)
    return w, s, b


def unpack_w4_bytes(w):
    """Nibbles of MLX 4-bit words read byte by byte (little-endian words: byte j
    holds elements 2j (low nibble) and 2j+1 (high nibble)): uint8 [N, K]."""
    by = np.ascontiguousarray(w, "<u4").view(np.uint8).reshape(w.shape[0], -1)
    out = np.empty((w.shape[0], by.shape[1] * 2), np.uint8)
    out[:, 0::2] = by & 0xF
    out[:, 1::2] = by >> 4
    return out


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ------------------------------------------------------- torch plumbing --

def dev(a, device="cuda:0"):
    """numpy -> contiguous torch device tensor (uint16 bf16 bits travel as int16)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(device)


def host(t, bf16=False):
    """torch device tensor -> numpy (int16 -> uint16 bf16 bits when bf16)."""
    a = t.detach().cpu().numpy()
    if bf16 or a.dtype == np.int16:
        a = a.view(np.uint16)
    return a


def say(*args):
    """Progress line naming the case about to run on the GPU (flushed)."""
    print("[gpu-case]", *args, flush=True)
