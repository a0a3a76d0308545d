"""Writes the golden fixtures of tests/golden from the oracle (oracle/).

The reference ships no GDN fixtures and cannot run here (a Rust crate over
unvendored MLX/Metal), so the fixtures freeze the oracle's outputs on seeded
inputs drawn as the baseline's single-layer decode case:
  bf16 activations ~N(0,1); q/k L2-normalised per head, q x 1/sqrt(Dk) for the
  recurrence-level entry; a, b bf16 ~N(0,1); A_log f32 ~U(0, ln 16); dt_bias
  f32 ~N(0, 0.1); recurrent state f32 ~N(0, 0.01); conv state bf16 ~N(0,1);
  conv weight bf16 ~N(0, 0.25^2) (the baseline leaves it open).
Large f32 states are not stored: they are regenerated from the recorded seed
(numpy PCG64, `state_seed`) and checked against a stored checksum; outputs
too large to keep whole are stored as a fixed subsample plus f64 checksums.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from gdn_testlib import O, DK, DV, K, conv_dim, gen_layer_params, gen_recurrent_inputs, gen_tokens  # noqa: E402

SUBSAMPLE = 4096


def regen_state(seed: int, shape) -> np.ndarray:
    """Recurrent state f32 ~N(0, 0.01) from its own PCG64 stream."""
    return (np.random.default_rng(seed).standard_normal(shape) * 0.01).astype(np.float32)


def checksum(a) -> np.ndarray:
    """(sum, sum of squares, sum of |x|) in f64 over the flattened array."""
    x = np.asarray(a, np.float64).ravel()
    return np.array([x.sum(), (x * x).sum(), np.abs(x).sum()])


def sub_index(n: int, seed: int) -> np.ndarray:
    return np.sort(np.random.default_rng(seed).choice(n, size=min(SUBSAMPLE, n), replace=False))


def config0_decode():
    """Fused S=1 decode, one layer, B=1, Hk=16, Hv=32. The conv state is drawn
    channel-major [D, K-1] as the baseline's single-layer case writes it; the
    pool and the oracle take time-major [K-1, D] rows (its transpose)."""
    Hk, Hv = 16, 32
    rng = np.random.default_rng(1000)
    p = gen_layer_params(rng, Hk, Hv)
    D = conv_dim(Hk, Hv)
    conv_cm = O.f32_to_bf16(rng.standard_normal((D, K - 1)).astype(np.float32))
    x, ab = gen_tokens(rng, 1, Hk, Hv)
    state_seed = 1001
    state = regen_state(state_seed, (1, Hv, DV, DK))
    y, conv_out, st_out = O.decode(np.ascontiguousarray(conv_cm.T)[None], state, x, ab,
                                   p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
    idx = sub_index(st_out.size, 1002)
    np.savez_compressed(os.path.join(HERE, "config0_decode.npz"),
                        Hk=Hk, Hv=Hv, conv_state_layout="channel-major [D, K-1]",
                        conv_state_cm=conv_cm, mixed_qkv=x, ab=ab, A_log=p["A_log"],
                        dt_bias=p["dt_bias"], conv_w=p["conv_w"], state_seed=state_seed,
                        state_checksum=checksum(state), y=y, conv_state_out=conv_out[0],
                        state_out_index=idx, state_out_sample=st_out.ravel()[idx],
                        state_out_checksum=checksum(st_out))


def config0_recurrent():
    """Recurrence-level entry (gated_delta_kernel contract), B=1, T=1."""
    Hk, Hv = 16, 32
    rng = np.random.default_rng(1100)
    r = gen_recurrent_inputs(rng, 1, 1, Hk, Hv)
    state_seed = 1101
    state = regen_state(state_seed, (1, Hv, DV, DK))
    y, st_out = O.recurrent(r["q"], r["k"], r["v"], r["g"], r["beta"], state)
    idx = sub_index(st_out.size, 1102)
    np.savez_compressed(os.path.join(HERE, "config0_recurrent.npz"),
                        Hk=Hk, Hv=Hv, q=r["q"], k=r["k"], v=r["v"], g=r["g"], beta=r["beta"],
                        state_seed=state_seed, state_checksum=checksum(state), y=y,
                        state_out_index=idx, state_out_sample=st_out.ravel()[idx],
                        state_out_checksum=checksum(st_out))


def tiny_prefill():
    """Packed varlen prefill, Hk=2, Hv=4, two sequences of 5 and 70 tokens
    (one partial chunk, one full chunk + partial), from nonzero states."""
    Hk, Hv = 2, 4
    lens = [5, 70]
    rng = np.random.default_rng(1200)
    p = gen_layer_params(rng, Hk, Hv)
    D = conv_dim(Hk, Hv)
    total = sum(lens)
    x, ab = gen_tokens(rng, total, Hk, Hv)
    conv_in = O.f32_to_bf16(rng.standard_normal((len(lens), K - 1, D)).astype(np.float32))
    state_seed = 1201
    state = regen_state(state_seed, (len(lens), Hv, DV, DK))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ys, convs, sts = [], [], []
    for i in range(len(lens)):
        a, b = cu[i], cu[i + 1]
        y, c, s = O.prefill(conv_in[i], state[i], x[a:b], ab[a:b], p["A_log"], p["dt_bias"],
                            p["conv_w"], Hk, Hv)
        ys.append(y)
        convs.append(c)
        sts.append(s)
    st_out = np.stack(sts)
    idx = sub_index(st_out.size, 1202)
    np.savez_compressed(os.path.join(HERE, "tiny_prefill.npz"),
                        Hk=Hk, Hv=Hv, cu_seqlens=cu, mixed_qkv=x, ab=ab, A_log=p["A_log"],
                        dt_bias=p["dt_bias"], conv_w=p["conv_w"], conv_state_in=conv_in,
                        state_seed=state_seed, state_checksum=checksum(state),
                        y=np.concatenate(ys), conv_state_out=np.stack(convs),
                        state_out_index=idx, state_out_sample=st_out.ravel()[idx],
                        state_out_checksum=checksum(st_out))


def tiny_slots():
    """Gather / scatter over a 6-slot pool (stack_caches / unstack_caches):
    slot ids [4, 0, 3] of a pool whose slot s holds the values s*1000 + i."""
    Hk, Hv, Dk, Dv = 1, 2, 4, 4
    D = conv_dim(Hk, Hv, Dk, Dv)
    S = 6
    pool_state = (np.arange(S)[:, None] * 1000 + np.arange(Hv * Dv * Dk)[None]).astype(
        np.float32).reshape(S, Hv, Dv, Dk)
    pool_conv = (np.arange(S)[:, None] * 100 + np.arange((K - 1) * D)[None]).astype(
        np.uint16).reshape(S, K - 1, D)
    ids = np.array([4, 0, 3], np.int32)
    np.savez_compressed(os.path.join(HERE, "tiny_slots.npz"), pool_state=pool_state,
                        pool_conv=pool_conv, slot_ids=ids,
                        stacked_state=O.stack(pool_state, ids), stacked_conv=O.stack(pool_conv, ids))


if __name__ == "__main__":
    config0_decode()
    config0_recurrent()
    tiny_prefill()
    tiny_slots()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
