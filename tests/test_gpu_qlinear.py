"""GPU parity of the 4-bit quantized input projection (gdn_qlinear_*) against
the oracle's quantized_matmul (qwen3_5.rs:572-586, merged at :1037-1053).

Bar: every output within half a bf16 ulp of the exact (float64) product plus
2^-20 * mag, where mag = sum_k |x_k| (|s| (128 + q) + |b|) is the size of the
terms the f32 accumulation runs over (the kernel's per-group sums of x (128+q)
and the final correction). Measured errors sit far inside the second term,
so almost every output is the correctly rounded bf16; the tests also require
at least 99% of outputs to be exactly that.
"""
import numpy as np
import pytest

from gdn_testlib import O, dev, host, quantize_w4, say

pytestmark = pytest.mark.gpu

QWEN_HIDDEN = 2048
# merged qkv|z and b|a rows of one GDN layer: q,k (2*16*128) + v (32*128), z (32*128), b, a (32 each)
QWEN_PARTS = [8192, 4096, 32, 32]


def _parts(rng, K, rows, std=0.02):
    return [quantize_w4(rng.standard_normal((n, K)) * std) for n in rows]


def _layer(K, parts):
    import gdn_amd
    return gdn_amd.QLinear(K, [(dev(w.view(np.int32)), dev(s), dev(b)) for w, s, b in parts])


def _merged(parts):
    return (np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts]),
            np.concatenate([p[2] for p in parts]))


def _check(y_gpu, y_exact, mag, y_ref, what):
    g = O.bf16_to_f32(y_gpu).astype(np.float64)
    a = np.maximum(np.abs(y_exact), np.abs(g))
    ulp = np.where(a > 0, 2.0 ** (np.floor(np.log2(np.maximum(a, 1e-300))) - 7), 0.0)
    err = np.abs(g - y_exact)
    tol = 0.5 * ulp + 2.0**-20 * mag
    worst = float(np.max(err / np.maximum(tol, 1e-300)))
    same = float(np.mean(y_gpu == y_ref))
    say(what, f"worst err/tol={worst:.3f} correctly-rounded={same:.5f}")
    assert np.all(err <= tol), (what, worst)
    assert same >= 0.99, (what, same)


def _run(gpu, M, K, rows, seed, x_pad=0, y_pad=0, x_scale=1.0):
    import torch
    rng = np.random.default_rng(seed)
    parts = _parts(rng, K, rows)
    N = sum(rows)
    x = O.f32_to_bf16((rng.standard_normal((M, K)) * x_scale).astype(np.float32))
    xb = np.zeros((M, K + x_pad), np.uint16)
    xb[:, :K] = x
    layer = _layer(K, parts)
    y = torch.full((M, N + y_pad), -1, dtype=torch.int16, device=gpu)
    layer.forward(dev(xb)[:, :K], y)
    torch.cuda.synchronize()
    yh = host(y)
    assert np.all(yh[:, N:] == 0xFFFF), "columns past N were written"
    yr, ye, mag = O.qmatmul_w4(x, *_merged(parts))
    _check(yh[:, :N], ye, mag, yr, f"qlinear M={M} K={K} rows={rows}")
    layer.close()


@pytest.mark.parametrize("M,K,rows,x_pad,y_pad", [
    (1, 512, [16], 0, 0),
    (3, 1024, [48, 16], 8, 4),
    (17, 512, [32, 32, 16], 0, 4),
    (64, QWEN_HIDDEN, QWEN_PARTS, 0, 0),       # batched decode, B = 64
    (65, 512, [128], 8, 0),                    # first multi-tile row count
    (130, QWEN_HIDDEN, [256, 64], 0, 8),
    (200, 4096, [144], 16, 4),                 # widest K, N not a tile multiple
    (40, 4096, [2048], 8, 4),                  # out_proj shape: K split in 4 slices of 1024
    (64, 2048, [1024, 16], 0, 0),              # narrow N: K split in 2 slices of 1024
])
def test_qlinear_matches_oracle(gpu, M, K, rows, x_pad, y_pad):
    say("gdn_qlinear_forward", f"M={M} K={K} rows={rows}")
    _run(gpu, M, K, rows, seed=500 + M + K, x_pad=x_pad, y_pad=y_pad)


def test_qlinear_extreme_values(gpu):
    """All-15 and all-0 nibbles, negative / zero / huge scales and biases,
    activations of +-3e4 mixed with tiny ones."""
    import torch
    say("gdn_qlinear_forward", "extremes M=40 K=1024 N=64")
    rng = np.random.default_rng(501)
    M, K, N = 40, 1024, 64
    w = rng.integers(0, 2**32, (N, K // 8), dtype=np.uint64).astype(np.uint32)
    w[0:8] = 0xFFFFFFFF
    w[8:16] = 0
    s = O.f32_to_bf16((rng.standard_normal((N, K // 64)) * 0.05).astype(np.float32))
    b = O.f32_to_bf16((rng.standard_normal((N, K // 64)) * 0.5).astype(np.float32))
    s[16:20] = O.f32_to_bf16(np.float32(-3.0e3))
    s[20:24] = 0
    b[24:28] = O.f32_to_bf16(np.float32(1.0e4))
    xf = rng.standard_normal((M, K)).astype(np.float32)
    xf[0:5] *= 3.0e4
    xf[5:10] *= 1e-6
    xf[10, :] = 0.0
    x = O.f32_to_bf16(xf)
    layer = _layer(K, [(w, s, b)])
    y = torch.empty((M, N), dtype=torch.int16, device=gpu)
    layer.forward(dev(x), y)
    torch.cuda.synchronize()
    yr, ye, mag = O.qmatmul_w4(x, w, s, b)
    _check(host(y), ye, mag, yr, "qlinear extremes")
    layer.close()


@pytest.mark.parametrize("M,K", [(1, 2048), (37, 2048), (64, 2048), (64, 512), (17, 1536),
                                 (64, 4096)])
def test_qlinear_wide_decode_columns_sampled(gpu, M, K):
    """Decode-sized call on a layer wide enough (131,088 columns) for the
    64 x 128 tile route that lm_head takes, at K = 2048 (lm_head's) and at
    the other stage counts its loop takes (K = 512, 1536; K = 4096, the
    kernel for K above 2048); the oracle checks 1,024 sampled columns
    (columns are independent: y[:, n] depends only on row n of the weights),
    the first and last included, and the padding past N stays unwritten."""
    import torch
    say("gdn_qlinear_forward", f"wide decode M={M} K={K} N=131088 (sampled columns)")
    rng = np.random.default_rng(503 + M + K)
    N = 131072 + 16
    w = rng.integers(0, 2**32, (N, K // 8), dtype=np.uint32)
    s = O.f32_to_bf16((rng.random((N, K // 64)) * 0.004 + 0.001).astype(np.float32))
    b = O.f32_to_bf16((rng.standard_normal((N, K // 64)) * 0.03).astype(np.float32))
    x = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    layer = _layer(K, [(w, s, b)])
    y = torch.full((M, N + 8), -1, dtype=torch.int16, device=gpu)
    layer.forward(dev(x), y)
    torch.cuda.synchronize()
    yh = host(y)
    assert np.all(yh[:, N:] == 0xFFFF), "columns past N were written"
    cols = np.sort(rng.choice(N, 1024, replace=False))
    cols[0], cols[-1] = 0, N - 1
    yr, ye, mag = O.qmatmul_w4(x, w[cols], s[cols], b[cols])
    _check(yh[:, cols], ye, mag, yr, f"qlinear wide M={M} sampled columns")
    layer.close()


def test_qlinear_prefill_rows_sampled(gpu):
    """Prefill-sized call (16384 tokens) on the full merged layer; the oracle
    checks 96 sampled rows (rows are independent), the rest are checked for
    determinism against a second call."""
    import torch
    say("gdn_qlinear_forward", "M=16384 K=2048 merged qwen layer (sampled rows)")
    rng = np.random.default_rng(502)
    parts = _parts(rng, QWEN_HIDDEN, QWEN_PARTS)
    M, N = 16384, sum(QWEN_PARTS)
    x = O.f32_to_bf16(rng.standard_normal((M, QWEN_HIDDEN)).astype(np.float32))
    layer = _layer(QWEN_HIDDEN, parts)
    xd = dev(x)
    y = torch.empty((M, N), dtype=torch.int16, device=gpu)
    y2 = torch.empty_like(y)
    layer.forward(xd, y)
    layer.forward(xd, y2)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    rows = np.sort(rng.choice(M, 96, replace=False))
    rows[-1] = M - 1
    yr, ye, mag = O.qmatmul_w4(x[rows], *_merged(parts))
    _check(host(y)[rows], ye, mag, yr, "qlinear M=16384 sampled")
    layer.close()


def test_qlinear_output_feeds_gated_decode_in_place(gpu):
    """Hidden states -> merged q|k|v|z|b|a projection -> gdn_decode_gated reading
    qkvz and ab as column slices of the one output (no copies), against the
    oracle fed the same projection bits."""
    import torch

    import gdn_amd
    from gdn_testlib import gen_layer_params, gen_states
    say("qlinear -> gdn_decode_gated", "B=8 Hk=16 Hv=32")
    rng = np.random.default_rng(503)
    Hk, Hv, Dv, B = 16, 32, 128, 8
    D = 2 * Hk * 128 + Hv * Dv
    parts = _parts(rng, QWEN_HIDDEN, QWEN_PARTS)
    layer = _layer(QWEN_HIDDEN, parts)
    N = layer.N
    assert N == D + Hv * Dv + 2 * Hv
    h = O.f32_to_bf16(rng.standard_normal((B, QWEN_HIDDEN)).astype(np.float32))
    proj = torch.empty((B, N), dtype=torch.int16, device=gpu)
    layer.forward(dev(h), proj)
    p = gen_layer_params(rng, Hk, Hv)
    st, cs = gen_states(rng, B, Hk, Hv)
    norm_w = O.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(Dv)).astype(np.float32))
    eps = 1e-6
    pool = gdn_amd.Pool(1, 16, Hk, Hv)
    slots = np.array([3, 11, 0, 7, 15, 1, 9, 4], np.int32)
    ids = dev(slots)
    pool.write(0, ids, dev(st), dev(cs))
    out = torch.empty((B, Hv, Dv), dtype=torch.int16, device=gpu)
    pool.decode_gated(0, ids, proj[:, :D + Hv * Dv], proj[:, D + Hv * Dv:], dev(p["A_log"]),
                      dev(p["dt_bias"]), dev(p["conv_w"]), dev(norm_w), eps, out)
    torch.cuda.synchronize()
    ph = host(proj)
    yr_, ye, mag = O.qmatmul_w4(h, *_merged(parts))
    _check(ph, ye, mag, yr_, "qlinear merged B=8")
    qkv, z, ab = ph[:, :D], ph[:, D:D + Hv * Dv], ph[:, D + Hv * Dv:]
    y_ref, _, _ = O.decode(cs, st, qkv, ab, p["A_log"], p["dt_bias"], p["conv_w"], Hk, Hv)
    out_ref = O.norm_gate(y_ref, z.reshape(B, Hv, Dv), norm_w, eps)
    d = np.max(np.abs(O.bf16_to_f32(host(out)) - O.bf16_to_f32(out_ref)))
    say("decode_gated on projection slices |d out|", d)
    assert d <= 2e-2
    assert pool.check() == 0
    pool.close()
    layer.close()


def test_qlinear_argument_checks(gpu):
    import torch

    import gdn_amd
    rng = np.random.default_rng(504)
    layer = _layer(512, _parts(rng, 512, [32]))
    x = torch.zeros((4, 520), dtype=torch.int16, device=gpu)
    y = torch.zeros((4, 32), dtype=torch.int16, device=gpu)
    with pytest.raises(gdn_amd.GdnError):
        layer.forward(x[:, 4:516], y)      # misaligned rows
    with pytest.raises(ValueError):
        layer.forward(x[:, :500], y)       # narrower than K
    layer.forward(x[:0, :512], y[:0])      # M = 0 is a no-op
    layer.close()
