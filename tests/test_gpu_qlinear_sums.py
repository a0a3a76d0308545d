"""GPU parity of the projection path the executor runs for every GDN in_proj:
the residual norm (gdn_add_rms_norm) forms each row's 64-column group sums,
split exactly into three bf16 parts, and the decode projection
(gdn_qlinear_forward_sums, qlinear_decode_kernel<8, 2, true>) takes them
instead of forming them with products of x. Shape: the merged GDN in_proj of
Qwen3.5-35B-A3B, K = 2048 -> N = 12,352 (q|k|v, z, b, a; qwen3_5.rs:572-586),
at M = 1, 37 and 64 rows.

Checks, in order:
- hn against the oracle's rms_norm_w (qwen3_5.rs:399-407): within one bf16 ulp,
  at least 99% exact;
- the group sums bit for bit: the f32 sum of each group's 64 hn values in the
  kernel's order (8 lanes of 8 values, pairwise lane tree), split as
  hi = bf16(s), mid = bf16(s - hi), lo = bf16(s - hi - mid), with
  hi + mid + lo == s exactly;
- y against the oracle's quantized_matmul at the qlinear bar (half a bf16 ulp
  of the exact product plus 2^-20 * mag, >= 99% correctly rounded), and the
  same bar for gdn_qlinear_forward on the same rows (the path that forms the
  sums itself).

The same holds for the lm_head tiles (qlinear_head_kernel<8, true>, layers at
least 131,072 columns wide), checked on sampled columns of a 131,088-column
layer at M = 1, 37 and 64.
"""
import numpy as np
import pytest

from gdn_testlib import O, dev, host, quantize_w4, say
from test_gpu_qlinear import QWEN_HIDDEN, QWEN_PARTS, _check, _layer, _merged, _parts

pytestmark = pytest.mark.gpu


def _group_sums_kernel_order(hn):
    """f32 group sums of bf16 rows hn [M, K] in add_norm_kernel's order."""
    x = O.bf16_to_f32(hn).astype(np.float32)
    M, K = x.shape
    t = x.reshape(M, K // 8, 8)  # one thread: 8 consecutive columns
    s = np.zeros((M, K // 8), np.float32)
    for e in range(4):
        s = (s + (t[:, :, 2 * e] + t[:, :, 2 * e + 1]).astype(np.float32)).astype(np.float32)
    s = s.reshape(M, K // 64, 8)
    for off in (1, 2, 4):  # lane tree: every lane adds its partner's value
        idx = np.arange(8) ^ off
        s = (s + s[:, :, idx]).astype(np.float32)
    return s[:, :, 0]


def _split3(s):
    hi = O.f32_to_bf16(s)
    r = (s - O.bf16_to_f32(hi)).astype(np.float32)
    md = O.f32_to_bf16(r)
    lo = O.f32_to_bf16((r - O.bf16_to_f32(md)).astype(np.float32))
    return hi, md, lo


@pytest.mark.parametrize("M", [1, 37, 64])
def test_norm_group_sums_projection_matches_oracle(gpu, M):
    import torch

    import gdn_amd
    K, rows, eps = QWEN_HIDDEN, QWEN_PARTS, 1e-6
    rng = np.random.default_rng(4100 + M)
    parts = _parts(rng, K, rows)
    N = sum(rows)
    h = O.f32_to_bf16((rng.standard_normal((M, K)) * 1.5).astype(np.float32))
    w = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    hd = dev(h)
    hn = torch.empty((M, K), dtype=torch.int16, device=gpu)
    gs = torch.full((3, 64, K // 64), -1, dtype=torch.int16, device=gpu)
    gdn_amd.add_rms_norm(hd, None, dev(w), eps, hn, gs)
    torch.cuda.synchronize()
    assert np.array_equal(host(hd), h), "h changed with no addend"
    hn_h = host(hn)
    # 1. the norm
    ref = O.rms_norm_w(h, w, eps)
    a = O.bf16_to_f32(hn_h).astype(np.float64)
    b = O.bf16_to_f32(ref).astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.maximum(np.abs(a), np.abs(b)), 1e-30))) - 7)
    assert np.all(np.abs(a - b) <= ulp), "hn more than one bf16 ulp from the oracle"
    same = float(np.mean(hn_h == ref))
    say(f"add_rms_norm M={M}", f"hn exact {same:.5f}")
    assert same >= 0.99
    # 2. the split group sums, bit for bit
    g = host(gs)
    s = _group_sums_kernel_order(hn_h)
    hi, md, lo = _split3(s)
    assert np.array_equal(g[0, :M], hi) and np.array_equal(g[1, :M], md) and \
        np.array_equal(g[2, :M], lo), "split group sums differ from the kernel-order f32 sums"
    recon = (O.bf16_to_f32(hi).astype(np.float64) + O.bf16_to_f32(md).astype(np.float64)
             + O.bf16_to_f32(lo).astype(np.float64))
    assert np.array_equal(recon, s.astype(np.float64)), "hi + mid + lo != the f32 sum"
    assert np.all(g[:, M:] == 0xFFFF), "rows past n were written"
    # 3. the projection with the supplied sums, and without
    layer = _layer(K, parts)
    yr, ye, mag = O.qmatmul_w4(hn_h, *_merged(parts))
    y_xs = torch.full((M, N), -1, dtype=torch.int16, device=gpu)
    layer.forward_sums(hn, gs, y_xs)
    y_pl = torch.full((M, N), -1, dtype=torch.int16, device=gpu)
    layer.forward(hn, y_pl)
    torch.cuda.synchronize()
    yx, yp = host(y_xs), host(y_pl)
    _check(yx, ye, mag, yr, f"in_proj with norm group sums M={M}")
    _check(yp, ye, mag, yr, f"in_proj forming its sums M={M}")
    say(f"M={M}", f"paths bit-identical on {float(np.mean(yx == yp)):.5f} of outputs")
    layer.close()


def test_add_rms_norm_adds_and_checks(gpu):
    """h <- bf16(h + d) before the norm, and argument checks on the host."""
    import torch

    import gdn_amd
    rng = np.random.default_rng(4200)
    M, K = 5, 512
    h = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    d = O.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    hd = dev(h)
    hn = torch.empty((M, K), dtype=torch.int16, device=gpu)
    gdn_amd.add_rms_norm(hd, dev(d), dev(w), 1e-6, hn)
    torch.cuda.synchronize()
    hsum = O.f32_to_bf16((O.bf16_to_f32(h) + O.bf16_to_f32(d)).astype(np.float32))
    assert np.array_equal(host(hd), hsum)
    same = float(np.mean(host(hn) == O.rms_norm_w(hsum, w, 1e-6)))
    assert same >= 0.99, same
    gs = torch.empty((3, 64, K // 64), dtype=torch.int16, device=gpu)
    big = torch.zeros((65, K), dtype=torch.int16, device=gpu)
    with pytest.raises(gdn_amd.GdnError):
        gdn_amd.add_rms_norm(big, None, dev(w), 1e-6, torch.empty_like(big), gs)  # n > 64 with sums
    odd = torch.zeros((2, 100), dtype=torch.int16, device=gpu)
    with pytest.raises(gdn_amd.GdnError):
        gdn_amd.add_rms_norm(odd, None, dev(w), 1e-6, torch.empty_like(odd))  # hidden % 8


@pytest.mark.parametrize("M,K", [(1, 2048), (37, 2048), (64, 2048), (5, 1024), (64, 4096)])
def test_norm_group_sums_wide_head_matches_oracle(gpu, M, K):
    """The lm_head route with the norm's group sums: 131,088 columns (over the
    131,072 threshold, the last 128-column tile part padding), K = 2048
    (lm_head's), 1024 and 4096 (the kernel for K above 2048). The oracle
    checks 1,024 sampled columns, the first and last included (y[:, n]
    depends only on row n of the weights); both paths meet the qlinear bar,
    and the padding past N stays unwritten."""
    import torch

    import gdn_amd
    N, eps = 131072 + 16, 1e-6
    rng = np.random.default_rng(4500 + M + K)
    w = rng.integers(0, 2**32, (N, K // 8), dtype=np.uint32)
    sc = O.f32_to_bf16((rng.random((N, K // 64)) * 0.004 + 0.001).astype(np.float32))
    bi = O.f32_to_bf16((rng.standard_normal((N, K // 64)) * 0.03).astype(np.float32))
    h = O.f32_to_bf16((rng.standard_normal((M, K)) * 1.5).astype(np.float32))
    nw = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    hn = torch.empty((M, K), dtype=torch.int16, device=gpu)
    gs = torch.full((3, 64, K // 64), -1, dtype=torch.int16, device=gpu)
    gdn_amd.add_rms_norm(dev(h), None, dev(nw), eps, hn, gs)
    layer = _layer(K, [(w, sc, bi)])
    y_xs = torch.full((M, N + 8), -1, dtype=torch.int16, device=gpu)
    layer.forward_sums(hn, gs, y_xs)
    y_pl = torch.full((M, N + 8), -1, dtype=torch.int16, device=gpu)
    layer.forward(hn, y_pl)
    torch.cuda.synchronize()
    yx, yp, hn_h = host(y_xs), host(y_pl), host(hn)
    assert np.all(yx[:, N:] == 0xFFFF) and np.all(yp[:, N:] == 0xFFFF), "columns past N written"
    cols = np.sort(rng.choice(N, 1024, replace=False))
    cols[0], cols[-1] = 0, N - 1
    yr, ye, mag = O.qmatmul_w4(hn_h, w[cols], sc[cols], bi[cols])
    _check(yx[:, cols], ye, mag, yr, f"lm_head tiles with norm group sums M={M}")
    _check(yp[:, cols], ye, mag, yr, f"lm_head tiles forming their sums M={M}")
    say(f"wide M={M}", f"paths bit-identical on {float(np.mean(yx[:, :N] == yp[:, :N])):.5f} of outputs")
    layer.close()
