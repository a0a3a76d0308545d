#!/usr/bin/env python3
"""Throughput of the GDN decode path on one MI355X through libgdn.

Workload (the reference's large ragged decode case): 30 independent GDN
layers, each with a 1024-slot state pool (2 GiB f32 recurrent state + 48 MiB
bf16 conv state per layer); B=64 active sequences at seeded random scattered
slots; every 16 steps 8 sequences retire and 8 new ones are admitted into the
freed slots with zeroed state (gdn_slots_zero over all layers). One step is
one fused gdn_decode launch per layer (conv update, q/k norm, gates,
recurrence, rolling state update), 30 launches. Shapes: Hk=16, Hv=32,
Dk=Dv=128, conv width 4 over 8192 channels. Inputs are synthetic bf16 ~N(0,1)
projection outputs resident in HBM before the timed region; weights are
random of the same shapes.

Prints one JSON line: tokens/s (B * steps / s), the dominant kernel's
achieved state-traffic bandwidth against the 8 TB/s HBM peak, and the CPU
baseline (the oracle's C restatement of the reference step, OpenMP).
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "qwen-mlx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "GDN tokens/s at B=64 decode, 30 layers; state-traffic HBM GB/s vs peak"
HK, HV, DK, DV, KW = 16, 32, 128, 128, 4
D = 2 * HK * DK + HV * DV
# Algorithmic HBM bytes per (sequence, layer, step): f32 recurrent state read
# + write, bf16 conv state read + write.
STATE_BYTES = 2 * HV * DV * DK * 4 + 2 * (KW - 1) * D * 2          # 4,292,608
ACT_BYTES = D * 2 + 2 * HV * 2 + HV * DV * 2                        # 24,704
LAYER_CONST_BYTES = D * KW * 2 + 2 * HV * 4                         # 65,792
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gdn_decode_b64_traffic.json")


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=30)
    ap.add_argument("--slots", type=int, default=1024)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--churn-every", type=int, default=16)
    ap.add_argument("--churn", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target duration of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (PMC byte-count calibration)")
    ap.add_argument("--no-placement", action="store_true",
                    help="skip the contiguous-slot timing of the same kernel")
    ap.add_argument("--placement-steps", type=int, default=16)
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the prefill sub-measurement of the default run")
    ap.add_argument("--prefill", action="store_true",
                    help="measure the chunked varlen prefill instead: 8 sequences x 16384 "
                         "tokens per layer over --layers layers")
    ap.add_argument("--prefill-seqs", type=int, default=8)
    ap.add_argument("--prefill-len", type=int, default=16384)
    ap.add_argument("--rmw-probe", action="store_true",
                    help="read-modify-write probes of the decode launch's state bytes "
                         "(lib/libgdn_probe.so) over slot placements; one JSON line")
    ap.add_argument("--placements", default="scattered,contiguous,every8,every16",
                    help="--rmw-probe placements (comma list of scattered, contiguous, "
                         "every8, every16)")
    ap.add_argument("--copy-floor", action="store_true",
                    help="only time plain device copies (torch copy_ and the streaming copy "
                         "kernel of lib/libgdn_probe.so) of the prefill qkv kernel's bytes "
                         "at --prefill-seqs x --prefill-len tokens; one JSON line")
    ap.add_argument("--rmw-ceiling", action="store_true",
                    help="only time a plain in-place multiply over 30 x 128 MiB buffers "
                         "(the decode's per-launch state bytes, read + write)")
    ap.add_argument("--gated", action="store_true",
                    help="decode through gdn_decode_gated (RMSNormGated epilogue, merged "
                         "qkvz rows) instead of gdn_decode")
    ap.add_argument("--qlinear", action="store_true",
                    help="measure the merged 4-bit input projection (gdn_qlinear_forward, "
                         "hidden 2048 -> q|k|v|z|b|a 12352) over --layers layers instead")
    ap.add_argument("--qlinear-rows", type=int, default=0,
                    help="rows (tokens) per qlinear launch; default --batch (decode)")
    ap.add_argument("--no-exec", action="store_true",
                    help="leave the executor sub-measurement out of the default line")
    ap.add_argument("--exec-steps", type=int, default=32,
                    help="steps of each executor loop in the default line's exec object")
    ap.add_argument("--no-components", action="store_true",
                    help="--exec: skip the per-kernel timing (e.g. under a kernel trace)")
    ap.add_argument("--exec", action="store_true",
                    help="the executor (gdn_exec) decode step over the GDN decoder stack: "
                         "embedding, per layer norm + in_proj + fused decode + out_proj, "
                         "final norm, lm_head, greedy pick")
    ap.add_argument("--vocab", type=int, default=248320)
    ap.add_argument("--hybrid", action="store_true",
                    help="with --exec: the 40-layer stack, an attention layer at every fourth "
                         "position (3, 7, ..., 39) between the GDN layers")
    ap.add_argument("--prompt-len", type=int, default=16,
                    help="with --exec: prompt tokens per sequence before the decode steps")
    ap.add_argument("--attn", action="store_true",
                    help="time the attention layers' decode step on the paged KV cache "
                         "(gdn_kv_step + gdn_attn_forward) instead")
    ap.add_argument("--attn-layers", type=int, default=10)
    ap.add_argument("--context", type=int, default=4096,
                    help="mean cached tokens per sequence (ragged, uniform in [C/2, 3C/2])")
    ap.add_argument("--seed", type=int, default=0)
    return ap.parse_args(argv)


def copy_calibration(mib: int):
    import torch
    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4,
                      "launches": 5}), flush=True)


# Algorithmic bytes of prefill_qkv_kernel per token (Hk = 16, Hv = 32, d = 128):
# mixed_qkv row read 16,384 + qn, kn, vc rows written 16,384 + b, a read 128 +
# beta written 64 + log decay written 128.
QKV_BYTES_PER_TOKEN = (2 * 16 + 32) * 128 * 2 * 2 + 2 * 32 * 2 + 32 * 2 + 32 * 4  # 33,088


def copy_floor(args, reps: int = 5):
    """The copy rate of the device for the prefill qkv kernel's bytes: half of
    them copied from one buffer to another (each byte read once and written
    once), by torch's copy_ (hipMemcpy device to device) and by a plain
    streaming copy kernel at several grid sizes, with and without nontemporal
    hints. A kernel that reads and writes the same bytes once takes at least
    about the best of these times. HIP events on the launch stream."""
    import ctypes

    import torch
    lib = ctypes.CDLL(os.path.join(ROOT, "qwen-mlx_amd", "lib", "libgdn_probe.so"))
    fn = lib.gdn_probe_copy
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                   ctypes.c_void_p]
    tokens = args.prefill_seqs * args.prefill_len
    moved = tokens * QKV_BYTES_PER_TOKEN           # bytes read + written
    half = (moved // 2) // 16 * 16                  # bytes copied
    src = torch.ones(half // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()

    def timed(launch):
        for _ in range(2):
            launch()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            launch()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    res = {"torch copy_ (hipMemcpy device to device)": timed(lambda: dst.copy_(src))}
    for grid in (8192, 16384, 32768, half // 16 // 1024):
        for nt in (0, 1):
            def launch(grid=grid, nt=nt):
                rc = fn(src.data_ptr(), dst.data_ptr(), half, grid, nt, stream.cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"gdn_probe_copy returned {rc}")
            res[f"copy kernel, grid {grid}{', nontemporal' if nt else ''}"] = timed(launch)
    best = min(res.values())
    out = {"copy_floor": {
        "workload": f"prefill qkv bytes of {args.prefill_seqs} x {args.prefill_len} tokens "
                    f"({QKV_BYTES_PER_TOKEN} B per token), half copied",
        "bytes_read_plus_written": 2 * half,
        "us": {k: round(v, 1) for k, v in res.items()},
        "TBps": {k: round(2 * half / v * 1e-6, 3) for k, v in res.items()},
        "best_us": round(best, 1),
        "floor_us_for_qkv_bytes": round(best * moved / (2 * half), 1)}}
    print(json.dumps(out), flush=True)
    return 0


def rmw_ceiling(layers: int = 30, mib: int = 128, reps: int = 8):
    """Reference rate of a plain streaming read-modify-write of the same bytes
    per launch as the decode kernel's state traffic (torch's in-place multiply,
    cycling `layers` buffers so nothing stays in the 256 MB memory-side cache)."""
    import torch
    bufs = [torch.zeros(mib * (1 << 20) // 4, device="cuda:0") for _ in range(layers)]
    for b in bufs:
        b.mul_(0.999)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        for b in bufs:
            b.mul_(0.999)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * layers)
    nbytes = 2 * mib * (1 << 20)
    print(json.dumps({"rmw_ceiling_us_per_launch": round(us, 2), "bytes_per_launch": nbytes,
                      "GBps": round(nbytes / us * 1e-3, 1)}), flush=True)


def placement_slots(name: str, batch: int, slots: int, seed: int):
    """Slot ids of the batch: the workload's seeded scattered set (the same
    draw as Workload), slots 0..B-1, or every 8th / 16th slot."""
    import numpy as np
    if name == "scattered":
        return [int(s) for s in np.random.default_rng(seed).choice(slots, batch, replace=False)]
    if name == "contiguous":
        return list(range(batch))
    if name.startswith("every"):
        k = int(name[5:])
        if k * (batch - 1) >= slots:
            raise ValueError(f"{name}: {batch} slots do not fit in {slots}")
        return [k * i for i in range(batch)]
    raise ValueError(f"unknown placement {name}")


def rmw_probe(args):
    """Plain read-modify-write kernels (no gated delta arithmetic) over the
    decode launch's state bytes -- B slots x 2 MiB read and written once per
    launch, `layers` pools of `slots` slots cycled so nothing stays in the
    256 MB memory-side cache -- in several access shapes and slot placements.
    They show what the memory system gives each access pattern: the decode
    kernel's own access (2 KiB-interleaved items, spaced loads), the previous
    kernel's (contiguous 128 KiB items, loads back to back), and small units
    swept in slot order or at random. Times from HIP events on the launch
    stream, us per launch."""
    import ctypes

    import numpy as np
    import torch
    lib = ctypes.CDLL(os.path.join(ROOT, "qwen-mlx_amd", "lib", "libgdn_probe.so"))
    fn = lib.gdn_probe_rmw
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p,
                   ctypes.POINTER(ctypes.c_int32), ctypes.c_int, ctypes.c_int, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L, S, B = args.layers, args.slots, args.batch
    slot_bytes = HV * DV * DK * 4
    gen = torch.Generator(device="cuda:0").manual_seed(args.seed)
    pools = []
    for _ in range(L):
        t = torch.empty(S * slot_bytes // 4, dtype=torch.float32, device="cuda:0")
        t.normal_(0.0, 0.01, generator=gen)
        pools.append(t)
    stream = torch.cuda.current_stream()
    shapes = [
        ("decode access: 2 KiB-interleaved items, XCD runs, spaced loads, 1 group/CU", 2, 0, 80 << 10, 1),
        ("decode access, loads back to back", 2, 0, 80 << 10, 0),
        ("previous decode access: contiguous 128 KiB items, item-first XCDs, 1 group/CU", 3, 0, 80 << 10, 0),
        ("4 KiB units in slot order", 0, 4096, 0, 0),
        ("16 KiB units in slot order", 0, 16384, 0, 0),
        ("4 KiB units in random order", 1, 4096, 0, 0),
    ]
    rng = np.random.default_rng(args.seed + 1)
    out = {"rmw_probe": {"layers": L, "slots": S, "batch": B,
                         "bytes_per_launch": 2 * B * slot_bytes, "us_per_launch": {}}}
    for pname in args.placements.split(","):
        ids_host = placement_slots(pname, B, S, args.seed)
        ids = torch.tensor(ids_host, dtype=torch.int32, device="cuda:0")
        hid = (ctypes.c_int32 * B)(*ids_host)
        res = {}
        for label, shape, unit, lds, gap in shapes:
            perm = None
            if shape == 1:
                perm = torch.from_numpy(rng.permutation(B * slot_bytes // unit).astype(np.int32)).cuda()

            def launch(l):
                rc = fn(pools[l].data_ptr(), S, slot_bytes, ids.data_ptr(), hid, B, shape, unit,
                        perm.data_ptr() if perm is not None else None, lds, gap,
                        stream.cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"gdn_probe_rmw returned {rc}")
            for l in range(L):
                launch(l)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 4
            e0.record()
            for _ in range(reps):
                for l in range(L):
                    launch(l)
            e1.record()
            torch.cuda.synchronize()
            res[label] = round(e0.elapsed_time(e1) * 1e3 / (reps * L), 2)
        out["rmw_probe"]["us_per_launch"][pname] = res
        print(json.dumps({pname: res}), file=sys.stderr, flush=True)
    print(json.dumps(out), flush=True)
    return 0


# Algorithmic FLOPs of the chunked (WY form, chunk C) prefill per (token,
# value head), d = Dk = Dv, the contract's count (WY factors W = T(beta K)
# and U = T(beta V) formed explicitly, C x C products counted in full):
#   12 C d + 6 d^2 + C^2/3 = 197,973 at C = 64, d = 128.
# Two further counts are reported beside it:
#   products this kernel needs, triangles at half (no explicit W, U):
#     K K^T, Q K^T 2 C^2 d; K S^T, Q S^T 4 C d^2; solve and P V' 2 C^2 d;
#     S^T update 2 C d^2 -> 4 C d + 6 d^2 = 131,072 per token
#   the sequential recurrence: 7 d^2 = 114,688 per token.
PREFILL_CHUNK = 64
PREFILL_FLOP_PER_TOKEN_HEAD = 12 * PREFILL_CHUNK * DK + 6 * DK * DK + PREFILL_CHUNK ** 2 / 3
PREFILL_FLOP_PER_TOKEN_HEAD_MIN = 4 * PREFILL_CHUNK * DK + 6 * DK * DK
PREFILL_FLOP_PER_TOKEN_HEAD_SEQ = 7 * DK * DK
PEAK_BF16_TFLOPS = 2500.0


def prefill_measure(L, n, P, seed=0, reps=1):
    """Chunked varlen prefill: n sequences of P tokens packed in one
    gdn_prefill_varlen call per layer, L layers, from zeroed slots, inputs
    resident in HBM. Returns (wall seconds, GPU seconds per pass, status
    flags); the GPU time comes from HIP events on the launch stream around
    each pass of L calls (3 launches each: qkv, conv state, chunk kernel)."""
    import torch

    import gdn_amd
    dev = torch.device("cuda:0")
    total = n * P
    pool = gdn_amd.Pool(L, n, HK, HV)
    gen = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    conv_w = [(torch.randn((D, KW), generator=gen, device=dev) * 0.25).to(bf) for _ in range(L)]
    A_log = [torch.rand(HV, generator=gen, device=dev) * math.log(16.0) for _ in range(L)]
    dt_bias = [torch.randn(HV, generator=gen, device=dev) * 0.1 for _ in range(L)]
    nsets = 2
    x = [torch.randn((total, D), generator=gen, device=dev).to(bf) for _ in range(nsets)]
    ab = [torch.randn((total, 2 * HV), generator=gen, device=dev).to(bf) for _ in range(nsets)]
    y = torch.empty((total, HV, DV), dtype=bf, device=dev)
    ids = torch.arange(n, dtype=torch.int32, device=dev)
    cu = torch.arange(n + 1, dtype=torch.int32, device=dev) * P

    def run_layers(events=None):
        pool.zero(-1, ids)
        if events:
            events[0].record()
        for l in range(L):
            pool.prefill(l, ids, cu, total, x[l % nsets], ab[l % nsets], A_log[l], dt_bias[l],
                         conv_w[l], y)
        if events:
            events[1].record()

    run_layers()  # warmup (also grows the workspace)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    torch.cuda.synchronize()
    gc.collect()
    gc.disable()  # no collector pause inside the timed region
    t0 = time.perf_counter()
    for e in ev:
        run_layers(e)
    torch.cuda.synchronize()
    elapsed = (time.perf_counter() - t0) / reps
    gc.enable()
    gpu_s = sum(a.elapsed_time(b) for a, b in ev) * 1e-3 / reps
    flags = pool.check()
    pool.close()
    del x, ab, y
    torch.cuda.empty_cache()
    return elapsed, gpu_s, flags


def prefill_summary(L, n, P, elapsed, gpu_s):
    total = n * P
    tflops = PREFILL_FLOP_PER_TOKEN_HEAD * total * HV * L / gpu_s / 1e12
    return {
        "workload": f"{n} x {P}-token prefills packed per layer, {L} layers, chunk 64",
        "tokens_per_s": round(total / elapsed, 1),
        "ms_per_layer": round(gpu_s * 1e3 / L, 4),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "flop_per_token_head": round(PREFILL_FLOP_PER_TOKEN_HEAD, 1),
                     "achieved_min_count": round(tflops * PREFILL_FLOP_PER_TOKEN_HEAD_MIN
                                                 / PREFILL_FLOP_PER_TOKEN_HEAD, 2),
                     "flop_per_token_head_min": PREFILL_FLOP_PER_TOKEN_HEAD_MIN,
                     "flop_per_token_head_sequential": PREFILL_FLOP_PER_TOKEN_HEAD_SEQ,
                     "timing": "HIP events around each pass of L gdn_prefill_varlen calls "
                               "(qkv, conv-state and chunk launches)"},
    }


def one_prompt_summary(args):
    """One prompt of prefill_len tokens per layer call: the latency case, where
    the split path (chunk records for all chunks at once, then 4 groups per
    value head: 128 work-groups) runs instead of the fused chunk kernel (32)."""
    L, P = args.layers, args.prefill_len
    el, gpu_s, flags = prefill_measure(L, 1, P, args.seed, reps=2)
    if flags:
        print(f"one-prompt prefill pool status flags 0x{flags:x}", file=sys.stderr)
        return None
    s = prefill_summary(L, 1, P, el, gpu_s)
    return {"workload": s["workload"], "tokens_per_s": s["tokens_per_s"],
            "ms_per_layer": s["ms_per_layer"], "tflops": s["roofline"]["achieved"]}


def prefill_bench(args):
    """The chunked prefill alone; prints one JSON line."""
    L, n, P = args.layers, args.prefill_seqs, args.prefill_len
    elapsed, gpu_s, flags = prefill_measure(L, n, P, args.seed, reps=2)
    if flags:
        print(f"pool status flags 0x{flags:x}", file=sys.stderr)
        return 1
    summ = prefill_summary(L, n, P, elapsed, gpu_s)
    summ["one_prompt"] = one_prompt_summary(args)
    if summ["one_prompt"] is None:
        return 1
    out = {
        "metric": "GDN chunked prefill tokens/s (packed varlen, all layers)",
        "value": summ["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "ms_per_step": round(elapsed * 1e3, 3),
        "higher_is_better": True,
        "dtype": "bf16 MFMA products, f32 state",
        "data": "synthetic",
        "config": {"workload": summ["workload"], "layers": L, "sequences": n,
                   "tokens_per_sequence": P},
        "roofline": summ["roofline"],
        "one_prompt": summ["one_prompt"],
    }
    print(json.dumps(out), flush=True)
    return 0


# Merged GDN input projection of Qwen3.5-35B-A3B (hidden 2048): in_proj_qkv
# (2*Hk*Dk + Hv*Dv rows), in_proj_z (Hv*Dv), in_proj_b, in_proj_a (Hv each).
QL_HIDDEN = 2048
QL_PARTS = [D, HV * DV, HV, HV]
QL_N = sum(QL_PARTS)


def qlinear_bench(args):
    """gdn_qlinear_forward on the merged q|k|v|z|b|a layer: `layers` distinct
    weight sets (426 MB at 30 layers, more than the 256 MB memory-side cache,
    so weights stream from HBM) and one launch per layer per step, inputs
    resident in HBM. Decode-sized launches (M = batch) are HBM-bound on the
    packed weights; prefill-sized ones (M in the thousands) are bound by the
    bf16 MFMA rate. Prints one JSON line."""
    import torch

    import gdn_amd
    dev = torch.device("cuda:0")
    L, Kd = args.layers, QL_HIDDEN
    M = args.qlinear_rows or args.batch
    N = sum(QL_PARTS)
    G = Kd // 64
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    layers = []
    for _ in range(L):
        parts = []
        for n in QL_PARTS:
            w = torch.randint(-2**31, 2**31 - 1, (n, Kd // 8), generator=gen, device=dev,
                              dtype=torch.int32)
            sc = (torch.rand((n, G), generator=gen, device=dev) * 0.01 + 0.001).to(torch.bfloat16)
            bi = (torch.randn((n, G), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
            parts.append((w, sc, bi))
        layers.append(gdn_amd.QLinear(Kd, parts))
        del parts
    nsets = 2
    x = [torch.randn((M, Kd), generator=gen, device=dev).to(torch.bfloat16) for _ in range(nsets)]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def step(i, events=None):
        if events is not None:
            events[0].record()
        for l in range(L):
            layers[l].forward(x[(i + l) % nsets], y)
        if events is not None:
            events[1].record()

    steps = args.steps if M <= 256 else max(3, min(args.steps, 20))
    for i in range(max(2, min(args.warmup, 8))):
        step(i)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i, ev[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    avg_ms = sum(a.elapsed_time(b) for a, b in ev) / (steps * L)
    wbytes = N * Kd // 2 + 2 * N * G * 2            # packed nibbles + scales + biases
    iobytes = M * Kd * 2 + M * N * 2
    flops = 2.0 * M * N * Kd
    decode = M <= 256
    if decode:
        achieved = (wbytes + iobytes) / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                "algorithmic_bytes_per_launch": wbytes + iobytes}
    else:
        tf = flops / (avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None,
                "flop_per_launch": flops}
    roof.update({"kernel": "qlinear_decode_kernel<8, 2>" if M <= 64 else "qlinear_kernel<2, 4, 2, 2>",
                 "kernel_avg_us": round(avg_ms * 1e3, 2),
                 "kernel_timing": "HIP events around each step's back-to-back launches / launches"})
    out = {
        "metric": "GDN input projection (4-bit merged q|k|v|z|b|a) tokens/s, all layers",
        "value": round(M * steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "ms_per_step": round(elapsed / steps * 1e3, 4),
        "higher_is_better": True,
        "dtype": "bf16 x 4-bit affine weights, f32 accumulation",
        "data": "synthetic",
        "config": {"workload": f"{M} rows x hidden {Kd} -> {N} outputs per layer, {L} layers, "
                               "MLX affine 4-bit group 64",
                   "rows": M, "hidden": Kd, "outputs": N, "layers": L},
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = qlinear_cpu_baseline(args.cpu_seconds, L)
    for q in layers:
        q.close()
    print(json.dumps(out), flush=True)
    return 0


def _rand_qlinear(K_, parts_rows, gen, dev):
    """A QLinear of random MLX-format 4-bit parts (scales ~U(0.001, 0.011),
    biases ~N(0, 0.02))."""
    import torch

    import gdn_amd
    G = K_ // 64
    parts = []
    for n in parts_rows:
        w = torch.randint(-2**31, 2**31 - 1, (n, K_ // 8), generator=gen, device=dev,
                          dtype=torch.int32)
        sc = (torch.rand((n, G), generator=gen, device=dev) * 0.01 + 0.001).to(torch.bfloat16)
        bi = (torch.randn((n, G), generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        parts.append((w, sc, bi))
    q = gdn_amd.QLinear(K_, parts)
    del parts
    return q


def _exec_build(args, max_batch):
    """The GDN decoder stack of Qwen3.5-35B-A3B's shapes with random weights
    (and, with --hybrid, the attention layers) behind one executor."""
    import torch

    import gdn_amd
    dev = torch.device("cuda:0")
    L, B, V = args.layers, max_batch, args.vocab
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    bf = torch.bfloat16
    pool = gdn_amd.Pool(L, args.slots, HK, HV)
    P = args.prompt_len
    gl, parts = [], []
    for l in range(L):
        inp = _rand_qlinear(QL_HIDDEN, QL_PARTS, gen, dev)
        outp = _rand_qlinear(HV * DV, [QL_HIDDEN], gen, dev)
        A_log = torch.rand(HV, generator=gen, device=dev) * math.log(16.0)
        dt_bias = torch.randn(HV, generator=gen, device=dev) * 0.1
        conv_w = (torch.randn((D, KW), generator=gen, device=dev) * 0.25).to(bf)
        norm_w = (1 + 0.1 * torch.randn(DV, generator=gen, device=dev)).to(bf)
        gl.append(gdn_amd.Layer(pool, l, inp, outp, A_log, dt_bias, conv_w, norm_w, 1e-6))
        parts.append((inp, outp, A_log, dt_bias, conv_w, norm_w))
    attn, kv, NA = [], None, 0
    if args.hybrid:
        # one attention layer after every three GDN layers (positions 3, 7, ...)
        NA = L // 3
        Hq, Hkv = ATT_HQ, ATT_HKV
        nqkv = Hq * 2 * ATT_HD + 2 * Hkv * ATT_HD
        grow = P + args.warmup + 2 * args.steps + 1
        per_seq = -(-grow // ATT_PAGE)
        kv = gdn_amd.KVCache(NA, args.slots, B * per_seq + 8, per_seq, Hq, Hkv,
                             max_step_tokens=max(B, 4 * P, 64))
        for i in range(NA):
            qkv = _rand_qlinear(QL_HIDDEN, [nqkv], gen, dev)
            o = _rand_qlinear(Hq * ATT_HD, [QL_HIDDEN], gen, dev)
            qn = (1 + 0.1 * torch.randn(ATT_HD, generator=gen, device=dev)).to(bf)
            kn = (1 + 0.1 * torch.randn(ATT_HD, generator=gen, device=dev)).to(bf)
            attn.append((4 * i + 3, qkv, o, qn, kn))
    in_norm = [(1 + 0.1 * torch.randn(QL_HIDDEN, generator=gen, device=dev)).to(bf)
               for _ in range(L + NA)]
    fin = (1 + 0.1 * torch.randn(QL_HIDDEN, generator=gen, device=dev)).to(bf)
    embed = torch.randn((V, QL_HIDDEN), generator=gen, device=dev).to(bf)
    head = _rand_qlinear(QL_HIDDEN, [V], gen, dev)
    ex = gdn_amd.Executor(pool, gl, in_norm, fin, embed, head, 1e-6, max_batch=B,
                          max_prompt=max(64, 4 * P), attn_layers=attn, kv=kv, rope_theta=ATT_THETA,
                          rotary_dim=ATT_ROT)
    return dict(pool=pool, layers=gl, parts=parts, attn=attn, kv=kv, NA=NA, in_norm=in_norm,
                fin=fin, head=head, ex=ex)


def _exec_components(st, L, B, V, reps=4):
    """Per-launch averages (us) of the decode step's kernels, from HIP events
    around HIP-graph replays of each kind of call made over all L layers with
    the executor's arguments (B rows, the same projections, norms and pool; the
    fused decode on B slots the executor does not use): the residual add +
    norm with the group sums, in_proj taking them, the fused decode with the
    RMSNormGated epilogue, out_proj (summing its K slices itself, where the
    executor's step leaves them to the next norm), and the final norm with the
    group sums + lm_head taking them. A graph of L back-to-back calls keeps the host out of the timed
    region."""
    import torch

    import gdn_amd
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    bf = torch.bfloat16
    pool, parts, in_norm = st["pool"], st["parts"], st["in_norm"]
    h = torch.randn((B, QL_HIDDEN), generator=g, device=dev).to(bf)
    d = torch.randn((B, QL_HIDDEN), generator=g, device=dev).to(bf)
    hn = torch.empty_like(h)
    gs = torch.empty((3, 64, QL_HIDDEN // 64), dtype=bf, device=dev)
    proj = torch.empty((B, QL_N), dtype=bf, device=dev)
    gated = torch.empty((B, HV * DV), dtype=bf, device=dev)
    out = torch.empty((B, QL_HIDDEN), dtype=bf, device=dev)
    logits = torch.empty((B, V), dtype=bf, device=dev)
    base = st["pool"].S - B
    ids = torch.arange(base, base + B, dtype=torch.int32, device=dev)
    qkvz, ab = proj[:, :D + HV * DV], proj[:, QL_N - 2 * HV:]

    def norm_all():
        for l in range(L):
            gdn_amd.add_rms_norm(h, d, in_norm[l], 1e-6, hn, gs)

    def in_all():
        for l in range(L):
            parts[l][0].forward_sums(hn, gs, proj)

    def dec_all():
        for l in range(L):
            inp, outp, A_log, dt_bias, conv_w, norm_w = parts[l]
            pool.decode_gated(l, ids, qkvz, ab, A_log, dt_bias, conv_w, norm_w, 1e-6, gated)

    def out_all():
        for l in range(L):
            parts[l][1].forward(gated, out)

    def head_one():
        gdn_amd.add_rms_norm(h, None, st["fin"], 1e-6, hn, gs)
        st["head"].forward_sums(hn, gs, logits)

    res = {}
    side = torch.cuda.Stream()
    for name, fn, n in (("residual_add_norm_us", norm_all, L), ("in_proj_us", in_all, L),
                        ("decode_gated_us", dec_all, L), ("out_proj_us", out_all, L),
                        ("final_norm_lm_head_us", head_one, 1)):
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()  # eager warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        res[name] = round(e0.elapsed_time(e1) * 1e3 / (reps * n), 2)
        del graph
    if pool.check():
        raise RuntimeError("pool status flags after the component timing")
    return res


def exec_measure(args, steps, warmup, components=False):
    """Time the executor's decode step over `steps` steps after `warmup`, B
    sequences prefilled with `prompt_len`-token prompts: the double-buffered
    loop (gdn_exec_submit_next: each step queued on the device picks of the
    step before while that one runs, as src/bin/qwen_mlx_infer.rs:136-187 does)
    and the host-fed loop (submit + collect, the picks through the host). Both
    include the host side (staging, launches, the wait for the picked tokens).
    Returns a dict, or None on a pool error."""
    import torch
    L, B, V, P = args.layers, args.batch, args.vocab, args.prompt_len
    st = _exec_build(args, B)
    ex, pool = st["ex"], st["pool"]
    rng = torch.Generator().manual_seed(args.seed)
    ids = list(range(1, B + 1))
    prompts = [torch.randint(0, V, (P,), generator=rng).tolist() for _ in ids]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    cur = [ex.prefill(i, p) for i, p in zip(ids, prompts)]
    pre_one = (time.perf_counter() - t0) / B
    # the same prompts again (known sequences start over), four per call
    g = min(4, B)
    t0 = time.perf_counter()
    again = []
    for k in range(0, B, g):
        again += ex.prefill_batch(ids[k:k + g], prompts[k:k + g])
    pre_batched = (time.perf_counter() - t0) / B
    if again != cur:
        print("batched prefill picked other first tokens than single prefills", file=sys.stderr)
    for _ in range(warmup):
        cur = ex.decode_batch(ids, cur)
    torch.cuda.synchronize()
    # Python's cyclic garbage collector can stop the host loop for tens of ms
    # (measured: one step of 40-65 ms in some runs, the median 2.17 ms); the
    # timed loops run with it off
    gc.collect()
    gc.disable()
    fed_steps = []
    t0 = time.perf_counter()
    for _ in range(steps):
        ts = time.perf_counter()
        ex.submit_batch(ids, cur)
        cur = ex.collect_batch(B)
        fed_steps.append(time.perf_counter() - ts)
    fed_elapsed = time.perf_counter() - t0
    fed_steps.sort()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ex.submit_batch(ids, cur)
    for _ in range(steps - 1):
        ex.submit_next(B)
        cur = ex.collect_batch(B)
    cur = ex.collect_batch(B)
    elapsed = time.perf_counter() - t0
    gc.enable()
    flags = pool.check()
    if flags:
        print(f"pool status flags 0x{flags:x}", file=sys.stderr)
        return None
    comp = _exec_components(st, L, B, V) if components and not args.hybrid else None
    NA = st["NA"]
    ex.close()
    for layer in st["layers"]:
        layer.close()
    ms = elapsed / steps * 1e3
    wbytes = L * (QL_N * QL_HIDDEN // 2 + 2 * QL_N * (QL_HIDDEN // 64) * 2
                  + QL_HIDDEN * HV * DV // 2 + 2 * QL_HIDDEN * (HV * DV // 64) * 2) \
        + V * QL_HIDDEN // 2 + 2 * V * (QL_HIDDEN // 64) * 2
    if args.hybrid:
        nqkv = ATT_HQ * 2 * ATT_HD + 2 * ATT_HKV * ATT_HD
        wbytes += NA * (nqkv * QL_HIDDEN // 2 + 2 * nqkv * (QL_HIDDEN // 64) * 2
                        + QL_HIDDEN * ATT_HQ * ATT_HD // 2
                        + 2 * QL_HIDDEN * (ATT_HQ * ATT_HD // 64) * 2)
    # cached keys read per step by the attention layers (mean context over the timed steps)
    kv_bytes = NA * B * (P + warmup + steps / 2) * ATT_HKV * ATT_HD * 2 * 2
    step_bytes = B * L * STATE_BYTES + wbytes + int(kv_bytes)
    return dict(tokens_per_s=B * steps / elapsed, ms=ms, fed_ms=fed_elapsed / steps * 1e3,
                fed_median_ms=fed_steps[len(fed_steps) // 2] * 1e3, fed_max_ms=fed_steps[-1] * 1e3,
                pre_one=pre_one, pre_batched=pre_batched, g=g, NA=NA, step_bytes=step_bytes,
                gbs=step_bytes / (ms * 1e-3) / 1e9, components=comp)


def exec_summary(args):
    """The executor sub-object of the default line: the decode step of the
    30-layer GDN decoder stack (in_proj, fused decode + norm-gate, out_proj,
    lm_head 2048 -> 248,320, greedy pick) at B = 64."""
    r = exec_measure(args, args.exec_steps, 8, components=True)
    if r is None:
        return None
    return {
        "workload": f"executor decode step: {args.layers} GDN layers (in_proj, fused decode + "
                    f"norm-gate, out_proj) + lm_head {QL_HIDDEN}->{args.vocab}, greedy pick, "
                    f"B={args.batch}, {args.slots}-slot pools, {args.prompt_len}-token prompts, "
                    "random 4-bit weights",
        "tokens_per_s": round(r["tokens_per_s"], 1),
        "ms_per_step_chained": round(r["ms"], 4),
        "ms_per_step_host_fed": round(r["fed_ms"], 4),
        "host_fed_step_median_ms": round(r["fed_median_ms"], 4),
        "host_fed_step_max_ms": round(r["fed_max_ms"], 4),
        "steps": args.exec_steps,
        "kernel_avg_us": r["components"],
        "kernel_timing": "HIP events around HIP-graph replays of each kind of call over all "
                         "layers (same arguments as the step), divided by the calls",
        "step_timing": "wall clock over the steps: chained = each step queued on the previous "
                       "step's device picks (gdn_exec_submit_next); host-fed = submit + collect",
    }


def exec_bench(args):
    """The executor's decode step over the GDN decoder stack of
    Qwen3.5-35B-A3B's shapes: hidden 2048, `layers` GDN layers (merged 4-bit
    in_proj 2048 -> 12352, fused conv/norm/gates/recurrence/norm-gate, 4-bit
    out_proj 4096 -> 2048), 4-bit lm_head 2048 -> vocab, greedy pick;
    `slots`-slot pools, B sequences prefilled with `prompt_len`-token prompts.
    Random weights; tokens are the executor's own picks. Prints one JSON line
    (see exec_measure for the two loops timed)."""
    L, B, V, P = args.layers, args.batch, args.vocab, args.prompt_len
    r = exec_measure(args, args.steps, args.warmup,
                     components=not (args.hybrid or args.no_components))
    if r is None:
        return 1
    NA, g = r["NA"], r["g"]
    out = {
        "metric": "GDN decoder-stack decode tokens/s through the executor (B sequences, all layers)",
        "value": round(r["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 4),
        "higher_is_better": True,
        "dtype": "bf16 activations, 4-bit affine weights, f32 state",
        "data": "synthetic",
        "config": {"workload": f"executor decode step: {L} GDN layers (in_proj, fused decode + "
                               f"norm-gate, out_proj)"
                               + (f" + {NA} attention layers (q|k|v proj, paged-KV attention, "
                                  f"o_proj) interleaved" if NA else "")
                               + f" + lm_head {QL_HIDDEN}->{V}, B={B}, {args.slots}-slot pools, "
                                 f"{P}-token prompts",
                   "layers": L, "attention_layers": NA, "batch": B, "slots": args.slots,
                   "hidden": QL_HIDDEN, "vocab": V, "prompt_tokens": P},
        "host_fed_ms_per_step": round(r["fed_ms"], 4),
        "host_fed_step_median_ms": round(r["fed_median_ms"], 4),
        "host_fed_step_max_ms": round(r["fed_max_ms"], 4),
        "timing": "wall clock over the steps, each queued on the previous step's device picks "
                  "(gdn_exec_submit_next) and collected after; host_fed_ms_per_step: submit + "
                  "collect per step, the picks through the host",
        "prefill_ms_per_sequence": {"prompt_tokens": P, "one_per_call": round(r["pre_one"] * 1e3, 3),
                                    f"{g}_per_call": round(r["pre_batched"] * 1e3, 3)},
        "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(r["gbs"] / PEAK_HBM_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_step": r["step_bytes"],
                     "note": "whole step (state read+write of B sequences in every GDN layer, "
                             "every weight byte once, every cached K/V byte once) over the "
                             "host-measured step time"},
    }
    if r["components"] is not None:
        out["kernel_avg_us"] = r["components"]
    print(json.dumps(out), flush=True)
    return 0


# Qwen3.5-35B-A3B's full-attention layers (every fourth of 40): 16 query
# heads (each 256 query + 256 gate outputs of q_proj), 2 kv heads, head dim
# 256, RoPE over the first 64 dimensions with base 1e7.
ATT_HQ, ATT_HKV, ATT_HD, ATT_ROT, ATT_THETA = 16, 2, 256, 64, 1.0e7
ATT_PAGE = 64


def attn_bench(args):
    """The attention layers' decode step: B sequences with ragged cached
    contexts (uniform in [C/2, 3C/2] tokens, written by chunked prefill steps
    through the same path), each appending one token per step in every layer:
    one gdn_kv_step, then one gdn_attn_forward per layer (q/k norm + RoPE and
    the K/V append, split softmax over the pages, merge + output gate). Inputs
    are synthetic bf16 projection outputs resident in HBM. Prints one JSON
    line; the dominant traffic is every cached K and V byte read once per
    layer."""
    import numpy as np
    import torch

    import gdn_amd
    dev = torch.device("cuda:0")
    L, B, C = args.attn_layers, args.batch, args.context
    Hq, Hkv, hd = ATT_HQ, ATT_HKV, ATT_HD
    rng = np.random.default_rng(args.seed)
    lens = rng.integers(C // 2, C + C // 2 + 1, B)
    grow = args.warmup + args.steps + 1
    pages = [int(-(-(n + grow) // ATT_PAGE)) for n in lens]
    chunk = 2048
    kv = gdn_amd.KVCache(L, B, sum(pages) + 4, max(pages), Hq, Hkv,
                         max_step_tokens=max(chunk, B))
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    bf = torch.bfloat16
    qn = [(1 + 0.1 * torch.randn(hd, generator=gen, device=dev)).to(bf) for _ in range(L)]
    kn = [(1 + 0.1 * torch.randn(hd, generator=gen, device=dev)).to(bf) for _ in range(L)]
    qbuf = torch.randn((chunk, Hq * 2 * hd), generator=gen, device=dev).to(bf)
    kbuf = torch.randn((chunk, Hkv * hd), generator=gen, device=dev).to(bf)
    vbuf = torch.randn((chunk, Hkv * hd), generator=gen, device=dev).to(bf)
    obuf = torch.empty((chunk, Hq * hd), dtype=bf, device=dev)

    def layers(T, events=None):
        for l in range(L):
            if events is not None:
                events[l][0].record()
            kv.forward(l, qbuf[:T], kbuf[:T], vbuf[:T], qn[l], kn[l], 1e-6, ATT_THETA, ATT_ROT,
                       obuf[:T])
            if events is not None:
                events[l][1].record()

    t0 = time.perf_counter()
    for b in range(B):   # fill the caches: prompts in steps of at most `chunk` tokens
        done = 0
        while done < lens[b]:
            n = int(min(chunk, lens[b] - done))
            kv.step([b], [n])
            layers(n)
            done += n
    torch.cuda.synchronize()
    fill_s = time.perf_counter() - t0
    ids = list(range(B))
    ones = [1] * B
    for _ in range(args.warmup):
        kv.step(ids, ones)
        layers(B)
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(L)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    keys0 = sum(kv.length(b) for b in ids)
    t0 = time.perf_counter()
    for i in range(args.steps):
        kv.step(ids, ones)
        layers(B, ev[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    avg_ms = sum(a.elapsed_time(b) for st in ev for a, b in st) / (args.steps * L)
    # keys attended per layer per step, averaged over the timed steps (each
    # sequence attends its cached keys plus the appended one)
    keys = keys0 + B * (args.steps + 1) / 2.0
    kv_bytes = keys * Hkv * hd * 2 * 2                       # K and V rows, bf16
    io_bytes = B * (Hq * 2 * hd + 2 * Hkv * hd + Hq * hd) * 2  # q|gate, k, v in; out
    achieved = (kv_bytes + io_bytes) / (avg_ms * 1e-3) / 1e9
    out = {
        "metric": "attention-layer decode tokens/s on the paged KV cache (B sequences, all "
                  "attention layers)",
        "value": round(B * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "dtype": "bf16 K/V, f32 softmax and accumulation",
        "data": "synthetic",
        "config": {"workload": f"{L} attention layers (16 q heads, 2 kv heads, head dim 256), "
                               f"B={B} ragged contexts uniform in [{C // 2}, {C + C // 2}] "
                               f"tokens, 64-token pages",
                   "layers": L, "batch": B, "mean_context": round(keys0 / B, 1),
                   "q_heads": Hq, "kv_heads": Hkv, "head_dim": hd},
        "cache_fill_s": round(fill_s, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "gdn_attn_forward (attn_prep_kernel + attn_block_kernel<8> + "
                               "attn_combine_kernel<8>)",
                     "kernel_avg_us": round(avg_ms * 1e3, 2),
                     "kernel_timing": "HIP events around each layer's gdn_attn_forward",
                     "algorithmic_bytes_per_launch": int(kv_bytes + io_bytes)},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = attn_cpu_baseline(args.cpu_seconds, L, C)
    kv.close()
    print(json.dumps(out), flush=True)
    return 0


def attn_cpu_baseline(seconds: float, layers: int, context: int):
    """The oracle's attention step (float64 numpy) decoding one sequence at
    `context` cached tokens, one token per call, for about `seconds`;
    reported per token through `layers` layers like the GPU figure."""
    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(5)
    hd = ATT_HD
    bf = lambda a: O.f32_to_bf16(a.astype(np.float32))  # noqa: E731
    ck = bf(rng.standard_normal((ATT_HKV, context, hd)))
    cv = bf(rng.standard_normal((ATT_HKV, context, hd)))
    w = bf(1 + 0.1 * rng.standard_normal(hd))
    q = bf(rng.standard_normal((1, ATT_HQ * 2 * hd)))
    k = bf(rng.standard_normal((1, ATT_HKV * hd)))
    v = bf(rng.standard_normal((1, ATT_HKV * hd)))
    n, t0 = 0, time.perf_counter()
    while True:
        O.attention_step(q, k, v, w, w, 1e-6, ATT_THETA, ATT_ROT, ck, cv, ATT_HQ, ATT_HKV)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 5000:
            break
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] + [1])
    except Exception:
        cores = 1
    return {"value": round(n / el / layers, 3), "unit": "tokens/s", "cores": cores,
            "kind": "port",
            "sample": f"{n} single-token steps of one sequence at {context} cached tokens through "
                      f"one layer ({el:.1f} s), scaled to {layers} layers, float64 oracle "
                      f"(numpy, BLAS threads {cores}), {_cpu_model()}"}


def qlinear_cpu_baseline(seconds: float, layers: int):
    """The oracle's quantized matmul (float64, OpenMP over outputs) on 8-row
    slices of the same layer shape, repeated for about `seconds`; reported per
    token through `layers` layers like the GPU figure."""
    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(3)
    N = sum(QL_PARTS)
    w = rng.integers(0, 2**32, (N, QL_HIDDEN // 8), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_bf16((rng.random((N, QL_HIDDEN // 64)) * 0.01).astype(np.float32))
    bi = O.f32_to_bf16((rng.standard_normal((N, QL_HIDDEN // 64)) * 0.02).astype(np.float32))
    x = O.f32_to_bf16(rng.standard_normal((8, QL_HIDDEN)).astype(np.float32))
    n, t0 = 0, time.perf_counter()
    while True:
        O.qmatmul_w4(x, w, sc, bi)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 200:
            break
    return {"value": round(8 * n / el / layers, 3), "unit": "tokens/s", "cores": O.num_threads(),
            "kind": "port",
            "sample": f"{n} x 8-row slices through one {QL_HIDDEN}->{N} layer ({el:.1f} s), "
                      f"scaled to {layers} layers, "
                      f"float64 oracle, {O.num_threads()} threads, {_cpu_model()}"}


class Workload:
    def __init__(self, args):
        import numpy as np
        import torch

        import gdn_amd

        self.args = args
        self.torch = torch
        self.dev = torch.device("cuda:0")
        L, S, B = args.layers, args.slots, args.batch
        self.L, self.S, self.B = L, S, B
        self.pool = gdn_amd.Pool(L, S, HK, HV)
        gen = torch.Generator(device=self.dev).manual_seed(args.seed)
        bf = torch.bfloat16
        self.conv_w = [(torch.randn((D, KW), generator=gen, device=self.dev) * 0.25).to(bf)
                       for _ in range(L)]
        self.A_log = [torch.rand(HV, generator=gen, device=self.dev) * math.log(16.0)
                      for _ in range(L)]
        self.dt_bias = [torch.randn(HV, generator=gen, device=self.dev) * 0.1 for _ in range(L)]
        self.nsets = 4
        if args.gated:
            # merged projection rows: q|k|v then z (qwen3_5.rs:572-577)
            self.qkvz = torch.randn((self.nsets, L, B, D + HV * DV), generator=gen,
                                    device=self.dev).to(bf)
            self.norm_w = [(1.0 + 0.1 * torch.randn(DV, generator=gen, device=self.dev)).to(bf)
                           for _ in range(L)]
            self.out = torch.empty((L, B, HV, DV), dtype=bf, device=self.dev)
        else:
            self.mixed = torch.randn((self.nsets, L, B, D), generator=gen, device=self.dev).to(bf)
        self.ab = torch.randn((self.nsets, L, B, 2 * HV), generator=gen, device=self.dev).to(bf)
        self.y = torch.empty((L, B, HV, DV), dtype=bf, device=self.dev)
        # initial states: every slot of every layer seeded random (state ~N(0,0.01),
        # conv ~N(0,1)), written through gdn_slots_write in chunks of 64 slots
        chunk = 64
        st = torch.empty((chunk, HV, DV, DK), dtype=torch.float32, device=self.dev)
        cs = torch.empty((chunk, KW - 1, D), dtype=bf, device=self.dev)
        for l in range(L):
            for s0 in range(0, S, chunk):
                n = min(chunk, S - s0)
                ids = torch.arange(s0, s0 + n, dtype=torch.int32, device=self.dev)
                st.normal_(0.0, 0.01, generator=gen)
                cs.normal_(0.0, 1.0, generator=gen)
                self.pool.write(l, ids, st[:n], cs[:n])
        self.rng = np.random.default_rng(args.seed)
        self.active = [int(s) for s in self.rng.choice(S, B, replace=False)]
        self.d_ids = torch.tensor(self.active, dtype=torch.int32, device=self.dev)
        self.d_new = torch.empty(args.churn, dtype=torch.int32, device=self.dev)
        self.step_no = 0
        torch.cuda.synchronize()

    def churn(self):
        """Retire `churn` sequences (random batch positions) and admit as many
        new ones into the freed slots with zeroed state; new sequences join the
        back of the batch (round-robin order of the reference scheduler)."""
        import numpy as np
        c = self.args.churn
        pos = set(int(p) for p in self.rng.choice(self.B, c, replace=False))
        freed = [self.active[p] for p in sorted(pos)]
        self.active = [s for i, s in enumerate(self.active) if i not in pos] + freed
        self.d_new.copy_(self.torch.from_numpy(np.asarray(freed, np.int32)), non_blocking=False)
        self.pool.zero(-1, self.d_new)
        self.d_ids.copy_(self.torch.from_numpy(np.asarray(self.active, np.int32)))

    def step(self, events=None):
        """One decode step: L back-to-back gdn_decode launches (bracketed by the
        event pair `events` on the launch stream when given), then churn."""
        k = self.step_no % self.nsets
        if events is not None:
            events[0].record()
        if self.args.gated:
            for l in range(self.L):
                self.pool.decode_gated(l, self.d_ids, self.qkvz[k, l], self.ab[k, l],
                                       self.A_log[l], self.dt_bias[l], self.conv_w[l],
                                       self.norm_w[l], 1e-6, self.out[l])
        else:
            for l in range(self.L):
                self.pool.decode(l, self.d_ids, self.mixed[k, l], self.ab[k, l], self.A_log[l],
                                 self.dt_bias[l], self.conv_w[l], self.y[l])
        if events is not None:
            events[1].record()
        self.step_no += 1
        if self.args.churn_every > 0 and self.step_no % self.args.churn_every == 0:
            self.churn()


def profiled_traffic(args):
    """HBM bytes per launch of the timed decode kernel from the committed PMC
    profile (FETCH_SIZE + WRITE_SIZE passes, calibrated on a plain copy), with
    a label saying so. The figure is used only when the profile was taken on
    this batch size, on the ungated kernel, and from the kernel source as it is
    now (sha256 of the source file); otherwise (None, reason)."""
    import hashlib
    if not os.path.exists(TRAFFIC_FILE):
        return None, "no PMC profile"
    with open(TRAFFIC_FILE) as f:
        tr = json.load(f)
    if tr.get("batch") != args.batch or args.gated:
        return None, "PMC profile is of another batch size or of the ungated kernel"
    src = os.path.join(ROOT, tr.get("kernel_source", ""))
    if not os.path.isfile(src):
        return None, "kernel source of the PMC profile not found"
    with open(src, "rb") as f:
        sha = hashlib.sha256(f.read()).hexdigest()[:16]
    if sha != tr.get("kernel_source_sha256_16"):
        return None, "kernel source changed since the PMC profile"
    return tr.get("hbm_bytes_per_launch"), (
        f"PMC FETCH_SIZE + WRITE_SIZE of {tr.get('kernel')} from {tr.get('source')} "
        f"(kernel source sha256 {sha}), not measured in this run")


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds: float, layers: int = 30, batch: int = 64):
    """Oracle restatement of the reference step (stack copy, out-of-place
    kernel, unstack as views) on the measured shape -- B=64, 30 layers -- or
    another (layers, batch), timed on this host for a bounded number of
    steps."""
    from oracle import oracle as O
    Bc = batch
    bs = O.BaselineStep(layers, Bc, HK, HV, DK, DV, KW, seed=1)
    bs.step()  # first touch of the output buffers
    n, t0 = 0, time.perf_counter()
    while True:
        bs.step()
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 3) or n >= 100000:
            break
    return {"value": round(Bc * n / el, 2), "unit": "tokens/s", "cores": O.num_threads(),
            "kind": "port",
            "sample": f"B={Bc} sequences x {layers} GDN layers x {n} decode steps ({el:.1f} s), "
                      f"OpenMP over (b, hv), {O.num_threads()} threads of {os.cpu_count()} "
                      f"logical CPUs, {_cpu_model()}"}


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the GDN path "
              "shards by sequence slots with no communication, so N GPUs run N independent "
              "copies of this workload.", file=sys.stderr)
        return 2
    import torch

    import gdn_amd
    gdn_amd.load()
    if not torch.cuda.is_available():
        print("bench.py needs the GPU", file=sys.stderr)
        return 1
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return 0
    if args.rmw_ceiling:
        rmw_ceiling()
        return 0
    if args.copy_floor:
        return copy_floor(args)
    if args.rmw_probe:
        return rmw_probe(args)
    if args.prefill:
        return prefill_bench(args)
    if args.qlinear:
        return qlinear_bench(args)
    if args.exec:
        return exec_bench(args)
    if args.attn:
        return attn_bench(args)
    w = Workload(args)
    for _ in range(args.warmup):
        w.step()
    # HIP events on the stream the kernels are launched on (torch's current
    # stream, which the binding passes to libgdn) bracket each step's L
    # back-to-back gdn_decode launches; slot churn runs outside the brackets.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    gc.collect()
    gc.disable()  # no collector pause inside the timed region
    t0 = time.perf_counter()
    for i in range(args.steps):
        w.step(ev[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gc.enable()
    tok_s = args.batch * args.steps / elapsed
    avg_ms = sum(a.elapsed_time(b) for a, b in ev) / (args.steps * args.layers)
    launch_bytes = args.batch * STATE_BYTES
    achieved = launch_bytes / (avg_ms * 1e-3) / 1e9
    traffic, traffic_source = profiled_traffic(args)
    flags = w.pool.check()
    if flags:
        print(f"pool status flags 0x{flags:x}", file=sys.stderr)
        return 1
    # The same 64 sequences' kernel time when they sit in slots 0..63
    # (contiguous), in the same run: the scattered placement above is the
    # measured workload, this one shows what the placement costs.
    placement = None
    if not args.no_placement:
        # The same 64 sequences moved to other slots (contiguous, every 16th
        # slot), same kernel, no churn: the scattered placement above is the
        # measured workload, these show how much the placement matters.
        import torch as _t
        w.args.churn_every = 0
        placement = {"scattered_slots_kernel_avg_us": round(avg_ms * 1e3, 2)}
        for pname in ("contiguous", "every16"):
            w.d_ids.copy_(_t.tensor(placement_slots(pname, args.batch, args.slots, args.seed),
                                    dtype=_t.int32))
            for _ in range(4):
                w.step()
            pev = [(_t.cuda.Event(enable_timing=True), _t.cuda.Event(enable_timing=True))
                   for _ in range(args.placement_steps)]
            _t.cuda.synchronize()
            for i in range(args.placement_steps):
                w.step(pev[i])
            _t.cuda.synchronize()
            p_ms = sum(a.elapsed_time(b) for a, b in pev) / (args.placement_steps * args.layers)
            key = "contiguous_slots" if pname == "contiguous" else "every16th_slot"
            placement[f"{key}_kernel_avg_us"] = round(p_ms * 1e3, 2)
            placement[f"{key}_frac"] = round(launch_bytes / (p_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
            if w.pool.check():
                print(f"pool status flags after the {pname} placement run", file=sys.stderr)
                return 1
        placement["note"] = ("same 64 sequences and kernel moved to slots 0..63 and to every 16th "
                             f"slot, no churn, {args.placement_steps} steps each")
    prefill = None
    if not args.no_prefill:
        del w
        import torch as _t
        _t.cuda.empty_cache()
        p_el, p_gpu, p_flags = prefill_measure(args.layers, args.prefill_seqs, args.prefill_len,
                                               args.seed, reps=2)
        if p_flags:
            print(f"prefill pool status flags 0x{p_flags:x}", file=sys.stderr)
            return 1
        prefill = prefill_summary(args.layers, args.prefill_seqs, args.prefill_len, p_el, p_gpu)
        prefill["one_prompt"] = one_prompt_summary(args)
        if prefill["one_prompt"] is None:
            return 1
    exec_obj = None
    if not args.no_exec:
        import torch as _t
        w = None
        _t.cuda.empty_cache()
        exec_obj = exec_summary(args)
        if exec_obj is None:
            return 1
    out = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "large ragged GDN decode: 30 layers x 1024-slot pools, B=64 scattered "
                        "slots, 8 retire + 8 admit (zeroed) every 16 steps",
            "layers": args.layers, "slots": args.slots, "batch": args.batch,
            "heads_k": HK, "heads_v": HV, "head_dim": DK, "conv_channels": D, "conv_width": KW,
            "io": "bf16 activations, f32 recurrent state, bf16 conv state",
            "epilogue": "RMSNormGated (gdn_decode_gated)" if args.gated else "none (gdn_decode)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "kernel": ("gdn_decode_gated (decode_kernel<2, true>)" if args.gated
                       else "gdn_decode (decode_kernel<2, false>)"),
            "kernel_avg_us": round(avg_ms * 1e3, 2),
            "kernel_timing": "HIP events around each step's back-to-back launches / launches",
            "algorithmic_bytes_per_launch": launch_bytes,
        },
        "state_traffic_gbs_whole_step": round(args.batch * args.layers * STATE_BYTES /
                                              (elapsed / args.steps) / 1e9, 1),
    }
    if placement is not None:
        out["placement"] = placement
    if prefill is not None:
        out["prefill"] = prefill
    if exec_obj is not None:
        out["exec"] = exec_obj
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
        # the reference's CPU-runnable case: one layer, one sequence
        out["cpu_baseline_1layer_b1"] = cpu_baseline(min(3.0, args.cpu_seconds), 1, 1)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
