"""NumPy front end of the CPU restatement in gdn_oracle.c.

TEST INFRASTRUCTURE ONLY: the checker for libgdn. Only tests, the smoke check
and the bench's CPU-baseline leg import this module; the product path never
does.

bf16 tensors are numpy uint16 arrays holding the raw bit patterns. Every
function returns new arrays and leaves its inputs untouched. The restated
reference lines are cited in gdn_oracle.c next to each C function.
StackForward (at the end) composes these pieces into the executor's decoder
stack; its composition is pinned by a closed form (mixers with zero output
weights leave lm_head(rms_norm(embed))) and by prefill / decode continuity.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_gdn.so")
_lib = None

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_c_int, _c_i64, _c_float = ctypes.c_int, ctypes.c_int64, ctypes.c_float


def build() -> str:
    """Compile liboracle_gdn.so with oracle/Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_gdn.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    L.orc_beta_g.argtypes = [_u16p, _c_i64, _c_int, _f32p, _f32p, _u16p, _f32p]
    L.orc_conv_update.argtypes = [_u16p, _u16p, _u16p, _c_int, _c_int, _c_int, _u16p, _u16p]
    L.orc_conv_prefill.argtypes = [_u16p, _u16p, _u16p, _c_int, _c_int, _c_int, _u16p, _u16p]
    L.orc_rms_norm.argtypes = [_u16p, _c_i64, _c_int, _c_float, _c_float, _u16p]
    L.orc_norm_gate.argtypes = [_u16p, _u16p, _u16p, _c_i64, _c_int, _c_float, _u16p]
    L.orc_q_norm_weight.argtypes = [_c_int]
    L.orc_q_norm_weight.restype = _c_float
    L.orc_k_norm_weight.argtypes = [_c_int]
    L.orc_k_norm_weight.restype = _c_float
    L.orc_recurrent_io.argtypes = [_u16p, _u16p, _u16p, _f32p, _u16p, _f32p, _f32p, _u16p,
                                   _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]
    L.orc_recurrent_f64.argtypes = [_u16p, _u16p, _u16p, _f32p, _u16p, _f32p, _u16p, _f64p,
                                    _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]
    L.orc_decode_io.argtypes = [_u16p, _u16p, _f32p, _f32p, _u16p, _u16p, _f32p, _f32p, _u16p,
                                _u16p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]
    L.orc_prefill.argtypes = [_u16p, _f32p, _u16p, _u16p, _f32p, _f32p, _u16p, _u16p,
                              _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]
    L.orc_num_threads.restype = _c_int
    L.orc_f64_to_bf16.argtypes = [ctypes.c_double]
    L.orc_f64_to_bf16.restype = ctypes.c_uint16
    L.orc_dequant_w4.argtypes = [_u32p, _u16p, _u16p, _c_int, _c_int, _f64p]
    L.orc_qmatmul_w4.argtypes = [_u16p, _c_i64, _c_int, _c_int, _u32p, _u16p, _u16p, _c_int,
                                 _f64p, _f64p, _u16p]
    L.orc_baseline_step.restype = None
    _lib = L
    return L


# --------------------------------------------------------------- bf16 -----

def f32_to_bf16(x) -> np.ndarray:
    """Round float32 to bf16 (round to nearest even), returned as uint16 bits.
    Finite values and infinities cannot overflow the uint32 sum; NaNs are
    patched to quiet NaNs afterwards."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(x))


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# -------------------------------------------------------------- steps -----

def beta_g(ab, A_log, dt_bias):
    """compiled_beta_g on merged ab [..., 2Hv] -> (beta bf16 [...,Hv], g f32 [...,Hv])."""
    ab = _c(ab, np.uint16)
    hv2 = ab.shape[-1]
    Hv = hv2 // 2
    ntok = ab.size // hv2
    beta = np.empty(ab.shape[:-1] + (Hv,), np.uint16)
    g = np.empty(ab.shape[:-1] + (Hv,), np.float32)
    lib().orc_beta_g(ab, ntok, Hv, _c(A_log, np.float32), _c(dt_bias, np.float32), beta, g)
    return beta, g


def conv_update(conv_state, x, w):
    """S=1 conv step. conv_state [B,K-1,D], x [B,D], w [D,K] -> (new_state, out[B,D])."""
    conv_state = _c(conv_state, np.uint16)
    B, km1, D = conv_state.shape
    out = np.empty((B, D), np.uint16)
    new = np.empty_like(conv_state)
    lib().orc_conv_update(conv_state, _c(x, np.uint16), _c(w, np.uint16), B, D, km1 + 1, new, out)
    return new, out


def conv_prefill(conv_state, x, w):
    """Prefill conv. conv_state [K-1,D], x [S,D], w [D,K] -> (new_state, out[S,D])."""
    conv_state = _c(conv_state, np.uint16)
    km1, D = conv_state.shape
    x = _c(x, np.uint16)
    S = x.shape[0]
    out = np.empty((S, D), np.uint16)
    new = np.empty_like(conv_state)
    lib().orc_conv_prefill(conv_state, x, _c(w, np.uint16), S, D, km1 + 1, new, out)
    return new, out


def rms_norm(x, w: float, eps: float = 1e-6):
    x = _c(x, np.uint16)
    dim = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_rms_norm(x, x.size // dim, dim, w, eps, out)
    return out


def norm_gate(y, z, w, eps: float = 1e-6):
    """RMSNormGated: silu(z) * rms_norm(y, w, eps) over the last axis.
    y, z bf16 [..., dim]; w bf16 [dim] -> bf16 [..., dim]."""
    y = _c(y, np.uint16)
    z = _c(z, np.uint16)
    w = _c(w, np.uint16)
    dim = y.shape[-1]
    assert z.shape == y.shape and w.shape == (dim,)
    out = np.empty_like(y)
    lib().orc_norm_gate(y, z, w, y.size // dim, dim, eps, out)
    return out


def q_norm_weight(dk: int) -> float:
    return float(lib().orc_q_norm_weight(dk))


def k_norm_weight(dk: int) -> float:
    return float(lib().orc_k_norm_weight(dk))


def recurrent(q, k, v, g, beta, state):
    """gated_delta_kernel on q,k [B,T,Hk,Dk], v [B,T,Hv,Dv], g [B,T,Hv] f32,
    beta [B,T,Hv] bf16, state [B,Hv,Dv,Dk] f32 -> (y [B,T,Hv,Dv], new_state)."""
    q, k, v = _c(q, np.uint16), _c(k, np.uint16), _c(v, np.uint16)
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    st = _c(state, np.float32)
    out_state = np.empty_like(st)
    y = np.empty((B, T, Hv, Dv), np.uint16)
    lib().orc_recurrent_io(q, k, v, _c(g, np.float32), _c(beta, np.uint16), st, out_state, y,
                           B, T, Hk, Hv, Dk, Dv)
    return y, out_state


def recurrent_f64(q, k, v, g, beta, state):
    """As recurrent() with f64 arithmetic; returns (y bf16, y f64, new_state f32)."""
    q, k, v = _c(q, np.uint16), _c(k, np.uint16), _c(v, np.uint16)
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    st = np.array(state, dtype=np.float32, copy=True, order="C")
    y = np.empty((B, T, Hv, Dv), np.uint16)
    y64 = np.empty((B, T, Hv, Dv), np.float64)
    lib().orc_recurrent_f64(q, k, v, _c(g, np.float32), _c(beta, np.uint16), st, y, y64,
                            B, T, Hk, Hv, Dk, Dv)
    return y, y64, st


def decode(conv_state, state, mixed_qkv, ab, A_log, dt_bias, conv_w, Hk: int, Hv: int):
    """Fused S=1 layer step on stacked states.
    conv_state [B,K-1,D], state [B,Hv,Dv,Dk], mixed_qkv [B,D], ab [B,2Hv],
    conv_w [D,K] -> (y [B,Hv,Dv], new_conv_state, new_state)."""
    cs = _c(conv_state, np.uint16)
    st = _c(state, np.float32)
    B, km1, D = cs.shape
    _, _, Dv, Dk = st.shape
    cs_out = np.empty_like(cs)
    st_out = np.empty_like(st)
    y = np.empty((B, Hv, Dv), np.uint16)
    lib().orc_decode_io(cs, cs_out, st, st_out, _c(mixed_qkv, np.uint16), _c(ab, np.uint16),
                        _c(A_log, np.float32), _c(dt_bias, np.float32), _c(conv_w, np.uint16),
                        y, B, Hk, Hv, Dk, Dv, km1 + 1)
    return y, cs_out, st_out


def prefill(conv_state, state, mixed_qkv, ab, A_log, dt_bias, conv_w, Hk: int, Hv: int,
            f64: bool = False):
    """One sequence of S tokens. conv_state [K-1,D], state [Hv,Dv,Dk],
    mixed_qkv [S,D], ab [S,2Hv] -> (y [S,Hv,Dv], new_conv_state, new_state)."""
    cs = np.array(conv_state, dtype=np.uint16, copy=True, order="C")
    st = np.array(state, dtype=np.float32, copy=True, order="C")
    km1, D = cs.shape
    _, Dv, Dk = st.shape
    x = _c(mixed_qkv, np.uint16)
    S = x.shape[0]
    y = np.empty((S, Hv, Dv), np.uint16)
    lib().orc_prefill(cs, st, x, _c(ab, np.uint16), _c(A_log, np.float32),
                      _c(dt_bias, np.float32), _c(conv_w, np.uint16), y, S, Hk, Hv, Dk, Dv,
                      km1 + 1, 1 if f64 else 0)
    return y, cs, st


def split_qkv(x, Hk: int, Hv: int, Dk: int, Dv: int):
    """Channel split of a conv output [..., D] into q, k [...,Hk,Dk], v [...,Hv,Dv]
    (src/models/qwen3_5.rs:626-634)."""
    qk = Hk * Dk
    q = x[..., :qk].reshape(x.shape[:-1] + (Hk, Dk))
    k = x[..., qk:2 * qk].reshape(x.shape[:-1] + (Hk, Dk))
    v = x[..., 2 * qk:].reshape(x.shape[:-1] + (Hv, Dv))
    return q, k, v


def f64_to_bf16(v: float) -> int:
    """Correctly rounded (nearest even) bf16 bits of a float64."""
    return int(lib().orc_f64_to_bf16(float(v)))


def dequant_w4(w, scales, biases):
    """MLX affine 4-bit dequantize, group 64 (qwen3_5.rs:852): w uint32 [N, K/8],
    scales/biases bf16 [N, K/64] -> float64 [N, K] (exact)."""
    w = np.ascontiguousarray(w, np.uint32)
    N, K = w.shape[0], w.shape[1] * 8
    out = np.empty((N, K), np.float64)
    lib().orc_dequant_w4(w, _c(scales, np.uint16), _c(biases, np.uint16), N, K, out)
    return out


def qmatmul_w4(x, w, scales, biases):
    """quantized_matmul(x, w, scales, biases, transpose=True, group_size=64,
    bits=4) (qwen3_5.rs:572-586): x bf16 [M, K] -> (y bf16 [M, N] correctly
    rounded, y_exact float64 [M, N], mag float64 [M, N] = sum |x|(|s|(128+q)+|b|))."""
    x = _c(x, np.uint16)
    w = np.ascontiguousarray(w, np.uint32)
    M, K = x.shape
    N = w.shape[0]
    assert w.shape[1] * 8 == K and K % 64 == 0
    ye = np.empty((M, N), np.float64)
    mag = np.empty((M, N), np.float64)
    y = np.empty((M, N), np.uint16)
    lib().orc_qmatmul_w4(x, K, M, K, w, _c(scales, np.uint16), _c(biases, np.uint16), N, ye, mag, y)
    return y, ye, mag


def stack(pool, slot_ids):
    """stack_caches for one GDN layer (mlx_executor.rs:42-55): gather by slot id."""
    return np.ascontiguousarray(pool[np.asarray(slot_ids, dtype=np.int64)])


def unstack(pool, slot_ids, batched):
    """unstack_caches (mlx_executor.rs:118-130): scatter rows back (in place)."""
    pool[np.asarray(slot_ids, dtype=np.int64)] = batched


def num_threads() -> int:
    return int(lib().orc_num_threads())


class BaselineStep:
    """CPU baseline of a B-sequence, L-layer decode step as the reference runs it
    (stack by concat copy, out-of-place kernel, unstack as views); see
    orc_baseline_step in gdn_oracle.c. Buffers are allocated once here."""

    def __init__(self, L, B, Hk, Hv, Dk, Dv, K, seed=0):
        self.L, self.B, self.Hk, self.Hv, self.Dk, self.Dv, self.K = L, B, Hk, Hv, Dk, Dv, K
        D = 2 * Hk * Dk + Hv * Dv
        se, ce = Hv * Dv * Dk, (K - 1) * D
        rng = np.random.default_rng(seed)
        # one random slot state, replicated: the timing does not depend on the values
        one_state = rng.standard_normal(se, dtype=np.float32) * 0.01
        one_conv = f32_to_bf16(rng.standard_normal(ce, dtype=np.float32))
        self.seq_state_buf = np.empty((L, B, se), np.float32)
        self.seq_state_buf[...] = one_state
        self.seq_conv_buf = np.empty((L, B, ce), np.uint16)
        self.seq_conv_buf[...] = one_conv
        self.out_state = np.zeros((L, B * se), np.float32)
        self.out_conv = np.zeros((L, B * ce), np.uint16)
        self.in_state = np.zeros(B * se, np.float32)
        self.in_conv = np.zeros(B * ce, np.uint16)
        self.mixed = f32_to_bf16(rng.standard_normal((L, B, D), dtype=np.float32))
        self.ab = f32_to_bf16(rng.standard_normal((L, B, 2 * Hv), dtype=np.float32))
        self.A_log = rng.uniform(0, np.log(16), (L, Hv)).astype(np.float32)
        self.dt_bias = (rng.standard_normal((L, Hv)) * 0.1).astype(np.float32)
        self.conv_w = f32_to_bf16(rng.standard_normal((L, D, K), dtype=np.float32) * 0.25)
        self.y = np.zeros((L, B, Hv, Dv), np.uint16)
        P = ctypes.POINTER
        self._ss = (P(ctypes.c_float) * (L * B))()
        self._sc = (P(ctypes.c_uint16) * (L * B))()
        for l in range(L):
            for b in range(B):
                self._ss[l * B + b] = self.seq_state_buf[l, b].ctypes.data_as(P(ctypes.c_float))
                self._sc[l * B + b] = self.seq_conv_buf[l, b].ctypes.data_as(P(ctypes.c_uint16))
        self._os = (P(ctypes.c_float) * L)(*[self.out_state[l].ctypes.data_as(P(ctypes.c_float))
                                             for l in range(L)])
        self._oc = (P(ctypes.c_uint16) * L)(*[self.out_conv[l].ctypes.data_as(P(ctypes.c_uint16))
                                              for l in range(L)])

    def step(self):
        vp = ctypes.c_void_p
        lib().orc_baseline_step(
            _c_int(self.L), _c_int(self.B), self._ss, self._sc,
            vp(self.in_state.ctypes.data), vp(self.in_conv.ctypes.data), self._os, self._oc,
            vp(self.mixed.ctypes.data), vp(self.ab.ctypes.data), vp(self.A_log.ctypes.data),
            vp(self.dt_bias.ctypes.data), vp(self.conv_w.ctypes.data), vp(self.y.ctypes.data),
            _c_int(self.Hk), _c_int(self.Hv), _c_int(self.Dk), _c_int(self.Dv), _c_int(self.K))


# ------------------------------------------------- attention layers -----
# Qwen35Attention::forward_with_cache (qwen3_5.rs:377-455) for one sequence,
# restated in float64 with the bf16 roundings of its MLX ops: fast::rms_norm
# (bf16(w * bf16(x * r))), fast::rope (rotate-half form over the first
# rotary_dim dimensions, traditional = false, result rounded to bf16),
# scaled_dot_product_attention (one rounding of the output), sigmoid gate
# (bf16) and the gated product (bf16).

def f64_to_bf16_array(x) -> np.ndarray:
    """Correctly rounded (nearest even) bf16 bits of float64 values, in one
    rounding step (no intermediate float32)."""
    x = np.asarray(x, dtype=np.float64)
    m, e = np.frexp(x)                      # x = m 2^e, 0.5 <= |m| < 1
    y = np.ldexp(np.rint(np.ldexp(m, 8)), e - 8)  # 8 significant bits, ties to even
    with np.errstate(over="ignore"):
        return f32_to_bf16(y.astype(np.float32))  # exact: y has at most 8 bits


def rms_norm_w(x, w, eps: float):
    """fast::rms_norm(x, w, eps) over the last axis (qwen3_5.rs:399-407): x bf16
    [..., d], w bf16 [d] -> bf16 bf16(w * bf16(x * (mean(x^2) + eps)^-1/2))."""
    xf = bf16_to_f32(x).astype(np.float64)
    wf = bf16_to_f32(w).astype(np.float64)
    rn = 1.0 / np.sqrt(np.mean(xf * xf, axis=-1, keepdims=True) + eps)
    return f64_to_bf16_array(wf * bf16_to_f32(f64_to_bf16_array(xf * rn)).astype(np.float64))


def rope_half_f64(x, pos, rot_dim: int, theta: float) -> np.ndarray:
    """fast::rope(x, rot_dim, traditional=false, base=theta, scale=1, offset)
    (qwen3_5.rs:411-417) in float64, before rounding: dimension i < rot_dim/2
    pairs with i + rot_dim/2 and turns by pos * theta^(-2i/rot_dim); the rest
    pass through. x bf16 [..., hd]; pos broadcasts against x[..., 0]."""
    xf = bf16_to_f32(x).astype(np.float64)
    out = xf.copy()
    h = rot_dim // 2
    if h == 0:
        return out
    inv = theta ** (-2.0 * np.arange(h) / rot_dim)
    ang = np.asarray(pos, np.float64)[..., None] * inv
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = xf[..., :h], xf[..., h:rot_dim]
    out[..., :h] = x1 * c - x2 * s
    out[..., h:rot_dim] = x1 * s + x2 * c
    return out


def attention_step(q_full, k, v, q_norm_w, k_norm_w, eps: float, theta: float, rot_dim: int,
                   cache_k, cache_v, Hq: int, Hkv: int):
    """One sequence's S new tokens through one attention layer: q_full bf16 [S,
    Hq * 512] (per head 256 query then 256 gate values), k, v bf16 [S, Hkv *
    256]; cache_k, cache_v bf16 [Hkv, L0, 256] (keys after norm and RoPE). The
    new tokens sit at positions L0 .. L0 + S - 1 and attend causally.
    Returns (out bf16 [S, Hq * 256], new cache_k, new cache_v)."""
    hd = 256
    G = Hq // Hkv
    S = q_full.shape[0]
    L0 = cache_k.shape[1]
    qf = np.asarray(q_full, np.uint16).reshape(S, Hq, 2, hd)
    pos = L0 + np.arange(S)
    qn = rms_norm_w(qf[:, :, 0, :], q_norm_w, eps)                            # [S, Hq, hd]
    qr = bf16_to_f32(f64_to_bf16_array(rope_half_f64(qn, pos[:, None], rot_dim, theta)))
    kn = rms_norm_w(np.asarray(k, np.uint16).reshape(S, Hkv, hd), k_norm_w, eps)
    kr = f64_to_bf16_array(rope_half_f64(kn, pos[:, None], rot_dim, theta))  # [S, Hkv, hd]
    ck = np.concatenate([np.asarray(cache_k, np.uint16), kr.transpose(1, 0, 2)], axis=1)
    cv = np.concatenate([np.asarray(cache_v, np.uint16),
                         np.asarray(v, np.uint16).reshape(S, Hkv, hd).transpose(1, 0, 2)], axis=1)
    kf = bf16_to_f32(ck).astype(np.float64)
    vf = bf16_to_f32(cv).astype(np.float64)
    gate = bf16_to_f32(qf[:, :, 1, :]).astype(np.float64)
    sg = bf16_to_f32(f64_to_bf16_array(1.0 / (1.0 + np.exp(-gate))))
    out = np.empty((S, Hq, hd), np.uint16)
    for i in range(S):
        n = L0 + i + 1
        for h in range(Hq):
            j = h // G
            sc = kf[j, :n] @ qr[i, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            o = (p @ vf[j, :n]) / p.sum()
            ob = bf16_to_f32(f64_to_bf16_array(o)).astype(np.float64)
            out[i, h] = f64_to_bf16_array(ob * sg[i, h])
    return out.reshape(S, Hq * hd), ck, cv


class StackForward:
    """The executor's decoder stack, composed from this module's pieces: the
    Qwen3.5 decoder without its MLPs, one sequence at a time.

      h = embed[tokens]                                   (qwen3_5.rs:835-855)
      per layer: h = bf16(h + mixer(rms_norm(h, in_norm)))  (qwen3_5.rs:723-743,
                                                           MLP half left out)
      logits = lm_head(rms_norm(h, final_norm))             (qwen3_5.rs:861-874)

    A GatedDeltaNet mixer (qwen3_5.rs:558-668): the merged 4-bit projections
    (q|k|v, z, b, a; :572-586), the S=1 step (`decode`, :593-610) for one
    token or the sequence form (`prefill`, :611-658) for several (the
    reference picks by the call's token count), RMSNormGated (`norm_gate`,
    :660-665) and out_proj (:668). An attention mixer (qwen3_5.rs:377-455):
    the q|gate, k, v projection, `attention_step` with the sequence's growing
    K/V (:419-424) and o_proj. Every 4-bit product is `qmatmul_w4` (exact,
    rounded once to bf16).

    layers: stack order; each a dict with "in_norm" and either
      {"in_parts": [(w, s, b)] x 4 (q|k|v, z, b, a), "out": (w, s, b), "A_log",
       "dt_bias", "conv_w", "norm_w"}  (GatedDeltaNet), or
      {"qkv": (w, s, b), "o": (w, s, b), "qn", "kn"}  (attention).
    Test infrastructure: host numpy arrays, float64 where not rounded."""

    def __init__(self, layers, final_norm_w, embed, head, eps, Hk, Hv, Hq=16, Hkv=2,
                 theta=1.0e7, rot_dim=64, Dk=128, Dv=128, K=4):
        self.layers, self.final_norm_w, self.embed, self.head = layers, final_norm_w, embed, head
        self.eps, self.Hk, self.Hv, self.Hq, self.Hkv = eps, Hk, Hv, Hq, Hkv
        self.theta, self.rot_dim, self.Dk, self.Dv, self.K = theta, rot_dim, Dk, Dv, K
        self.D = 2 * Hk * Dk + Hv * Dv
        self.seqs = {}

    def _fresh(self):
        st = []
        for L in self.layers:
            if "in_parts" in L:
                st.append([np.zeros((self.K - 1, self.D), np.uint16),
                           np.zeros((self.Hv, self.Dv, self.Dk), np.float32)])
            else:
                st.append([np.zeros((self.Hkv, 0, 256), np.uint16),
                           np.zeros((self.Hkv, 0, 256), np.uint16)])
        return st

    def forward(self, sid, tokens, fresh=False):
        """Run `tokens` of sequence `sid` (a new sequence when fresh) and return
        the last token's logits: (bf16 [vocab], exact float64 [vocab])."""
        if fresh or sid not in self.seqs:
            self.seqs[sid] = self._fresh()
        st = self.seqs[sid]
        toks = np.asarray(tokens, np.int64)
        S = len(toks)
        h = np.asarray(self.embed, np.uint16)[toks]
        Hv, Dv, D = self.Hv, self.Dv, self.D
        for L, ls in zip(self.layers, st):
            hn = rms_norm_w(h, L["in_norm"], self.eps)
            if "in_parts" in L:
                proj = np.concatenate([qmatmul_w4(hn, *p)[0] for p in L["in_parts"]], axis=1)
                mixed, z, ab = proj[:, :D], proj[:, D:D + Hv * Dv], proj[:, D + Hv * Dv:]
                if S == 1:
                    y, cs, ss = decode(ls[0][None], ls[1][None], mixed, ab, L["A_log"],
                                       L["dt_bias"], L["conv_w"], self.Hk, Hv)
                    ls[0], ls[1] = cs[0], ss[0]
                else:
                    y, ls[0], ls[1] = prefill(ls[0], ls[1], mixed, ab, L["A_log"], L["dt_bias"],
                                              L["conv_w"], self.Hk, Hv)
                g = norm_gate(y.reshape(S, Hv, Dv), z.reshape(S, Hv, Dv), L["norm_w"], self.eps)
                d = qmatmul_w4(g.reshape(S, Hv * Dv), *L["out"])[0]
            else:
                qkv = qmatmul_w4(hn, *L["qkv"])[0]
                nq, nk = self.Hq * 512, self.Hkv * 256
                att, ls[0], ls[1] = attention_step(qkv[:, :nq], qkv[:, nq:nq + nk],
                                                   qkv[:, nq + nk:nq + 2 * nk], L["qn"], L["kn"],
                                                   self.eps, self.theta, self.rot_dim, ls[0],
                                                   ls[1], self.Hq, self.Hkv)
                d = qmatmul_w4(att, *L["o"])[0]
            # residual add of two bf16 arrays: the exact sum rounded once
            h = f64_to_bf16_array(bf16_to_f32(h).astype(np.float64) +
                                  bf16_to_f32(d).astype(np.float64))
        hn = rms_norm_w(h[-1:], self.final_norm_w, self.eps)
        y, ye, _ = qmatmul_w4(hn, *self.head)
        return y[0], ye[0]
