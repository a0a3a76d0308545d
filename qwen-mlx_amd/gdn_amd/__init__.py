"""ctypes binding of libgdn (include/gdn.h) for torch device tensors.

The library is the product; this module only passes device pointers across
the C ABI. It never computes anything itself and has no CPU fallback: if
lib/libgdn.so is missing or the GPU is absent, calls raise.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, "lib", "libgdn.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_ROOT), "include", "gdn.h")

GDN_OK = 0
GDN_ERR_INVALID = 1
GDN_ERR_UNSUPPORTED = 2
GDN_ERR_HIP = 3
GDN_ERR_OOM = 4
GDN_ERR_SLOTS = 5
GDN_FLAG_BAD_SLOT = 0x1
GDN_FLAG_DUP_SLOT = 0x2
GDN_FLAG_BAD_SEQLENS = 0x4
GDN_ALL_LAYERS = -1

# Exported symbols and their signatures (restype is int status unless noted).
_VP = ctypes.c_void_p
_I32 = ctypes.c_int32
SIGNATURES = {
    "gdn_last_error": ([], ctypes.c_char_p),
    "gdn_version": ([], ctypes.c_char_p),
    "gdn_pool_create": ([_VP, ctypes.POINTER(_VP)], ctypes.c_int),
    "gdn_pool_destroy": ([_VP], ctypes.c_int),
    "gdn_pool_layer_state": ([_VP, _I32, ctypes.POINTER(_VP), ctypes.POINTER(_VP)], ctypes.c_int),
    "gdn_pool_slot_bytes": ([_VP, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
                            ctypes.c_int),
    "gdn_pool_check": ([_VP, _VP, ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int),
    "gdn_slot_alloc": ([_VP, ctypes.POINTER(_I32)], ctypes.c_int),
    "gdn_slot_free": ([_VP, _I32], ctypes.c_int),
    "gdn_slots_in_use": ([_VP, ctypes.POINTER(_I32)], ctypes.c_int),
    "gdn_slots_zero": ([_VP, _I32, _VP, _I32, _VP], ctypes.c_int),
    "gdn_slots_read": ([_VP, _I32, _VP, _I32, _VP, _VP, _VP], ctypes.c_int),
    "gdn_slots_write": ([_VP, _I32, _VP, _I32, _VP, _VP, _VP], ctypes.c_int),
    "gdn_slots_validate": ([_VP, _VP, _I32, _VP], ctypes.c_int),
    "gdn_recurrent": ([_VP, _I32, _VP, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP],
                      ctypes.c_int),
    "gdn_decode": ([_VP, _I32, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP], ctypes.c_int),
    "gdn_decode_gated": ([_VP, _I32, _VP, _I32, _VP, ctypes.c_int64, _VP, ctypes.c_int64, _VP,
                          _VP, _VP, _VP, ctypes.c_float, _VP, _VP, _VP], ctypes.c_int),
    "gdn_prefill_varlen": ([_VP, _I32, _VP, _VP, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP],
                           ctypes.c_int),
    "gdn_prefill_varlen_noalloc": ([_VP, _I32, _VP, _VP, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _VP,
                                    _VP], ctypes.c_int),
    "gdn_prefill_varlen_gated": ([_VP, _I32, _VP, _VP, _I32, _I32, _VP, ctypes.c_int64, _VP,
                                  ctypes.c_int64, _VP, _VP, _VP, _VP, ctypes.c_float, _VP, _VP,
                                  _VP], ctypes.c_int),
    "gdn_qlinear_create": ([_I32, _I32, _VP, _VP, _VP, _VP, _I32, _I32, _I32, _VP,
                            ctypes.POINTER(_VP)], ctypes.c_int),
    "gdn_qlinear_destroy": ([_VP], ctypes.c_int),
    "gdn_qlinear_dims": ([_VP, ctypes.POINTER(_I32), ctypes.POINTER(_I32)], ctypes.c_int),
    "gdn_qlinear_forward": ([_VP, _VP, ctypes.c_int64, _I32, _VP, ctypes.c_int64, _VP],
                            ctypes.c_int),
    "gdn_qlinear_forward_sums": ([_VP, _VP, ctypes.c_int64, _VP, _I32, _VP, ctypes.c_int64, _VP],
                                 ctypes.c_int),
    "gdn_add_rms_norm": ([_VP, _VP, _I32, _I32, _VP, ctypes.c_float, _VP, _VP, _VP], ctypes.c_int),
    "gdn_exec_create": ([_VP, _VP, ctypes.POINTER(_VP)], ctypes.c_int),
    "gdn_exec_destroy": ([_VP], ctypes.c_int),
    "gdn_exec_prefill": ([_VP, ctypes.c_uint64, _VP, _I32, ctypes.POINTER(ctypes.c_uint32)],
                         ctypes.c_int),
    "gdn_exec_prefill_batch": ([_VP, _I32, _VP, _VP, _VP, _VP], ctypes.c_int),
    "gdn_exec_decode_batch": ([_VP, _VP, _VP, _I32, _VP], ctypes.c_int),
    "gdn_exec_submit_batch": ([_VP, _VP, _VP, _I32], ctypes.c_int),
    "gdn_exec_collect_batch": ([_VP, _VP, _I32], ctypes.c_int),
    "gdn_exec_submit_next": ([_VP, _I32], ctypes.c_int),
    "gdn_exec_release": ([_VP, ctypes.c_uint64], ctypes.c_int),
    "gdn_exec_max_batch_size": ([_VP], _I32),
    "gdn_exec_supports_pipeline": ([_VP], _I32),
    "gdn_exec_seq_slot": ([_VP, ctypes.c_uint64, ctypes.POINTER(_I32)], ctypes.c_int),
    "gdn_exec_logits": ([_VP, ctypes.POINTER(_VP), ctypes.POINTER(_I32), ctypes.POINTER(_I32)],
                        ctypes.c_int),
    "gdn_kv_create": ([_VP, ctypes.POINTER(_VP)], ctypes.c_int),
    "gdn_kv_describe": ([_VP, _VP], ctypes.c_int),
    "gdn_pool_describe": ([_VP, _VP], ctypes.c_int),
    "gdn_kv_destroy": ([_VP], ctypes.c_int),
    "gdn_kv_release": ([_VP, _I32], ctypes.c_int),
    "gdn_kv_length": ([_VP, _I32, ctypes.POINTER(ctypes.c_int64)], ctypes.c_int),
    "gdn_kv_free_pages": ([_VP, ctypes.POINTER(_I32)], ctypes.c_int),
    "gdn_kv_step": ([_VP, _I32, _VP, _VP, _VP], ctypes.c_int),
    "gdn_attn_forward": ([_VP, _I32, _VP, ctypes.c_int64, _VP, ctypes.c_int64, _VP,
                          ctypes.c_int64, _VP, _VP, ctypes.c_float, ctypes.c_float, _I32, _VP,
                          ctypes.c_int64, _VP], ctypes.c_int),
    "gdn_kv_read": ([_VP, _I32, _I32, _VP, _VP, _VP], ctypes.c_int),
    "gdn_layer_create": ([_VP, ctypes.POINTER(_VP)], ctypes.c_int),
    "gdn_layer_destroy": ([_VP], ctypes.c_int),
    "gdn_pool_reserve": ([_VP, _I32, _VP], ctypes.c_int),
    "gdn_layer_decode": ([_VP, _VP, _I32, _VP, ctypes.c_int64, _VP, ctypes.c_int64, _VP],
                         ctypes.c_int),
    "gdn_layer_prefill": ([_VP, _VP, _VP, _I32, _I32, _VP, ctypes.c_int64, _VP, ctypes.c_int64,
                           _VP], ctypes.c_int),
}


class GdnError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"libgdn status {status}: {msg}")
        self.status = status


class LayerDesc(ctypes.Structure):
    _fields_ = [("pool", _VP), ("layer", _I32), ("in_proj", _VP), ("out_proj", _VP),
                ("A_log", _VP), ("dt_bias", _VP), ("conv_w", _VP), ("norm_w", _VP),
                ("norm_eps", ctypes.c_float)]


class KVDesc(ctypes.Structure):
    _fields_ = [("num_layers", _I32), ("num_slots", _I32), ("num_pages", _I32),
                ("max_pages_per_slot", _I32), ("num_q_heads", _I32), ("num_kv_heads", _I32),
                ("head_dim", _I32), ("max_step_tokens", _I32), ("device", _I32),
                ("max_workers", _I32)]


class ExecAttnLayer(ctypes.Structure):
    _fields_ = [("position", _I32), ("qkv_proj", _VP), ("o_proj", _VP), ("q_norm_w", _VP),
                ("k_norm_w", _VP)]


class ExecDesc(ctypes.Structure):
    _fields_ = [("pool", _VP), ("num_layers", _I32), ("layers", ctypes.POINTER(_VP)),
                ("input_norm_w", ctypes.POINTER(_VP)), ("final_norm_w", _VP),
                ("rms_eps", ctypes.c_float), ("embed", _VP), ("head", _VP),
                ("max_batch", _I32), ("max_prompt", _I32), ("device", _I32),
                ("num_attn_layers", _I32), ("attn_layers", ctypes.POINTER(ExecAttnLayer)),
                ("kv", _VP), ("rope_theta", ctypes.c_float), ("rotary_dim", _I32)]


class PoolDesc(ctypes.Structure):
    _fields_ = [("num_layers", _I32), ("num_slots", _I32), ("num_k_heads", _I32),
                ("num_v_heads", _I32), ("head_k_dim", _I32), ("head_v_dim", _I32),
                ("conv_kernel", _I32), ("device", _I32)]


_lib = None


def build(jobs: int = 4) -> str:
    """Compile lib/libgdn.so for gfx950 with the package Makefile (hipcc)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", _PKG_ROOT, "lib/libgdn.so"], check=True)
    return LIB_PATH


def load(path: str = LIB_PATH):
    """Load libgdn.so and bind its signatures. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
    # torch ships its own HIP runtime; loading it first makes libgdn bind to the
    # same runtime instance, so device pointers from torch's allocator and its
    # streams are valid inside the library.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def _check(status: int):
    if status != GDN_OK:
        raise GdnError(status, load().gdn_last_error().decode())


def _ptr(t) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("libgdn takes device tensors")
    if not t.is_contiguous():
        raise ValueError("libgdn takes contiguous tensors")
    return t.data_ptr()


def _rows(t) -> tuple[int, int]:
    """(pointer, row stride in elements) of a 2-D device tensor whose rows are
    contiguous (a column slice of a wider matrix is fine)."""
    if not t.is_cuda:
        raise ValueError("libgdn takes device tensors")
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError("expected a 2-D tensor with contiguous rows")
    return t.data_ptr(), t.stride(0)


def _stream(stream) -> int | None:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


class _Dependents:
    """Destroy order of library objects whose C destroy touches another object.

    An executor's gdn_exec_destroy returns its sequences' slots to the pool and
    their pages to the KV cache, so the pool and the cache must outlive it.
    Python finalizes objects in any order when they die together (a failed
    test's frame, interpreter exit), so the pool and the cache destroy their
    registered dependents first. The list holds its dependents (objects with
    `_destroy()`) strongly: a live executor and its pool form a reference cycle
    that the garbage collector frees as one unit, and whichever of the two is
    finalized first destroys the executor before the pool. A closed executor
    leaves the list, so it no longer keeps the pool alive."""

    def __init__(self):
        self.items = []

    def add(self, obj):
        self.items.append(obj)

    def remove(self, obj):
        self.items = [o for o in self.items if o is not obj]

    def close_all(self):
        items, self.items = self.items, []
        for obj in reversed(items):
            obj._destroy()


def add_rms_norm(h, d, w, eps, hn, group_sums=None, stream=None):
    """h <- bf16(h + d) (d may be None), hn = rms_norm(h) * w over the rows of
    h [n, hidden]; group_sums [3, 64, hidden/64] (or None) receives the split
    64-column group sums of hn."""
    n, hidden = h.shape
    _check(load().gdn_add_rms_norm(_ptr(h), _ptr(d), n, hidden, _ptr(w), float(eps), _ptr(hn),
                                   _ptr(group_sums), _stream(stream)))


class Pool:
    """Device-resident GDN state pool: per layer `slots` slots of Hv*Dv*Dk f32 recurrent
    state and [slots,K-1,D] bf16 conv state. Tensors passed in are torch device
    tensors; bf16 tensors may be torch.bfloat16 or int16/uint16 bit patterns."""

    def __init__(self, num_layers: int, num_slots: int, num_k_heads: int = 16,
                 num_v_heads: int = 32, head_k_dim: int = 128, head_v_dim: int = 128,
                 conv_kernel: int = 4, device: int = 0):
        self.lib = load()
        self.desc = PoolDesc(num_layers, num_slots, num_k_heads, num_v_heads, head_k_dim,
                             head_v_dim, conv_kernel, device)
        h = _VP()
        _check(self.lib.gdn_pool_create(ctypes.byref(self.desc), ctypes.byref(h)))
        self.handle = h
        self.L, self.S = num_layers, num_slots
        self.Hk, self.Hv, self.Dk, self.Dv, self.K = (num_k_heads, num_v_heads, head_k_dim,
                                                       head_v_dim, conv_kernel)
        self.D = 2 * num_k_heads * head_k_dim + num_v_heads * head_v_dim
        self.device = device

    def close(self):
        deps = getattr(self, "_deps", None)
        if deps is not None:
            deps.close_all()
        if getattr(self, "handle", None):
            _check(self.lib.gdn_pool_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- views of the pool memory (no copies) --
    def layer_views(self, layer: int):
        """(state [S, Hv*Dv*Dk] f32, conv [S,K-1,D] int16) torch views of one layer's
        pool memory. A slot's state rows are in the pool's interleaved order (see
        gdn.h); read() and write() give the [Hv, Dv, Dk] order."""
        import torch
        sp, cp = _VP(), _VP()
        _check(self.lib.gdn_pool_layer_state(self.handle, layer, ctypes.byref(sp), ctypes.byref(cp)))
        n_state = self.S * self.Hv * self.Dv * self.Dk
        n_conv = self.S * (self.K - 1) * self.D
        state = _wrap_device(sp.value, n_state, torch.float32, self.device).view(
            self.S, self.Hv * self.Dv * self.Dk)
        conv = _wrap_device(cp.value, n_conv, torch.int16, self.device).view(
            self.S, self.K - 1, self.D)
        return state, conv

    def check(self, stream=None) -> int:
        f = ctypes.c_uint32()
        _check(self.lib.gdn_pool_check(self.handle, _stream(stream), ctypes.byref(f)))
        return f.value

    def reserve(self, max_tokens: int, stream=None):
        """Size the activation buffer and prefill workspace for Layer calls of up
        to max_tokens tokens."""
        _check(self.lib.gdn_pool_reserve(self.handle, max_tokens, _stream(stream)))

    def alloc_slot(self) -> int:
        s = _I32()
        _check(self.lib.gdn_slot_alloc(self.handle, ctypes.byref(s)))
        return s.value

    def free_slot(self, slot: int):
        _check(self.lib.gdn_slot_free(self.handle, slot))

    def slots_in_use(self) -> int:
        c = _I32()
        _check(self.lib.gdn_slots_in_use(self.handle, ctypes.byref(c)))
        return c.value

    def zero(self, layer: int, slot_ids, stream=None):
        _check(self.lib.gdn_slots_zero(self.handle, layer, _ptr(slot_ids), slot_ids.numel(),
                                       _stream(stream)))

    def read(self, layer: int, slot_ids, state_out=None, conv_out=None, stream=None):
        _check(self.lib.gdn_slots_read(self.handle, layer, _ptr(slot_ids), slot_ids.numel(),
                                       _ptr(state_out), _ptr(conv_out), _stream(stream)))

    def write(self, layer: int, slot_ids, state_in=None, conv_in=None, stream=None):
        _check(self.lib.gdn_slots_write(self.handle, layer, _ptr(slot_ids), slot_ids.numel(),
                                        _ptr(state_in), _ptr(conv_in), _stream(stream)))

    def validate(self, slot_ids, stream=None):
        _check(self.lib.gdn_slots_validate(self.handle, _ptr(slot_ids), slot_ids.numel(),
                                           _stream(stream)))

    def recurrent(self, layer, slot_ids, q, k, v, g, beta, y, stream=None):
        B, T = q.shape[0], q.shape[1]
        _check(self.lib.gdn_recurrent(self.handle, layer, _ptr(slot_ids), B, T, _ptr(q), _ptr(k),
                                      _ptr(v), _ptr(g), _ptr(beta), _ptr(y), _stream(stream)))

    def decode(self, layer, slot_ids, mixed_qkv, ab, A_log, dt_bias, conv_w, y, stream=None):
        _check(self.lib.gdn_decode(self.handle, layer, _ptr(slot_ids), slot_ids.numel(),
                                   _ptr(mixed_qkv), _ptr(ab), _ptr(A_log), _ptr(dt_bias),
                                   _ptr(conv_w), _ptr(y), _stream(stream)))

    def decode_gated(self, layer, slot_ids, qkvz, ab, A_log, dt_bias, conv_w, norm_w, norm_eps,
                     out, y=None, stream=None):
        """Decode with the RMSNormGated epilogue. qkvz: [B, >= D + Hv*Dv] rows holding
        q|k|v then z, ab: [B, >= 2*Hv] rows holding b|a; either may be a column
        slice of the merged projection output. out (and optional y) [B,Hv,Dv]."""
        xp, xs = _rows(qkvz)
        ap, as_ = _rows(ab)
        _check(self.lib.gdn_decode_gated(self.handle, layer, _ptr(slot_ids), slot_ids.numel(),
                                         xp, xs, ap, as_, _ptr(A_log), _ptr(dt_bias),
                                         _ptr(conv_w), _ptr(norm_w), float(norm_eps), _ptr(out),
                                         _ptr(y), _stream(stream)))

    def prefill(self, layer, slot_ids, cu_seqlens, total_tokens, mixed_qkv, ab, A_log, dt_bias,
                conv_w, y, stream=None):
        _check(self.lib.gdn_prefill_varlen(self.handle, layer, _ptr(slot_ids), _ptr(cu_seqlens),
                                           slot_ids.numel(), total_tokens, _ptr(mixed_qkv),
                                           _ptr(ab), _ptr(A_log), _ptr(dt_bias), _ptr(conv_w),
                                           _ptr(y), _stream(stream)))

    def prefill_noalloc(self, layer, slot_ids, cu_seqlens, total_tokens, mixed_qkv, ab, A_log,
                        dt_bias, conv_w, y, stream=None):
        """prefill with the library's fixed per-device scratch as its workspace
        (gdn_prefill_varlen_noalloc): no device allocation, bounded size."""
        _check(self.lib.gdn_prefill_varlen_noalloc(self.handle, layer, _ptr(slot_ids),
                                                   _ptr(cu_seqlens), slot_ids.numel(),
                                                   total_tokens, _ptr(mixed_qkv), _ptr(ab),
                                                   _ptr(A_log), _ptr(dt_bias), _ptr(conv_w),
                                                   _ptr(y), _stream(stream)))

    def prefill_gated(self, layer, slot_ids, cu_seqlens, total_tokens, qkvz, ab, A_log, dt_bias,
                      conv_w, norm_w, norm_eps, out, y=None, stream=None):
        """Prefill with the RMSNormGated epilogue; qkvz / ab as in decode_gated, one
        row per packed token. out (and optional y) [total_tokens, Hv, Dv]."""
        xp, xs = _rows(qkvz)
        ap, as_ = _rows(ab)
        _check(self.lib.gdn_prefill_varlen_gated(self.handle, layer, _ptr(slot_ids),
                                                 _ptr(cu_seqlens), slot_ids.numel(), total_tokens,
                                                 xp, xs, ap, as_, _ptr(A_log), _ptr(dt_bias),
                                                 _ptr(conv_w), _ptr(norm_w), float(norm_eps),
                                                 _ptr(out), _ptr(y), _stream(stream)))


class QLinear:
    """4-bit affine-quantized linear layer (MLX format, group 64) built from one
    or more weight parts merged along the output axis, e.g. the GDN block's
    [in_proj_qkv, in_proj_z, in_proj_b, in_proj_a]. parts: list of (w uint32
    [N_i, K/8], scales [N_i, K/64], biases [N_i, K/64]) device tensors (bf16 as
    torch.bfloat16 or int16 bit patterns; uint32 as int32 bit patterns)."""

    def __init__(self, K: int, parts, device: int = 0, stream=None, group_size: int = 64,
                 bits: int = 4):
        self.lib = load()
        n = len(parts)
        rows = (_I32 * n)(*[int(p[0].shape[0]) for p in parts])
        ws = (_VP * n)(*[_ptr(p[0]) for p in parts])
        ss = (_VP * n)(*[_ptr(p[1]) for p in parts])
        bs = (_VP * n)(*[_ptr(p[2]) for p in parts])
        h = _VP()
        _check(self.lib.gdn_qlinear_create(K, n, rows, ws, ss, bs, group_size, bits, device,
                                           _stream(stream), ctypes.byref(h)))
        self.handle = h
        k, nn = _I32(), _I32()
        _check(self.lib.gdn_qlinear_dims(h, ctypes.byref(k), ctypes.byref(nn)))
        self.K, self.N = k.value, nn.value
        self.device = device

    def forward(self, x, y, stream=None):
        """y[:, :N] = x . W^T; x [M, >= K], y [M, >= N], rows contiguous."""
        xp, xs = _rows(x)
        yp, ys = _rows(y)
        if y.shape[0] != x.shape[0]:
            raise ValueError("x and y row counts differ")
        if x.shape[1] < self.K or y.shape[1] < self.N:
            raise ValueError(f"need x [M, >= {self.K}] and y [M, >= {self.N}]")
        _check(self.lib.gdn_qlinear_forward(self.handle, xp, xs, x.shape[0], yp, ys,
                                            _stream(stream)))

    def forward_sums(self, x, group_sums, y, stream=None):
        """forward() with x's 64-column group sums supplied (add_rms_norm's
        group_sums of the same rows)."""
        xp, xs = _rows(x)
        yp, ys = _rows(y)
        if y.shape[0] != x.shape[0]:
            raise ValueError("x and y row counts differ")
        if x.shape[1] < self.K or y.shape[1] < self.N:
            raise ValueError(f"need x [M, >= {self.K}] and y [M, >= {self.N}]")
        _check(self.lib.gdn_qlinear_forward_sums(self.handle, xp, xs, _ptr(group_sums),
                                                 x.shape[0], yp, ys, _stream(stream)))

    def close(self):
        if getattr(self, "handle", None):
            _check(self.lib.gdn_qlinear_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Layer:
    """One GatedDeltaNet layer (in_proj -> conv/norm/gates/recurrence/RMSNormGated
    -> out_proj) on pool layer `layer`. in_proj, out_proj: QLinear; the weight
    tensors are device tensors kept alive by this object."""

    def __init__(self, pool, layer: int, in_proj, out_proj, A_log, dt_bias, conv_w, norm_w,
                 norm_eps: float):
        self.lib = load()
        self._keep = (pool, in_proj, out_proj, A_log, dt_bias, conv_w, norm_w)
        d = LayerDesc(pool.handle, layer, in_proj.handle, out_proj.handle, _ptr(A_log),
                      _ptr(dt_bias), _ptr(conv_w), _ptr(norm_w), float(norm_eps))
        h = _VP()
        _check(self.lib.gdn_layer_create(ctypes.byref(d), ctypes.byref(h)))
        self.handle = h
        self.hidden = in_proj.K

    def decode(self, slot_ids, x, out, stream=None):
        xp, xs = _rows(x)
        op, os_ = _rows(out)
        if x.shape[0] != slot_ids.numel() or out.shape[0] != x.shape[0]:
            raise ValueError("x / out rows must match the slot count")
        _check(self.lib.gdn_layer_decode(self.handle, _ptr(slot_ids), slot_ids.numel(), xp, xs,
                                         op, os_, _stream(stream)))

    def prefill(self, slot_ids, cu_seqlens, total_tokens, x, out, stream=None):
        xp, xs = _rows(x)
        op, os_ = _rows(out)
        if total_tokens and (x.shape[0] < total_tokens or out.shape[0] < total_tokens):
            raise ValueError("x / out hold fewer rows than total_tokens")
        _check(self.lib.gdn_layer_prefill(self.handle, _ptr(slot_ids), _ptr(cu_seqlens),
                                          slot_ids.numel(), total_tokens, xp, xs, op, os_,
                                          _stream(stream)))

    def close(self):
        if getattr(self, "handle", None):
            _check(self.lib.gdn_layer_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVCache:
    """Paged KV cache of the attention layers (64-token pages) and the
    attention step: step(slots, ntok) plans the packed tokens, then
    forward(layer, ...) runs one attention layer on them."""

    def __init__(self, num_layers: int, num_slots: int, num_pages: int, max_pages_per_slot: int,
                 num_q_heads: int = 16, num_kv_heads: int = 2, max_step_tokens: int = 4096,
                 device: int = 0, max_workers: int = 0):
        self.lib = load()
        d = KVDesc(num_layers, num_slots, num_pages, max_pages_per_slot, num_q_heads,
                   num_kv_heads, 256, max_step_tokens, device, max_workers)
        h = _VP()
        _check(self.lib.gdn_kv_create(ctypes.byref(d), ctypes.byref(h)))
        self.handle = h
        self.Hq, self.Hkv, self.device = num_q_heads, num_kv_heads, device

    def step(self, slots, ntok, stream=None):
        n = len(slots)
        s = (_I32 * n)(*[int(x) for x in slots])
        t = (_I32 * n)(*[int(x) for x in ntok])
        _check(self.lib.gdn_kv_step(self.handle, n, s, t, _stream(stream)))

    def forward(self, layer, q_full, k, v, q_norm_w, k_norm_w, eps, rope_theta, rotary_dim, out,
                stream=None):
        qp, qs = _rows(q_full)
        kp, ks = _rows(k)
        vp, vs = _rows(v)
        op, os_ = _rows(out)
        _check(self.lib.gdn_attn_forward(self.handle, layer, qp, qs, kp, ks, vp, vs,
                                         _ptr(q_norm_w), _ptr(k_norm_w), float(eps),
                                         float(rope_theta), int(rotary_dim), op, os_,
                                         _stream(stream)))

    def release(self, slot: int):
        _check(self.lib.gdn_kv_release(self.handle, slot))

    def length(self, slot: int) -> int:
        n = ctypes.c_int64()
        _check(self.lib.gdn_kv_length(self.handle, slot, ctypes.byref(n)))
        return n.value

    def free_pages(self) -> int:
        c = _I32()
        _check(self.lib.gdn_kv_free_pages(self.handle, ctypes.byref(c)))
        return c.value

    def read(self, layer: int, slot: int, stream=None):
        """(k, v) int16 [Hkv, len, 256] device copies of a slot's cache."""
        import torch
        L = self.length(slot)
        k = torch.empty((self.Hkv, L, 256), dtype=torch.int16, device=f"cuda:{self.device}")
        v = torch.empty_like(k)
        if L:
            _check(self.lib.gdn_kv_read(self.handle, layer, slot, _ptr(k), _ptr(v),
                                        _stream(stream)))
        return k, v

    def close(self):
        deps = getattr(self, "_deps", None)
        if deps is not None:
            deps.close_all()
        if getattr(self, "handle", None):
            _check(self.lib.gdn_kv_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Executor:
    """ModelExecutor (src/scheduler/executor.rs:21-49) over pool slots: the
    decoder stack h = embed[tok]; h += mixer_l(rms_norm(h, w_l)) per layer;
    greedy token of lm_head(rms_norm(h, w_final)). layers: GDN Layer objects on
    `pool`, in order; attn_layers: (position, qkv QLinear, o_proj QLinear,
    q_norm_w, k_norm_w) per attention layer, on the KVCache `kv`; input_norm_w:
    one per decoder layer in stack order; embed [vocab, hidden] bf16 device
    tensor; head: QLinear hidden -> vocab. Sequence ids are caller-chosen
    integers."""

    def __init__(self, pool, layers, input_norm_w, final_norm_w, embed, head, rms_eps=1e-6,
                 max_batch=64, max_prompt=4096, device=0, stream=None, attn_layers=(), kv=None,
                 rope_theta=1.0e7, rotary_dim=64):
        self.lib = load()
        attn_layers = list(attn_layers)
        self._keep = (pool, list(layers), list(input_norm_w), final_norm_w, embed, head,
                      attn_layers, kv)
        n = len(layers)
        na = len(attn_layers)
        self._layers = (_VP * max(n, 1))(*[l.handle.value for l in layers])
        self._norms = (_VP * max(len(input_norm_w), 1))(*[_ptr(w) for w in input_norm_w])
        self._attn = (ExecAttnLayer * max(na, 1))(
            *[ExecAttnLayer(int(p), qkv.handle, o.handle, _ptr(qn), _ptr(kn))
              for p, qkv, o, qn, kn in attn_layers])
        d = ExecDesc(pool.handle, n, self._layers, self._norms, _ptr(final_norm_w),
                     float(rms_eps), _ptr(embed), head.handle, max_batch, max_prompt, device,
                     na, self._attn, kv.handle if kv is not None else None, float(rope_theta),
                     int(rotary_dim))
        h = _VP()
        self._stream = stream
        _check(self.lib.gdn_exec_create(ctypes.byref(d), _stream(stream), ctypes.byref(h)))
        self.handle = h
        self._owners = []
        for owner in (pool, kv):
            if owner is not None:
                if getattr(owner, "_deps", None) is None:
                    owner._deps = _Dependents()
                owner._deps.add(self)
                self._owners.append(owner._deps)

    def prefill(self, seq_id: int, prompt) -> int:
        p = (_I32 * len(prompt))(*[int(t) for t in prompt])
        t = ctypes.c_uint32()
        _check(self.lib.gdn_exec_prefill(self.handle, seq_id, p, len(prompt), ctypes.byref(t)))
        return t.value

    def prefill_batch(self, seq_ids, prompts) -> list:
        """Prefill several sequences in one pass; prompts: one token list each."""
        n = len(seq_ids)
        if len(prompts) != n:
            raise ValueError("one prompt per sequence")
        flat = [int(t) for p in prompts for t in p]
        ids = (ctypes.c_uint64 * max(n, 1))(*[int(s) for s in seq_ids])
        toks = (_I32 * max(len(flat), 1))(*flat)
        lens = (_I32 * max(n, 1))(*[len(p) for p in prompts])
        out = (ctypes.c_uint32 * max(n, 1))()
        _check(self.lib.gdn_exec_prefill_batch(self.handle, n, ids, toks, lens, out))
        return list(out[:n])

    @staticmethod
    def _batch(seq_ids, tokens):
        B = len(seq_ids)
        if len(tokens) != B:
            raise ValueError("one current token per sequence")
        return (B, (ctypes.c_uint64 * B)(*[int(s) for s in seq_ids]),
                (ctypes.c_uint32 * B)(*[int(t) for t in tokens]))

    def decode_batch(self, seq_ids, tokens) -> list:
        B, s, t = self._batch(seq_ids, tokens)
        out = (ctypes.c_uint32 * max(B, 1))()
        _check(self.lib.gdn_exec_decode_batch(self.handle, s, t, B, out))
        return list(out[:B])

    def submit_batch(self, seq_ids, tokens) -> int:
        B, s, t = self._batch(seq_ids, tokens)
        _check(self.lib.gdn_exec_submit_batch(self.handle, s, t, B))
        return B

    def submit_next(self, B: int) -> int:
        """Queue another step for the last submitted batch, fed its picks on the
        device (the double-buffered decode, src/bin/qwen_mlx_infer.rs:136-187)."""
        _check(self.lib.gdn_exec_submit_next(self.handle, B))
        return B

    def collect_batch(self, B: int) -> list:
        out = (ctypes.c_uint32 * max(B, 1))()
        _check(self.lib.gdn_exec_collect_batch(self.handle, out, B))
        return list(out[:B])

    def release(self, seq_id: int):
        _check(self.lib.gdn_exec_release(self.handle, seq_id))

    def max_batch_size(self) -> int:
        return self.lib.gdn_exec_max_batch_size(self.handle)

    def supports_pipeline(self) -> bool:
        return bool(self.lib.gdn_exec_supports_pipeline(self.handle))

    def slot(self, seq_id: int) -> int:
        s = _I32()
        _check(self.lib.gdn_exec_seq_slot(self.handle, seq_id, ctypes.byref(s)))
        return s.value

    def logits(self):
        """Device logits of the last forward as a [rows, vocab] int16 (bf16 bits) view."""
        p, r, v = _VP(), _I32(), _I32()
        _check(self.lib.gdn_exec_logits(self.handle, ctypes.byref(p), ctypes.byref(r),
                                        ctypes.byref(v)))
        dev_idx = self._keep[0].device
        return _wrap_device(p.value, r.value * v.value, __import__("torch").int16,
                            dev_idx).view(r.value, v.value)

    def _destroy(self):
        if getattr(self, "handle", None):
            h, self.handle = self.handle, None
            _check(self.lib.gdn_exec_destroy(h))
        # leave the owners' lists: a closed executor no longer pins the pool
        for deps in getattr(self, "_owners", ()):
            deps.remove(self)
        self._owners = []

    def close(self):
        self._destroy()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _wrap_device(ptr: int, numel: int, dtype, device: int):
    """Zero-copy torch view of device memory owned by the pool."""
    import torch

    class _Holder:
        def __init__(self, p, n, nbytes):
            self.__cuda_array_interface__ = {
                "shape": (n,), "typestr": {torch.float32: "<f4", torch.int16: "<i2"}[dtype],
                "data": (p, False), "version": 3, "strides": None,
            }
    esz = torch.empty(0, dtype=dtype).element_size()
    with torch.cuda.device(device):
        return torch.as_tensor(_Holder(ptr, numel, numel * esz), device=f"cuda:{device}")
