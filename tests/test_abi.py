"""CPU checks of the C ABI: libgdn.so loads, exports every function that
include/gdn.h declares, and rejects bad arguments on the host (no GPU call)."""
import ctypes
import re

import pytest

import gdn_amd


def _declared():
    src = open(gdn_amd.HEADER_PATH).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(gdn_[a-z_0-9]+)\s*\(", src)))


def test_header_declares_the_bound_functions():
    assert _declared() == sorted(gdn_amd.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = gdn_amd.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert b"gfx950" in lib.gdn_version()


def test_invalid_pool_descriptors_fail_on_host():
    lib = gdn_amd.load()
    h = ctypes.c_void_p()
    cases = [
        (gdn_amd.PoolDesc(0, 4, 16, 32, 128, 128, 4, 0), gdn_amd.GDN_ERR_INVALID),
        (gdn_amd.PoolDesc(1, 4, 16, 24, 128, 128, 4, 0), gdn_amd.GDN_ERR_INVALID),
        (gdn_amd.PoolDesc(1, 4, 4, 32, 128, 128, 4, 0), gdn_amd.GDN_ERR_UNSUPPORTED),
        (gdn_amd.PoolDesc(1, 4, 16, 32, 64, 128, 4, 0), gdn_amd.GDN_ERR_UNSUPPORTED),
        (gdn_amd.PoolDesc(1, 4, 16, 32, 128, 128, 3, 0), gdn_amd.GDN_ERR_UNSUPPORTED),
    ]
    for desc, code in cases:
        assert lib.gdn_pool_create(ctypes.byref(desc), ctypes.byref(h)) == code
        assert h.value is None
        assert lib.gdn_last_error()
    assert lib.gdn_pool_create(None, ctypes.byref(h)) == gdn_amd.GDN_ERR_INVALID


def test_null_pool_is_rejected():
    lib = gdn_amd.load()
    assert lib.gdn_decode(None, 0, None, 1, None, None, None, None, None, None, None) \
        == gdn_amd.GDN_ERR_INVALID
    assert b"NULL" in lib.gdn_last_error()
    assert lib.gdn_pool_destroy(None) == gdn_amd.GDN_OK
    assert lib.gdn_slot_free(None, 0) == gdn_amd.GDN_ERR_INVALID


def test_product_has_no_cpu_fallback():
    """The binding only forwards device pointers: host tensors are refused."""
    import torch
    with pytest.raises(ValueError):
        gdn_amd._ptr(torch.zeros(4))


def test_qlinear_rejects_unsupported_formats_on_host():
    """gdn_qlinear_create checks format and shapes before touching a device."""
    lib = gdn_amd.load()
    h = ctypes.c_void_p()
    fake = ctypes.c_void_p(0x1000)
    rows = (ctypes.c_int32 * 1)(16)
    ptrs = (ctypes.c_void_p * 1)(fake)

    def create(K, rows_, gs=64, bits=4, n=1):
        return lib.gdn_qlinear_create(K, n, rows_, ptrs, ptrs, ptrs, gs, bits, 0, None,
                                      ctypes.byref(h))

    assert create(2048, rows, bits=8) == gdn_amd.GDN_ERR_UNSUPPORTED
    assert create(2048, rows, gs=32) == gdn_amd.GDN_ERR_UNSUPPORTED
    assert create(1000, rows) == gdn_amd.GDN_ERR_UNSUPPORTED       # K % 512
    assert create(8192, rows) == gdn_amd.GDN_ERR_UNSUPPORTED       # K > 4096
    assert create(2048, (ctypes.c_int32 * 1)(24)) == gdn_amd.GDN_ERR_UNSUPPORTED  # rows % 16
    assert create(2048, rows, n=0) == gdn_amd.GDN_ERR_INVALID
    assert h.value is None
    assert lib.gdn_qlinear_create(2048, 1, rows, ptrs, ptrs, ptrs, 64, 4, 0, None, None) \
        == gdn_amd.GDN_ERR_INVALID
    assert lib.gdn_qlinear_forward(None, None, 0, 1, None, 0, None) == gdn_amd.GDN_ERR_INVALID
    assert lib.gdn_qlinear_destroy(None) == gdn_amd.GDN_OK


def test_layer_and_executor_entries_reject_null_on_host():
    """The whole-layer, reserve, gated-prefill and executor entries check their
    handles and descriptors before touching a device."""
    lib = gdn_amd.load()
    h = ctypes.c_void_p()
    E = gdn_amd.GDN_ERR_INVALID
    assert lib.gdn_layer_create(None, ctypes.byref(h)) == E
    desc = gdn_amd.LayerDesc()  # NULL pool
    assert lib.gdn_layer_create(ctypes.byref(desc), ctypes.byref(h)) == E
    assert h.value is None
    assert lib.gdn_layer_destroy(None) == gdn_amd.GDN_OK
    assert lib.gdn_layer_decode(None, None, 1, None, 0, None, 0, None) == E
    assert lib.gdn_layer_prefill(None, None, None, 1, 4, None, 0, None, 0, None) == E
    assert lib.gdn_pool_reserve(None, 16, None) == E
    assert lib.gdn_prefill_varlen_gated(None, 0, None, None, 1, 1, None, 0, None, 0, None, None,
                                        None, None, ctypes.c_float(1e-6), None, None,
                                        None) == E
    assert lib.gdn_exec_create(None, None, ctypes.byref(h)) == E
    ed = gdn_amd.ExecDesc()  # NULL pool / weights
    assert lib.gdn_exec_create(ctypes.byref(ed), None, ctypes.byref(h)) == E
    assert h.value is None
    assert b"NULL" in lib.gdn_last_error()
    assert lib.gdn_exec_destroy(None) == gdn_amd.GDN_OK
    tok = ctypes.c_uint32()
    prompt = (ctypes.c_int32 * 1)(0)
    ids = (ctypes.c_uint64 * 1)(1)
    toks = (ctypes.c_uint32 * 1)(0)
    assert lib.gdn_exec_prefill(None, 1, prompt, 1, ctypes.byref(tok)) == E
    assert lib.gdn_exec_decode_batch(None, ids, toks, 1, toks) == E
    assert lib.gdn_exec_submit_batch(None, ids, toks, 1) == E
    assert lib.gdn_exec_collect_batch(None, toks, 1) == E
    assert lib.gdn_exec_submit_next(None, 1) == E
    assert lib.gdn_exec_release(None, 1) == E
    assert lib.gdn_exec_max_batch_size(None) == 0
    assert lib.gdn_exec_supports_pipeline(None) == 0


def test_kv_entries_reject_bad_arguments_on_host():
    """The paged-KV entries check handles and descriptors before touching a
    device: unsupported head dim or query-head ratio, bad worker limits, NULL
    handles."""
    lib = gdn_amd.load()
    h = ctypes.c_void_p()
    E = gdn_amd.GDN_ERR_INVALID
    assert lib.gdn_kv_create(None, ctypes.byref(h)) == E

    def desc(**kw):
        f = dict(num_layers=1, num_slots=2, num_pages=4, max_pages_per_slot=2, num_q_heads=16,
                 num_kv_heads=2, head_dim=256, max_step_tokens=8, device=0, max_workers=0)
        f.update(kw)
        return gdn_amd.KVDesc(**f)

    for bad, code in ((dict(head_dim=128), gdn_amd.GDN_ERR_UNSUPPORTED),
                      (dict(num_q_heads=6), gdn_amd.GDN_ERR_UNSUPPORTED),
                      (dict(num_q_heads=32), gdn_amd.GDN_ERR_UNSUPPORTED),
                      (dict(num_pages=0), E), (dict(max_step_tokens=0), E),
                      (dict(max_workers=-1), E), (dict(max_workers=1 << 20), E)):
        d = desc(**bad)
        assert lib.gdn_kv_create(ctypes.byref(d), ctypes.byref(h)) == code, bad
        assert h.value is None
    assert lib.gdn_kv_destroy(None) == gdn_amd.GDN_OK
    one = (ctypes.c_int32 * 1)(1)
    n64 = ctypes.c_int64()
    n32 = ctypes.c_int32()
    assert lib.gdn_kv_release(None, 0) == E
    assert lib.gdn_kv_length(None, 0, ctypes.byref(n64)) == E
    assert lib.gdn_kv_free_pages(None, ctypes.byref(n32)) == E
    assert lib.gdn_kv_step(None, 1, one, one, None) == E
    assert lib.gdn_attn_forward(None, 0, None, 0, None, 0, None, 0, None, None,
                                ctypes.c_float(1e-6), ctypes.c_float(1e7), 64, None, 0,
                                None) == E
    assert lib.gdn_kv_read(None, 0, 0, None, None, None) == E
