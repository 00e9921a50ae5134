"""The C ABI of libgt_attn.so without a GPU: every declared symbol is exported, host-side
lifecycle calls behave like the reference's (csrc/gt_core.cpp:457-1087), and failures come
back as NULL / non-zero plus a message, never as an abort (gguf_train/_C.py:680-710)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C, _bridge
from gguf_train_amd.nn import functional as F

HEADER = Path(__file__).resolve().parent.parent / "include" / "gt_attn.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"GT_API\s+[\w\s\*]+?\b(gt_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(_C.lib, n)]
    assert not missing, missing


def i64(vals):
    return (ctypes.c_int64 * max(len(vals), 1))(*vals)


def test_host_tensor_lifecycle_round_trip():
    data = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    p = _C.lib.gt_tensor_from_data(3, i64(data.shape), _C.GT_F32, _C.GT_DEV_CPU, 0,
                                   data.ctypes.data_as(ctypes.c_void_p), data.nbytes)
    h = _bridge.Handle(_C.check_ptr(p))
    assert _C.lib.gt_tensor_ndim(h.ptr) == 3 and _C.lib.gt_tensor_numel(h.ptr) == 24
    assert _C.lib.gt_tensor_is_contiguous(h.ptr) == 1 and _C.lib.gt_tensor_nbytes(h.ptr) == 96
    st = i64([0, 0, 0])
    _C.lib.gt_tensor_strides(h.ptr, st)
    assert list(st) == [12, 4, 1]
    # a transposed view, copied out densely
    v = _bridge.Handle(_C.check_ptr(_C.lib.gt_tensor_view(h.ptr, 2, i64([4, 6]), i64([1, 4]), 0)))
    out = np.empty((4, 6), dtype=np.float32)
    assert _C.lib.gt_tensor_copy_to_host(v.ptr, out.ctypes.data_as(ctypes.c_void_p), out.nbytes) == 0
    assert np.array_equal(out, data.reshape(6, 4).T)
    # dtype conversion rounds like the reference writes (float -> half RNE)
    x = torch.randn(5, 7)
    hx = _bridge.borrow(x)  # the handle must outlive the calls that use it
    y = _bridge.adopt(_C.lib.gt_tensor_to_dtype(hx.ptr, _C.GT_F16))
    assert torch.equal(y, x.half())
    y = _bridge.adopt(_C.lib.gt_tensor_to_dtype(hx.ptr, _C.GT_BF16))
    assert torch.equal(y, x.bfloat16())
    # strided borrowed input, clone is dense
    xt = x.t()
    hxt = _bridge.borrow(xt)
    c = _bridge.adopt(_C.lib.gt_tensor_clone(hxt.ptr))
    assert torch.equal(c, xt) and c.is_contiguous()


def test_external_memory_token_is_reported_on_release():
    toks = (ctypes.c_uint64 * 64)()
    while _C.lib.gt_external_released(toks, 64):  # drop the tokens of earlier borrows
        pass
    buf = np.zeros(8, dtype=np.float64)
    p = _C.lib.gt_tensor_from_external(1, i64([8]), i64([1]), _C.GT_F64, buf.ctypes.data_as(ctypes.c_void_p), 4242)
    _C.check_ptr(p)
    view = _C.lib.gt_tensor_view(p, 1, i64([4]), i64([2]), 0)
    _C.lib.gt_tensor_free(p)
    assert _C.lib.gt_external_released(toks, 4) == 0  # the view still holds the memory
    _C.lib.gt_tensor_free(view)
    n = _C.lib.gt_external_released(toks, 4)
    assert n == 1 and toks[0] == 4242


def test_invalid_arguments_fail_with_a_message():
    assert not _C.lib.gt_tensor_empty(13, i64([1] * 13), _C.GT_F32, _C.GT_DEV_CPU, 0)
    assert "ndim" in _C.last_error()
    assert not _C.lib.gt_tensor_empty(1, i64([-1]), _C.GT_F32, _C.GT_DEV_CPU, 0)
    assert "Negative" in _C.last_error()
    assert not _C.lib.gt_tensor_empty(1, i64([4]), 10, _C.GT_DEV_CPU, 0)  # complex64
    assert "not supported" in _C.last_error()
    h = _bridge.borrow(torch.zeros(4))
    assert not _C.lib.gt_tensor_view(h.ptr, 1, i64([5]), i64([1]), 0)
    assert "outside the storage" in _C.last_error()
    assert not _C.lib.gt_flash_attention(None, None, None, None, ctypes.c_float(0), 0)
    assert _C.last_error() == "flash_attention expects 4D q, k, v tensors (B, H, L, D)"
    buf = np.zeros(4, np.float32)
    assert not _C.lib.gt_tensor_from_external(1, i64([4]), i64([1]), _C.GT_F32, buf.ctypes.data_as(ctypes.c_void_p), 0)
    assert "token" in _C.last_error()


def test_allocation_failure_is_reported(monkeypatch):
    monkeypatch.setenv("GT_ATTN_FAIL_ALLOC", "1")
    assert not _C.lib.gt_tensor_empty(1, i64([16]), _C.GT_F32, _C.GT_DEV_CPU, 0)
    assert "out of memory" in _C.last_error()
    h = _bridge.borrow(torch.zeros(3))
    with pytest.raises(RuntimeError, match="out of memory"):
        _bridge.adopt(_C.lib.gt_tensor_clone(h.ptr), "clone")
    monkeypatch.delenv("GT_ATTN_FAIL_ALLOC")
    assert _C.lib.gt_tensor_empty(1, i64([16]), _C.GT_F32, _C.GT_DEV_CPU, 0)


def test_shape_errors_match_the_reference_text():
    q, k, v = torch.randn(2, 3, 4, 6), torch.randn(2, 3, 5, 6), torch.randn(2, 3, 5, 6)
    # tests/test_pooling_and_attention.py:375-386
    for shape in ((2, 3), (4, 6), (7, 4, 5), (2, 3, 4, 5, 1)):
        with pytest.raises(RuntimeError, match="cannot be broadcast"):
            F.scaled_dot_product_attention(q, k, v, attn_mask=torch.ones(*shape, dtype=torch.bool))
    for shape in ((2, 3), (5,), (2, 4, 5)):
        with pytest.raises(RuntimeError, match="cannot be broadcast"):
            g.FlashAttentionFn.apply(q, k, v, torch.ones(*shape, dtype=torch.bool), 0.4, False)
    with pytest.raises(RuntimeError, match="num_heads must be divisible by num_kv_heads"):
        g.flash_attention(torch.randn(1, 3, 4, 8), torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8))
    with pytest.raises(RuntimeError, match="do not fit together"):
        g.flash_attention(torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 7), torch.randn(1, 2, 4, 8))


def test_dropout_probability_is_checked_first():
    q = torch.randn(1, 1, 2, 4)
    for p in (-0.1, 1.5, float("nan")):
        with pytest.raises(RuntimeError, match="dropout probability has to be between 0 and 1"):
            g.flash_attention_dropout(q, q, q, None, 0.0, False, p, 1)
        with pytest.raises(RuntimeError, match="dropout probability has to be between 0 and 1"):
            g.attention_dropout_mask((1, 1, 2, 2), p, 1, device="cuda:0")


@pytest.mark.skipif(_C.device_count() > 0, reason="checks the behaviour without a HIP device")
def test_compute_without_a_device_fails_loudly():
    q = torch.randn(1, 1, 2, 4)
    with pytest.raises(RuntimeError, match="no HIP device"):
        g.flash_attention(q, q, q)
    with pytest.raises(RuntimeError, match="no HIP device"):
        g.quantize(torch.randn(64))
    with pytest.raises(RuntimeError, match="no HIP device"):
        g.flash_attention_dropout(q, q, q, None, 0.0, False, 0.5, 1)


def test_library_matches_the_sources_beside_it():
    # the loaded library carries the fingerprint of the sources it was built from
    from gguf_train_amd._srchash import source_hash

    assert _C.lib.gt_source_hash().decode() == source_hash()

    class Stale:
        class gt_source_hash:  # a library built from other sources
            argtypes = restype = None

            def __new__(cls):
                return b"0" * 64

    with pytest.raises(ImportError, match="built from other sources"):
        _C._check_sources(Stale)
