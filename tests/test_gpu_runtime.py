"""The C ABI's runtime queries and tensor-lifecycle calls on device tensors, with the reference's
semantics: runtime / errors (csrc/gguf_train.h:170-186), gt_tensor_contiguous
(csrc/gt_core.cpp:769-781: a view when already dense, else a dense copy), gt_tensor_copy_from_host
(csrc/gt_core.cpp:947-985: honours the destination's offset and strides) and
gt_tensor_copy_inplace (csrc/gt_core.cpp:987-1060: broadcast from the right, dtype conversion)."""

import ctypes

import numpy as np
import pytest
import torch

from gguf_train_amd import _bridge, _C

pytestmark = pytest.mark.gpu

lib = _C.lib


def i64(vals):
    return (ctypes.c_int64 * max(len(vals), 1))(*vals)


def on_device(arr, code):
    arr = np.ascontiguousarray(arr)
    p = lib.gt_tensor_from_data(arr.ndim, i64(arr.shape), code, _C.GT_DEV_CUDA, 0,
                                arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)
    return _bridge.Handle(_C.check_ptr(p, "from_data"))


def view(h, shape, strides, offset):
    return _bridge.Handle(_C.check_ptr(lib.gt_tensor_view(h.ptr, len(shape), i64(shape), i64(strides), offset), "view"))


def to_host(h, shape, np_dtype):
    out = np.empty(shape, np_dtype)
    assert lib.gt_tensor_copy_to_host(h.ptr, out.ctypes.data_as(ctypes.c_void_p), out.nbytes) == 0, _C.last_error()
    return out


def test_runtime_queries_errors_and_stream(dev):
    lib.gt_init()
    lib.gt_init()  # idempotent
    assert lib.gt_device_count(_C.GT_DEV_CUDA) >= 1
    assert lib.gt_device_count(_C.GT_DEV_CPU) == 1
    name = ctypes.create_string_buffer(256)
    lib.gt_device_name(_C.GT_DEV_CUDA, 0, name, 256)
    assert name.value
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    lib.gt_device_memory(_C.GT_DEV_CUDA, 0, ctypes.byref(free), ctypes.byref(total))
    assert 0 < free.value <= total.value
    # a library layered on top records its own failure as this thread's last error
    lib.gt_set_last_error(b"layered library: something failed")
    assert _C.last_error() == "layered library: something failed"
    lib.gt_clear_error()
    assert not _C.last_error()
    # the stream this thread's calls enqueue on
    old = lib.gt_get_stream()
    s = torch.cuda.Stream(device=dev)
    lib.gt_set_stream(ctypes.c_void_p(s.cuda_stream))
    try:
        assert lib.gt_get_stream() == s.cuda_stream
        h = on_device(np.arange(6, dtype=np.float32), _C.GT_F32)  # work enqueued on s, then read back
        assert np.array_equal(to_host(h, (6,), np.float32), np.arange(6, dtype=np.float32))
    finally:
        lib.gt_set_stream(ctypes.c_void_p(old))
    assert lib.gt_get_stream() == old


def test_device_tensor_metadata(dev):
    for code, size in ((_C.GT_F32, 4), (_C.GT_F16, 2), (_C.GT_BF16, 2), (_C.GT_F64, 8), (_C.GT_I32, 4),
                       (_C.GT_I64, 8), (_C.GT_BOOL, 1)):
        assert lib.gt_tensor_elem_size(code) == size
    h = on_device(np.arange(24, dtype=np.float32).reshape(2, 3, 4), _C.GT_F32)
    assert lib.gt_tensor_device_type(h.ptr) == _C.GT_DEV_CUDA
    assert lib.gt_tensor_device_index(h.ptr) == 0
    assert lib.gt_tensor_storage_nbytes(h.ptr) >= 96
    v = view(h, (3,), (4,), 5)  # a view shares the storage
    assert lib.gt_tensor_storage_nbytes(v.ptr) == lib.gt_tensor_storage_nbytes(h.ptr)
    assert lib.gt_tensor_data_ptr(v.ptr) == lib.gt_tensor_data_ptr(h.ptr) + 5 * 4


def test_copy_from_host_honours_the_views_offset_and_strides(dev):
    base = on_device(np.zeros((4, 6), np.float32), _C.GT_F32)
    v = view(base, (3, 2), (6, 2), 1)  # element (r, c) at 1 + 6 r + 2 c
    src = np.arange(1, 7, dtype=np.float32).reshape(3, 2)
    assert lib.gt_tensor_copy_from_host(v.ptr, src.ctypes.data_as(ctypes.c_void_p), src.nbytes) == 0
    want = np.zeros(24, np.float32)
    for r in range(3):
        for c in range(2):
            want[1 + 6 * r + 2 * c] = src[r, c]
    assert np.array_equal(to_host(base, (4, 6), np.float32), want.reshape(4, 6))
    # fewer source bytes than the view holds: an error, nothing written
    assert lib.gt_tensor_copy_from_host(v.ptr, src.ctypes.data_as(ctypes.c_void_p), 8) != 0
    assert _C.last_error()
    assert np.array_equal(to_host(base, (4, 6), np.float32), want.reshape(4, 6))


def test_copy_inplace_broadcasts_and_converts(dev):
    dst = on_device(np.zeros((2, 3, 4), np.float16), _C.GT_F16)
    col = np.array([[1.5], [2.25], [-3.125]], np.float32)  # (3, 1) broadcast over (2, 3, 4)
    src = on_device(col, _C.GT_F32)
    assert lib.gt_tensor_copy_inplace(dst.ptr, src.ptr) == 0, _C.last_error()
    assert np.array_equal(to_host(dst, (2, 3, 4), np.float16), np.broadcast_to(col, (2, 3, 4)).astype(np.float16))
    # a transposed source of the same shape, float64 -> float32 (rounded once)
    a = np.random.default_rng(0).standard_normal((4, 3))
    src64 = on_device(a, _C.GT_F64)
    srcT = view(src64, (3, 4), (1, 3), 0)
    dst2 = on_device(np.zeros((3, 4), np.float32), _C.GT_F32)
    assert lib.gt_tensor_copy_inplace(dst2.ptr, srcT.ptr) == 0, _C.last_error()
    assert np.array_equal(to_host(dst2, (3, 4), np.float32), a.T.astype(np.float32))
    # shapes that do not broadcast
    bad = on_device(np.zeros(5, np.float32), _C.GT_F32)
    assert lib.gt_tensor_copy_inplace(dst.ptr, bad.ptr) != 0
    assert "broadcast" in _C.last_error()


def test_contiguous_copies_a_view_and_shares_a_dense_tensor(dev):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    h = on_device(a, _C.GT_F32)
    t = view(h, (4, 3), (1, 4), 0)
    c = _bridge.Handle(_C.check_ptr(lib.gt_tensor_contiguous(t.ptr), "contiguous"))
    assert lib.gt_tensor_is_contiguous(c.ptr) == 1
    assert lib.gt_tensor_data_ptr(c.ptr) != lib.gt_tensor_data_ptr(h.ptr)
    assert np.array_equal(to_host(c, (4, 3), np.float32), a.T)
    d = _bridge.Handle(_C.check_ptr(lib.gt_tensor_contiguous(h.ptr), "contiguous"))
    assert lib.gt_tensor_data_ptr(d.ptr) == lib.gt_tensor_data_ptr(h.ptr)  # already dense: a view
