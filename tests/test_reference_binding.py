"""libgt_attn.so bound the way the reference's ctypes loader binds its own library
(gguf_train/_C.py:226-309 lifecycle, :467-472 RoPE and attention, :527-558 GGUF read side and
Q8_0 codec): a fresh CDLL with exactly those argtypes / restypes, then calls that need no GPU -
host tensors in and out, the thread-local error text, the GGUF reader - and the compute entry
points failing cleanly (NULL + message) on a host without a HIP device.  This is the drop-in
claim: the reference's loader needs no change to call this library."""

import ctypes
import struct
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_uint64, c_void_p

import numpy as np
import pytest

from gguf_train_amd import _C

import _gguf_file as gf
from _gguf_file import GGUFBuilder

p_i64, p_vp = POINTER(c_int64), POINTER(c_void_p)

# name: (argtypes, restype) as declared by the reference loader (file:line of gguf_train/_C.py)
REFERENCE_BINDINGS = {
    "gt_init": ([], None),                                                            # :226-227
    "gt_last_error": ([], c_char_p),                                                  # :250-251
    "gt_tensor_from_data": ([c_int, p_i64, c_int, c_int, c_int, c_void_p, c_size_t], c_void_p),  # :258-259
    "gt_tensor_free": ([c_void_p], None),                                             # :270-271
    "gt_tensor_ndim": ([c_void_p], c_int),                                            # :273-274
    "gt_tensor_shape": ([c_void_p, p_i64], None),                                     # :275-276
    "gt_tensor_dtype": ([c_void_p], c_int),                                           # :283-284
    "gt_tensor_from_external": ([c_int, p_i64, p_i64, c_int, c_void_p, c_uint64], c_void_p),  # :299-300
    "gt_external_released": ([POINTER(c_uint64), c_int64], c_int64),                  # :301-302
    "gt_tensor_copy_to_host": ([c_void_p, c_void_p, c_size_t], c_int),                # :308-309
    "gt_rope": ([c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_float], c_void_p),           # :467-468
    "gt_rope_backward": ([c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_float], c_void_p),  # :469-470
    "gt_flash_attention": ([c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int], c_void_p),   # :471-472
    "gt_gguf_open": ([c_char_p], c_void_p),                                           # :527-528
    "gt_gguf_close": ([c_void_p], None),                                              # :529-530
    "gt_gguf_n_tensors": ([c_void_p], c_int64),                                       # :531-532
    "gt_gguf_tensor_name": ([c_void_p, c_int64], c_char_p),                           # :533-534
    "gt_gguf_get_tensor": ([c_void_p, c_char_p, c_int], c_void_p),                    # :535-536
    "gt_gguf_n_kv": ([c_void_p], c_int64),                                            # :537-538
    "gt_gguf_kv_key": ([c_void_p, c_int64], c_char_p),                                # :539-540
    "gt_gguf_kv_type": ([c_void_p, c_int64], c_int),                                  # :541-542
    "gt_gguf_kv_val_str": ([c_void_p, c_int64, c_char_p, c_int], c_int),              # :543-544
    "gt_gguf_kv_arr_type": ([c_void_p, c_int64], c_int),                              # :547-548
    "gt_gguf_kv_arr_n": ([c_void_p, c_int64], c_int64),                               # :549-550
    "gt_gguf_kv_arr_data": ([c_void_p, c_int64], c_void_p),                           # :551-552
    "gt_gguf_kv_arr_str": ([c_void_p, c_int64, c_int64], c_char_p),                   # :553-554
    "gt_quantize": ([c_void_p, c_int], c_void_p),                                     # :555-556
    "gt_dequantize": ([c_void_p, c_int], c_void_p),                                   # :557-558
}


@pytest.fixture(scope="module")
def ref():
    """A second, independent CDLL of the library, configured only with the reference's types."""
    lib = ctypes.CDLL(str(_C.LIB_PATH))
    for name, (args, res) in REFERENCE_BINDINGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    lib.gt_init()
    return lib


def _i64(vals):
    return (c_int64 * max(len(vals), 1))(*vals)


def _host(ref, arr, code):
    arr = np.ascontiguousarray(arr)
    p = ref.gt_tensor_from_data(arr.ndim, _i64(arr.shape), code, 0, 0, arr.ctypes.data_as(c_void_p), arr.nbytes)
    assert p, ref.gt_last_error()
    return p


def test_host_tensors_through_the_reference_types(ref):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    h = _host(ref, a, 0)
    assert ref.gt_tensor_ndim(h) == 2 and ref.gt_tensor_dtype(h) == 0
    shape = _i64([0, 0])
    ref.gt_tensor_shape(h, shape)
    assert list(shape) == [3, 4]
    out = np.empty_like(a)
    assert ref.gt_tensor_copy_to_host(h, out.ctypes.data_as(c_void_p), out.nbytes) == 0
    assert np.array_equal(out, a)
    # borrowed host memory (no copy) and its release token
    b = np.arange(6, dtype=np.float64)
    e = ref.gt_tensor_from_external(1, _i64([6]), _i64([1]), 3, b.ctypes.data_as(c_void_p), 4242)
    assert e
    ref.gt_tensor_free(e)
    toks = (c_uint64 * 64)()
    n = ref.gt_external_released(toks, 64)
    assert 4242 in list(toks[:n])
    ref.gt_tensor_free(h)


def test_gguf_reader_through_the_reference_types(ref, tmp_path):
    p = (GGUFBuilder()
         .kv("general.name", gf.STRING, "binding")
         .kv("n", gf.U32, 7)
         .kv("xs", gf.ARRAY, [1.5, -2.0], elem=gf.F32)
         .tensor("w", [2, 2], gf.T_F32, struct.pack("<4f", 1, 2, 3, 4))
         .write(tmp_path / "b.gguf"))
    f = ref.gt_gguf_open(str(p).encode())
    assert f, ref.gt_last_error()
    try:
        assert ref.gt_gguf_n_tensors(f) == 1 and ref.gt_gguf_tensor_name(f, 0) == b"w"
        keys = {ref.gt_gguf_kv_key(f, i): i for i in range(ref.gt_gguf_n_kv(f))}
        i = keys[b"n"]
        buf = ctypes.create_string_buffer(16)
        assert ref.gt_gguf_kv_val_str(f, i, buf, 16) == 1 and buf.value == b"7"
        j = keys[b"xs"]
        assert ref.gt_gguf_kv_arr_type(f, j) == gf.F32 and ref.gt_gguf_kv_arr_n(f, j) == 2
        vals = ctypes.cast(ref.gt_gguf_kv_arr_data(f, j), POINTER(c_float * 2)).contents[:]
        assert vals == [1.5, -2.0]
        t = ref.gt_gguf_get_tensor(f, b"w", 0)
        assert t, ref.gt_last_error()
        out = np.empty((2, 2), np.float32)
        assert ref.gt_tensor_copy_to_host(t, out.ctypes.data_as(c_void_p), out.nbytes) == 0
        assert out.tolist() == [[1.0, 2.0], [3.0, 4.0]]
        ref.gt_tensor_free(t)
    finally:
        ref.gt_gguf_close(f)
    assert not ref.gt_gguf_open(str(tmp_path / "missing.gguf").encode())
    assert b"Failed to open GGUF file" in ref.gt_last_error()


def test_compute_entry_points_fail_cleanly_without_a_device(ref):
    # argument errors come first, with the reference's text
    q = _host(ref, np.zeros((1, 2, 3, 4), np.float32), 0)
    k = _host(ref, np.zeros((1, 2, 5, 4), np.float32), 0)
    bad = _host(ref, np.zeros((2, 3, 5), np.float32), 0)
    assert not ref.gt_flash_attention(q, k, k, bad, c_float(0.0), 0)
    assert b"cannot be broadcast to the attention weights [1, 2, 3, 5]" in ref.gt_last_error()
    if _C.device_count() == 0:
        # no HIP device here: the computation itself is refused with a message, never run on the CPU
        assert not ref.gt_flash_attention(q, k, k, None, c_float(0.0), 1)
        assert b"no HIP device" in ref.gt_last_error()
        assert not ref.gt_quantize(_host(ref, np.zeros((2, 32), np.float32), 0), 8)
        assert b"no HIP device" in ref.gt_last_error()
    for h in (q, k, bad):
        ref.gt_tensor_free(h)
