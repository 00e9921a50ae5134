"""GGUF reader on the host: files built byte by byte (tests/_gguf_file.py) read back with the
reference's shape and dtype rules (csrc/gt_ops_extra.cpp:1846-1918), metadata of every value
type (csrc/gt_ops_extra.cpp:1936-1990, gguf_train/gguf/__init__.py:36-66), and files ggml's reader
refuses failing with "Failed to open GGUF file" instead of giving a wrong tensor.  The cases
follow the reference's tests/test_gguf_roundtrip.py (files from other writers, recorded dtype,
inconsistent records, metadata written by another tool, long strings)."""

import ctypes
import math
import struct

import numpy as np
import pytest
import torch

import oracle
from gguf_train_amd import _C, _bridge
from gguf_train_amd.gguf import GGUFFile, inspect_gguf, load_gguf

import _gguf_file as gf
from _gguf_file import GGUFBuilder


def f32s(*v):
    return struct.pack(f"<{len(v)}f", *v)


def test_files_from_other_writers(tmp_path):
    p = (GGUFBuilder()
         .kv("general.name", gf.STRING, "foreign")
         .tensor("m", [3, 2], gf.T_F32, f32s(*range(6)))
         .tensor("b", [4], gf.T_I8, struct.pack("<4b", -1, 0, 1, 127))
         .write(tmp_path / "foreign.gguf"))
    loaded = load_gguf(p)
    assert loaded["m"].tolist() == [[0.0, 1.0, 2.0], [3.0, 4.0, 5.0]]
    assert loaded["b"].dtype == torch.int8 and loaded["b"].tolist() == [-1, 0, 1, 127]
    assert loaded.metadata == {"general.name": "foreign"}
    assert list(loaded.keys()) == ["m", "b"] and len(loaded) == 2 and "m" in loaded


def test_gguf_files_compare_and_hash_by_identity(tmp_path):
    # the reference's GGUFFile is a plain class (gguf_train/gguf/__init__.py:69): identity
    # equality, hashable - two readings of one file are two objects
    p = GGUFBuilder().tensor("m", [4], gf.T_F32, f32s(1, 2, 3, 4)).write(tmp_path / "eq.gguf")
    a, b = load_gguf(p), load_gguf(p)
    assert a == a and a != b
    assert len({a, b, a}) == 2 and {a: 1}[a] == 1


def test_every_plain_type_and_natural_shapes(tmp_path):
    rng = np.random.default_rng(1)
    cases = {
        "f32": (gf.T_F32, rng.standard_normal(24).astype(np.float32), torch.float32),
        "f16": (gf.T_F16, rng.standard_normal(24).astype(np.float16), torch.float16),
        "f64": (gf.T_F64, rng.standard_normal(24), torch.float64),
        "i16": (gf.T_I16, rng.integers(-30000, 30000, 24).astype(np.int16), torch.int16),
        "i32": (gf.T_I32, rng.integers(-2**31, 2**31 - 1, 24).astype(np.int32), torch.int32),
        "i64": (gf.T_I64, rng.integers(-2**62, 2**62, 24).astype(np.int64), torch.int64),
    }
    b = GGUFBuilder()
    for name, (tt, arr, _) in cases.items():
        b.tensor(name, [4, 3, 2], tt, arr.tobytes())
    bf = oracle.f32_to_bf16_bits(rng.standard_normal(8).astype(np.float32))
    b.tensor("bf16", [8], gf.T_BF16, bf.astype(np.uint16).tobytes())
    b.tensor("trailing_ones", [5, 1, 1], gf.T_F32, f32s(*range(5)))
    b.tensor("outer_one", [1, 3], gf.T_F32, f32s(1, 2, 3))
    b.tensor("empty", [0], gf.T_F32, b"")
    loaded = load_gguf(b.write(tmp_path / "types.gguf"))
    for name, (_, arr, dt) in cases.items():
        t = loaded[name]
        assert t.dtype == dt and t.shape == (2, 3, 4)
        assert np.array_equal(t.numpy().reshape(-1), arr)
    assert loaded["bf16"].dtype == torch.bfloat16
    assert np.array_equal(loaded["bf16"].view(torch.int16).numpy().view(np.uint16), bf.astype(np.uint16))
    assert loaded["trailing_ones"].shape == (5,)
    assert loaded["outer_one"].shape == (3, 1)
    assert loaded["empty"].shape == (0,)


def test_recorded_dtype_and_shape_are_applied(tmp_path):
    p = (GGUFBuilder()
         .kv("gguf_train.dtype.u", gf.STRING, "uint8")
         .kv("gguf_train.dtype.f", gf.STRING, "bool")
         .kv("gguf_train.shape.s", gf.ARRAY, [], gf.I64)
         .kv("gguf_train.shape.r", gf.ARRAY, [2, 1, 3, 1, 1, 2], gf.I64)
         .kv("user", gf.I32, 7)
         .tensor("u", [3], gf.T_I8, bytes([1, 200, 255]))
         .tensor("f", [2], gf.T_I8, bytes([0, 1]))
         .tensor("s", [1], gf.T_F32, f32s(2.5))
         .tensor("r", [12], gf.T_F32, f32s(*range(12)))
         .write(tmp_path / "typed.gguf"))
    loaded = load_gguf(p)
    assert loaded["u"].dtype == torch.uint8 and loaded["u"].tolist() == [1, 200, 255]
    assert loaded["f"].dtype == torch.bool and loaded["f"].tolist() == [False, True]
    assert loaded["s"].shape == () and loaded["s"].item() == 2.5
    assert loaded["r"].shape == (2, 1, 3, 1, 1, 2)
    assert loaded["r"].reshape(-1).tolist() == list(map(float, range(12)))
    # the recording keys are not metadata
    assert loaded.metadata == {"user": 7}


@pytest.mark.parametrize("label,kvs", [
    ("shape", [("gguf_train.shape.t", gf.ARRAY, [3, 3], gf.I64)]),
    ("negative", [("gguf_train.shape.t", gf.ARRAY, [-2, -2], gf.I64)]),
    ("shape type", [("gguf_train.shape.t", gf.STRING, "2,2", None)]),
    ("shape elements", [("gguf_train.shape.t", gf.ARRAY, [2, 2], gf.I32)]),
    ("too many dims", [("gguf_train.shape.t", gf.ARRAY, [1] * 13, gf.I64)]),
    ("carrier", [("gguf_train.dtype.t", gf.STRING, "bool", None)]),
    ("unknown dtype", [("gguf_train.dtype.t", gf.STRING, "float128", None)]),
    ("dtype type", [("gguf_train.dtype.t", gf.U32, 9, None)]),
])
def test_inconsistent_records_are_an_error(tmp_path, label, kvs):
    b = GGUFBuilder()
    for key, vt, val, elem in kvs:
        b.kv(key, vt, val, elem)
    p = b.tensor("t", [4], gf.T_F32, f32s(1, 2, 3, 4)).write(tmp_path / "bad.gguf")
    with pytest.raises(RuntimeError, match="tensor 't'"):
        load_gguf(p)


def test_complex_records(tmp_path):
    odd = (GGUFBuilder().kv("gguf_train.dtype.t", gf.STRING, "complex64", None)
           .tensor("t", [3], gf.T_F32, f32s(1, 2, 3)).write(tmp_path / "odd.gguf"))
    with pytest.raises(RuntimeError, match="even number"):
        load_gguf(odd)
    even = (GGUFBuilder().kv("gguf_train.dtype.t", gf.STRING, "complex64", None)
            .tensor("t", [2, 2], gf.T_F32, f32s(1, 2, 3, 4)).write(tmp_path / "even.gguf"))
    with pytest.raises(RuntimeError, match="complex tensors are not supported"):
        load_gguf(even)


def test_metadata_of_every_type(tmp_path):
    template = "{% for m in messages %}" + "x" * 5000 + "{% endfor %}"
    p = (GGUFBuilder()
         .kv("u8", gf.U8, 255).kv("i8", gf.I8, -128).kv("u16", gf.U16, 65535).kv("i16", gf.I16, -32768)
         .kv("u32", gf.U32, 2**32 - 1).kv("i32", gf.I32, -2**31).kv("u64", gf.U64, 2**64 - 1)
         .kv("i64", gf.I64, -2**63).kv("f32", gf.F32, 0.1).kv("f64", gf.F64, math.pi)
         .kv("t", gf.BOOL, True).kv("f", gf.BOOL, False).kv("s", gf.STRING, "héllo")
         .kv("long", gf.STRING, template)
         .kv("ints", gf.ARRAY, [1, -2, 3], gf.I32).kv("u64s", gf.ARRAY, [2**64 - 1, 0], gf.U64)
         .kv("floats", gf.ARRAY, [0.5, -1.25], gf.F32).kv("bools", gf.ARRAY, [True, False, True], gf.BOOL)
         .kv("strs", gf.ARRAY, ["<unk>", "", "▁w0"], gf.STRING).kv("none", gf.ARRAY, [], gf.I32)
         .tensor("x", [2], gf.T_F32, f32s(1, 2))
         .write(tmp_path / "meta.gguf"))
    md = load_gguf(p).metadata
    assert md["u8"] == 255 and md["i8"] == -128 and md["u16"] == 65535 and md["i16"] == -32768
    assert md["u32"] == 2**32 - 1 and md["i32"] == -2**31 and md["u64"] == 2**64 - 1 and md["i64"] == -2**63
    assert md["f32"] == float(np.float32(0.1)) and md["f64"] == math.pi
    assert md["t"] is True and md["f"] is False and md["s"] == "héllo"
    assert md["long"] == template
    assert md["ints"] == [1, -2, 3] and md["u64s"] == [2**64 - 1, 0]
    assert md["floats"] == [0.5, -1.25] and md["bools"] == [True, False, True]
    assert md["strs"] == ["<unk>", "", "▁w0"] and md["none"] == []
    assert list(md)[:4] == ["u8", "i8", "u16", "i16"]


def test_value_text_is_cut_like_snprintf(tmp_path):
    p = GGUFBuilder().kv("s", gf.STRING, "abcdef").kv("n", gf.I32, -12345).kv(
        "a", gf.ARRAY, [1, 2], gf.I32).write(tmp_path / "cut.gguf")
    h = _C.check_ptr(_C.lib.gt_gguf_open(str(p).encode()))
    try:
        buf = ctypes.create_string_buffer(4)
        assert _C.lib.gt_gguf_kv_val_str(h, 0, buf, 4) == 6 and buf.value == b"abc"
        assert _C.lib.gt_gguf_kv_val_str(h, 1, None, 0) == 6
        assert _C.lib.gt_gguf_kv_val_str(h, 1, buf, 4) == 6 and buf.value == b"-12"
        big = ctypes.create_string_buffer(64)
        assert _C.lib.gt_gguf_kv_val_str(h, 2, big, 64) == len("<array len=2>") and big.value == b"<array len=2>"
        assert _C.lib.gt_gguf_kv_val_str(h, 3, big, 64) == -1
        assert _C.lib.gt_gguf_kv_type(h, 2) == gf.ARRAY and _C.lib.gt_gguf_kv_type(h, 9) == -1
        assert _C.lib.gt_gguf_kv_arr_type(h, 2) == gf.I32 and _C.lib.gt_gguf_kv_arr_type(h, 0) == -1
        assert _C.lib.gt_gguf_kv_arr_n(h, 2) == 2 and _C.lib.gt_gguf_kv_arr_n(h, 1) == -1
        assert _C.lib.gt_gguf_kv_arr_str(h, 2, 0) is None and _C.lib.gt_gguf_kv_key(h, 3) is None
        assert _C.lib.gt_gguf_tensor_name(h, 0) is None and _C.lib.gt_gguf_n_tensors(h) == 0
    finally:
        _C.lib.gt_gguf_close(h)


def test_q8_0_blocks_are_read_as_stored(tmp_path):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    blocks = oracle.q8_0_quantize(x)
    p = GGUFBuilder().tensor("kq", [64, 3], gf.T_Q8_0, blocks.tobytes()).write(tmp_path / "q8.gguf")
    t = load_gguf(p)["kq"]
    assert isinstance(t, _bridge.QuantizedTensor) and t.shape == (3, 64)
    assert t.data.device.type == "cpu" and np.array_equal(t.data.numpy(), blocks)
    info = inspect_gguf(p)
    assert info["n_tensors"] == 1 and info["tensors"]["kq"] == {"shape": (3, 64), "dtype": "q8_0"}


def test_other_quantized_types_are_refused_by_name(tmp_path):
    p = (GGUFBuilder().tensor("ok", [2], gf.T_F32, f32s(1, 2))
         .tensor("w4", [32], gf.T_Q4_0, bytes(18)).write(tmp_path / "q4.gguf"))
    h = _C.check_ptr(_C.lib.gt_gguf_open(str(p).encode()))
    try:
        assert _C.lib.gt_gguf_n_tensors(h) == 2 and _C.lib.gt_gguf_tensor_name(h, 1) == b"w4"
        ok = _bridge.adopt(_C.lib.gt_gguf_get_tensor(h, b"ok", 0))
        assert ok.tolist() == [1.0, 2.0]
        assert not _C.lib.gt_gguf_get_tensor(h, b"w4", 0)
        assert "q4_0 is not supported" in _C.last_error()
        assert not _C.lib.gt_gguf_get_tensor(h, b"missing", 0)
        assert _C.last_error() == "gguf: no tensor named 'missing'"
    finally:
        _C.lib.gt_gguf_close(h)


def test_alignment_and_version_two(tmp_path):
    b = GGUFBuilder(version=2, alignment=64).kv("general.alignment", gf.U32, 64)
    b.tensor("a", [3], gf.T_F32, f32s(1, 2, 3)).tensor("b", [5], gf.T_F32, f32s(*range(5)))
    loaded = load_gguf(b.write(tmp_path / "a64.gguf"))
    assert loaded["b"].tolist() == [0.0, 1.0, 2.0, 3.0, 4.0]
    assert loaded.metadata == {"general.alignment": 64}


def _refused(tmp_path, data: bytes, why: str):
    p = tmp_path / "refused.gguf"
    p.write_bytes(data)
    with pytest.raises(RuntimeError, match="Failed to open GGUF file") as e:
        GGUFFile(p)
    assert why in str(e.value)


def test_files_ggml_refuses_fail_to_open(tmp_path):
    one = lambda: GGUFBuilder().tensor("t", [4], gf.T_F32, f32s(1, 2, 3, 4))  # noqa: E731
    _refused(tmp_path, b"GGUX" + one().to_bytes()[4:], "bad magic")
    _refused(tmp_path, GGUFBuilder(version=1).to_bytes(), "GGUFv1")
    _refused(tmp_path, GGUFBuilder(version=4).to_bytes(), "version 4")
    _refused(tmp_path, one().to_bytes(truncate=4), "data section")
    _refused(tmp_path, one().to_bytes()[:30], "truncated")
    _refused(tmp_path, GGUFBuilder().tensor("t", [4], gf.T_F32, f32s(1, 2, 3, 4), offset=32).to_bytes(),
             "has offset 32, expected 0")
    _refused(tmp_path, one().tensor("t", [1], gf.T_F32, f32s(1)).to_bytes(), "duplicate tensor name 't'")
    _refused(tmp_path, GGUFBuilder().kv("k", gf.I32, 1).kv("k", gf.I32, 2).to_bytes(), "duplicate key 'k'")
    _refused(tmp_path, GGUFBuilder().tensor("n" * 64, [1], gf.T_F32, f32s(1)).to_bytes(), "64 bytes long")
    _refused(tmp_path, GGUFBuilder().tensor("t", [1] * 5, gf.T_F32, f32s(1)).to_bytes(), "5 dimensions")
    _refused(tmp_path, GGUFBuilder().tensor("t", [16], gf.T_Q8_0, bytes(17)).to_bytes(), "block size 32")
    _refused(tmp_path, GGUFBuilder().tensor("t", [4], 4, bytes(16)).to_bytes(), "unknown ggml type 4")
    _refused(tmp_path, GGUFBuilder().tensor("t", [4], 99, bytes(16)).to_bytes(), "unknown ggml type 99")
    _refused(tmp_path, one().kv("general.alignment", gf.I64, 32).to_bytes(), "general.alignment is not a u32")
    _refused(tmp_path, GGUFBuilder(alignment=48).kv("general.alignment", gf.U32, 48).to_bytes(), "power of two")
    _refused(tmp_path, GGUFBuilder().kv("k", gf.ARRAY, [], gf.ARRAY).to_bytes(), "element type 9")
    with pytest.raises(RuntimeError, match="Failed to open GGUF file"):
        GGUFFile(tmp_path / "does-not-exist.gguf")
    with pytest.raises(RuntimeError, match="not a regular file"):
        GGUFFile(tmp_path)


def test_device_argument_is_checked(tmp_path):
    p = GGUFBuilder().tensor("t", [2], gf.T_F32, f32s(1, 2)).write(tmp_path / "d.gguf")
    with pytest.raises(ValueError, match="only 'cpu' and HIP"):
        load_gguf(p, device="meta")
    assert load_gguf(p, device="cpu")["t"].tolist() == [1.0, 2.0]
