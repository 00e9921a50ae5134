"""ctypes loader of libgt_attn.so.

Same conventions as the reference's loader (gguf_train/_C.py): one CDLL with its argtypes and
restypes declared up front, `check_ptr` / `check_rc` turning a NULL / non-zero native result
into a Python exception built from the thread-local `gt_last_error()`, and the
"IndexError: " message prefix mapping to IndexError (gguf_train/_C.py:680-710).

The library is built in-tree (python gguf_train_amd/_build.py).  Importing this module never
builds, downloads or falls back to anything: a missing library is an ImportError.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_uint64, c_void_p
from pathlib import Path

_PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = _PKG_DIR / "libgt_attn.so"

# dtype / device codes (csrc/gguf_train.h:22-44)
GT_F32, GT_F16, GT_BF16, GT_F64 = 0, 1, 2, 3
GT_I8, GT_U8, GT_I16, GT_I32, GT_I64, GT_BOOL = 4, 5, 6, 7, 8, 9
GT_Q_BASE = 100
GT_Q8_0 = GT_Q_BASE + 8
GT_DEV_CPU, GT_DEV_CUDA = 0, 1


def _load_native() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built; build it with `python gguf_train_amd/_build.py` "
            "(hipcc, gfx950). There is no CPU fallback."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    _check_sources(lib)
    return lib


def _check_sources(lib: ctypes.CDLL) -> None:
    """Refuses a library built from other sources than those beside it (a stale build)."""
    from ._srchash import source_hash

    want = source_hash()
    if want is None:  # no sources here: nothing to compare with
        return
    lib.gt_source_hash.argtypes = []
    lib.gt_source_hash.restype = c_char_p
    got = (lib.gt_source_hash() or b"").decode()
    if got != want:
        raise ImportError(
            f"{LIB_PATH} was built from other sources (library {got[:12]}, tree {want[:12]}); "
            "rebuild it with `python gguf_train_amd/_build.py`"
        )


def _configure(lib: ctypes.CDLL) -> ctypes.CDLL:
    p_i64 = POINTER(c_int64)
    p_vp = POINTER(c_void_p)

    lib.gt_init.argtypes = []
    lib.gt_init.restype = None
    lib.gt_device_count.argtypes = [c_int]
    lib.gt_device_count.restype = c_int
    lib.gt_device_name.argtypes = [c_int, c_int, c_char_p, c_int]
    lib.gt_device_name.restype = None
    lib.gt_device_memory.argtypes = [c_int, c_int, POINTER(c_size_t), POINTER(c_size_t)]
    lib.gt_device_memory.restype = None
    lib.gt_synchronize.argtypes = [c_int, c_int]
    lib.gt_synchronize.restype = None
    lib.gt_last_error.argtypes = []
    lib.gt_last_error.restype = c_char_p
    lib.gt_clear_error.argtypes = []
    lib.gt_clear_error.restype = None
    lib.gt_set_last_error.argtypes = [c_char_p]
    lib.gt_set_last_error.restype = None
    lib.gt_set_stream.argtypes = [c_void_p]
    lib.gt_set_stream.restype = None
    lib.gt_get_stream.argtypes = []
    lib.gt_get_stream.restype = c_void_p
    lib.gt_last_launch.argtypes = []
    lib.gt_last_launch.restype = c_char_p

    lib.gt_tensor_empty.argtypes = [c_int, p_i64, c_int, c_int, c_int]
    lib.gt_tensor_empty.restype = c_void_p
    lib.gt_tensor_from_data.argtypes = [c_int, p_i64, c_int, c_int, c_int, c_void_p, c_size_t]
    lib.gt_tensor_from_data.restype = c_void_p
    lib.gt_tensor_from_external.argtypes = [c_int, p_i64, p_i64, c_int, c_void_p, c_uint64]
    lib.gt_tensor_from_external.restype = c_void_p
    lib.gt_external_released.argtypes = [POINTER(c_uint64), c_int64]
    lib.gt_external_released.restype = c_int64
    lib.gt_tensor_from_device_ptr.argtypes = [c_int, p_i64, p_i64, c_int, c_int, c_void_p, c_uint64]
    lib.gt_tensor_from_device_ptr.restype = c_void_p
    lib.gt_tensor_clone.argtypes = [c_void_p]
    lib.gt_tensor_clone.restype = c_void_p
    lib.gt_tensor_view.argtypes = [c_void_p, c_int, p_i64, p_i64, c_int64]
    lib.gt_tensor_view.restype = c_void_p
    lib.gt_tensor_contiguous.argtypes = [c_void_p]
    lib.gt_tensor_contiguous.restype = c_void_p
    lib.gt_tensor_to_dtype.argtypes = [c_void_p, c_int]
    lib.gt_tensor_to_dtype.restype = c_void_p
    lib.gt_tensor_to_device.argtypes = [c_void_p, c_int, c_int]
    lib.gt_tensor_to_device.restype = c_void_p
    lib.gt_tensor_free.argtypes = [c_void_p]
    lib.gt_tensor_free.restype = None

    lib.gt_tensor_ndim.argtypes = [c_void_p]
    lib.gt_tensor_ndim.restype = c_int
    lib.gt_tensor_shape.argtypes = [c_void_p, p_i64]
    lib.gt_tensor_shape.restype = None
    lib.gt_tensor_strides.argtypes = [c_void_p, p_i64]
    lib.gt_tensor_strides.restype = None
    lib.gt_tensor_offset.argtypes = [c_void_p]
    lib.gt_tensor_offset.restype = c_int64
    lib.gt_tensor_numel.argtypes = [c_void_p]
    lib.gt_tensor_numel.restype = c_int64
    lib.gt_tensor_dtype.argtypes = [c_void_p]
    lib.gt_tensor_dtype.restype = c_int
    lib.gt_tensor_device_type.argtypes = [c_void_p]
    lib.gt_tensor_device_type.restype = c_int
    lib.gt_tensor_device_index.argtypes = [c_void_p]
    lib.gt_tensor_device_index.restype = c_int
    lib.gt_tensor_is_contiguous.argtypes = [c_void_p]
    lib.gt_tensor_is_contiguous.restype = c_int
    lib.gt_tensor_data_ptr.argtypes = [c_void_p]
    lib.gt_tensor_data_ptr.restype = c_uint64
    lib.gt_tensor_storage_nbytes.argtypes = [c_void_p]
    lib.gt_tensor_storage_nbytes.restype = c_size_t
    lib.gt_tensor_nbytes.argtypes = [c_void_p]
    lib.gt_tensor_nbytes.restype = c_size_t
    lib.gt_tensor_elem_size.argtypes = [c_int]
    lib.gt_tensor_elem_size.restype = c_size_t
    lib.gt_tensor_copy_to_host.argtypes = [c_void_p, c_void_p, c_size_t]
    lib.gt_tensor_copy_to_host.restype = c_int
    lib.gt_tensor_copy_from_host.argtypes = [c_void_p, c_void_p, c_size_t]
    lib.gt_tensor_copy_from_host.restype = c_int
    lib.gt_tensor_copy_inplace.argtypes = [c_void_p, c_void_p]
    lib.gt_tensor_copy_inplace.restype = c_int
    lib.gt_tensor_to_dlpack.argtypes = [c_void_p]
    lib.gt_tensor_to_dlpack.restype = c_void_p

    # attention (csrc/gguf_train.h:311; gguf_train/_C.py:471-472)
    lib.gt_flash_attention.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int]
    lib.gt_flash_attention.restype = c_void_p
    lib.gt_flash_attention_lse.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, p_vp, p_vp]
    lib.gt_flash_attention_lse.restype = c_int
    lib.gt_flash_attention_train.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, p_vp, p_vp, p_vp]
    lib.gt_flash_attention_train.restype = c_int
    lib.gt_flash_attention_backward.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                c_void_p, c_float, c_int, p_vp, p_vp, p_vp]
    lib.gt_flash_attention_backward.restype = c_int
    lib.gt_flash_attention_noalloc.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, c_void_p]
    lib.gt_flash_attention_noalloc.restype = c_int

    lib.gt_attention_weights.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, c_int]
    lib.gt_attention_weights.restype = c_void_p

    # dropout of the attention probabilities (replaces gguf_train/nn/functional.py:750-767 and
    # gguf_train/nn/modules/transformer.py:162-163; no counterpart in the reference ABI)
    lib.gt_flash_attention_dropout.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, c_double,
                                               c_uint64, c_uint64, p_vp, p_vp, p_vp]
    lib.gt_flash_attention_dropout.restype = c_int
    lib.gt_flash_attention_dropout_backward.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                        c_void_p, c_float, c_int, c_double, c_uint64, c_uint64, p_vp,
                                                        p_vp, p_vp]
    lib.gt_flash_attention_dropout_backward.restype = c_int
    lib.gt_attention_weights_dropout.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, c_int,
                                                 c_double, c_uint64, c_uint64]
    lib.gt_attention_weights_dropout.restype = c_void_p
    lib.gt_attention_dropout_mask.argtypes = [c_int64, c_int64, c_int64, c_int64, c_double, c_uint64, c_uint64, c_int]
    lib.gt_attention_dropout_mask.restype = c_void_p

    # RoPE (csrc/gguf_train.h:309-310; gguf_train/_C.py binds them with the same types)
    lib.gt_rope.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_float]
    lib.gt_rope.restype = c_void_p
    lib.gt_rope_backward.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_float]
    lib.gt_rope_backward.restype = c_void_p
    lib.gt_flash_attention_rope.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_int, c_void_p, c_int,
                                            c_int, c_float, c_float]
    lib.gt_flash_attention_rope.restype = c_void_p

    # Q8_0 (csrc/gguf_train.h:381-382)
    lib.gt_quantize.argtypes = [c_void_p, c_int]
    lib.gt_quantize.restype = c_void_p
    lib.gt_dequantize.argtypes = [c_void_p, c_int]
    lib.gt_dequantize.restype = c_void_p

    # KV cache (no counterpart in the reference ABI; behaviour of LlamaContext's cache,
    # csrc/llama_bridge.cpp:245-296)
    lib.gt_kv_cache_create.argtypes = [c_int64, c_int64, c_int64, c_int64, c_int, c_int]
    lib.gt_kv_cache_create.restype = c_void_p
    lib.gt_kv_cache_free.argtypes = [c_void_p]
    lib.gt_kv_cache_free.restype = None
    lib.gt_kv_cache_clear.argtypes = [c_void_p, c_int64]
    lib.gt_kv_cache_clear.restype = c_int
    lib.gt_kv_cache_length.argtypes = [c_void_p, c_int64]
    lib.gt_kv_cache_length.restype = c_int64
    lib.gt_kv_cache_capacity.argtypes = [c_void_p]
    lib.gt_kv_cache_capacity.restype = c_int64
    lib.gt_kv_cache_keys.argtypes = [c_void_p]
    lib.gt_kv_cache_keys.restype = c_void_p
    lib.gt_kv_cache_values.argtypes = [c_void_p]
    lib.gt_kv_cache_values.restype = c_void_p
    lib.gt_kv_cache_append.argtypes = [c_void_p, c_void_p, c_void_p, c_int64]
    lib.gt_kv_cache_append.restype = c_int
    lib.gt_kv_cache_append_rope.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_float, c_float]
    lib.gt_kv_cache_append_rope.restype = c_int
    lib.gt_kv_cache_attention.argtypes = [c_void_p, c_void_p, c_float, c_int]
    lib.gt_kv_cache_attention.restype = c_void_p

    # GGUF read side (csrc/gguf_train.h:363-379; gguf_train/_C.py:527-560)
    lib.gt_gguf_open.argtypes = [c_char_p]
    lib.gt_gguf_open.restype = c_void_p
    lib.gt_gguf_close.argtypes = [c_void_p]
    lib.gt_gguf_close.restype = None
    lib.gt_gguf_n_tensors.argtypes = [c_void_p]
    lib.gt_gguf_n_tensors.restype = c_int64
    lib.gt_gguf_tensor_name.argtypes = [c_void_p, c_int64]
    lib.gt_gguf_tensor_name.restype = c_char_p
    lib.gt_gguf_get_tensor.argtypes = [c_void_p, c_char_p, c_int]
    lib.gt_gguf_get_tensor.restype = c_void_p
    lib.gt_gguf_get_tensor_device.argtypes = [c_void_p, c_char_p, c_int, c_int]
    lib.gt_gguf_get_tensor_device.restype = c_void_p
    lib.gt_gguf_n_kv.argtypes = [c_void_p]
    lib.gt_gguf_n_kv.restype = c_int64
    lib.gt_gguf_kv_key.argtypes = [c_void_p, c_int64]
    lib.gt_gguf_kv_key.restype = c_char_p
    lib.gt_gguf_kv_type.argtypes = [c_void_p, c_int64]
    lib.gt_gguf_kv_type.restype = c_int
    lib.gt_gguf_kv_val_str.argtypes = [c_void_p, c_int64, c_char_p, c_int]
    lib.gt_gguf_kv_val_str.restype = c_int
    lib.gt_gguf_kv_arr_type.argtypes = [c_void_p, c_int64]
    lib.gt_gguf_kv_arr_type.restype = c_int
    lib.gt_gguf_kv_arr_n.argtypes = [c_void_p, c_int64]
    lib.gt_gguf_kv_arr_n.restype = c_int64
    lib.gt_gguf_kv_arr_data.argtypes = [c_void_p, c_int64]
    lib.gt_gguf_kv_arr_data.restype = c_void_p
    lib.gt_gguf_kv_arr_str.argtypes = [c_void_p, c_int64, c_int64]
    lib.gt_gguf_kv_arr_str.restype = c_char_p

    lib.gt_init()
    return lib


lib = _configure(_load_native())


def last_launch() -> str:
    """The kernels this thread's last attention call launched (gt_last_launch)."""
    msg = lib.gt_last_launch()
    return msg.decode("utf-8", errors="replace") if msg else ""


def last_error() -> str:
    msg = lib.gt_last_error()
    return msg.decode("utf-8", errors="replace") if msg else ""


_NATIVE_ERROR_TYPES = {"IndexError": IndexError}


def _native_error(ctx: str, err: str, fallback: str) -> Exception:
    for name, exc_type in _NATIVE_ERROR_TYPES.items():
        tag = name + ": "
        if err.startswith(tag):
            return exc_type(err[len(tag):])
    if ctx and err:
        return RuntimeError(err if err.startswith(ctx + ":") else f"{ctx}: {err}")
    return RuntimeError(err or ctx or fallback)


def check_ptr(ptr: int | None, ctx: str = "") -> int:
    if not ptr:
        raise _native_error(ctx, last_error(), "Native operation returned NULL")
    return ptr


def check_rc(rc: int, ctx: str = "") -> None:
    if rc != 0:
        raise _native_error(ctx, last_error(), f"Native operation failed with code {rc}")


def device_count() -> int:
    return int(lib.gt_device_count(GT_DEV_CUDA))
