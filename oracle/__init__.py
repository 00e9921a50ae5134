"""CPU oracle for the attention path - TEST INFRASTRUCTURE ONLY.

numpy front end of oracle/oracle_attn.c (a float64 C restatement of the reference's
gt_flash_attention, csrc/gt_ops_nn.cpp:2423-2525, of FlashAttentionFn.backward,
gguf_train/_functions.py:1933-1965, of the GGUF Q8_0 codec, csrc/gt_core.cpp:800-832, of
gt_rope / gt_rope_backward, csrc/gt_ops_nn.cpp:2298-2421, and of the dropout path of
scaled_dot_product_attention, gguf_train/nn/functional.py:750-767), plus the dropout
decisions' generator, Philox4x32-10 (Salmon et al., SC 2011), in numpy.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, to
check results or time the CPU baseline; the product (gguf_train_amd) never does.

Arrays are passed as numpy arrays; bfloat16 data travels as its uint16 bit patterns wrapped
in `BF16(bits)`.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "liboracle_attn.so"

F32, F16, BF16_CODE, F64, I8, U8, I16, I32, I64, BOOL = 0, 1, 2, 3, 4, 5, 6, 7, 8, 9

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built (python oracle/build.py)")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_flash_attention.argtypes = [vp, c_int, vp, c_int, vp, c_int, vp, c_int, c_int, vp,
                                             i64, i64, i64, i64, i64, i64, i64, ctypes.c_float, c_int,
                                             vp, c_int, vp, c_int]
        L.oracle_flash_attention.restype = c_int
        L.oracle_flash_attention_backward.argtypes = [vp, c_int, vp, c_int, vp, c_int, vp, c_int, vp, c_int,
                                                      c_int, vp, i64, i64, i64, i64, i64, i64, i64,
                                                      ctypes.c_float, c_int, vp, vp, vp, c_int]
        L.oracle_flash_attention_backward.restype = c_int
        for name in ("oracle_f32_to_f16_array", "oracle_f16_to_f32_array", "oracle_f32_to_bf16_array",
                     "oracle_bf16_to_f32_array"):
            getattr(L, name).argtypes = [vp, vp, i64]
            getattr(L, name).restype = None
        L.oracle_q8_0_quantize.argtypes = [vp, vp, i64]
        L.oracle_q8_0_dequantize.argtypes = [vp, vp, i64]
        L.oracle_max_threads.restype = c_int
        L.oracle_rope.argtypes = [vp, c_int, i64, i64, i64, i64, vp, c_int, c_int, ctypes.c_float, ctypes.c_float,
                                  c_int, vp]
        L.oracle_rope.restype = c_int
        L.oracle_attention_dropout.argtypes = [vp, c_int, vp, c_int, vp, c_int, vp, c_int, c_int, vp, vp,
                                               ctypes.c_double, vp, c_int, i64, i64, i64, i64, i64, i64, i64,
                                               ctypes.c_float, c_int, vp, c_int, vp, vp, vp, c_int]
        L.oracle_attention_dropout.restype = c_int
        _lib = L
    return _lib


@dataclass
class BF16:
    """bfloat16 data as uint16 bit patterns."""

    bits: np.ndarray

    @property
    def shape(self):
        return self.bits.shape


def _code(a) -> tuple[np.ndarray, int]:
    if isinstance(a, BF16):
        return np.ascontiguousarray(a.bits, dtype=np.uint16), BF16_CODE
    a = np.ascontiguousarray(a)
    codes = {np.float32: F32, np.float16: F16, np.float64: F64, np.int8: I8, np.uint8: U8, np.int16: I16,
             np.int32: I32, np.int64: I64, np.bool_: BOOL}
    for t, c in codes.items():
        if a.dtype == t:
            return a, c
    raise TypeError(f"oracle: unsupported dtype {a.dtype}")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---- conversions ---------------------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_ptr(x), _ptr(y), x.size)
    return y


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_ptr(h), _ptr(y), h.size)
    return y


def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16_array(_ptr(x), _ptr(y), x.size)
    return y


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    y = np.empty(b.shape, dtype=np.float32)
    lib().oracle_bf16_to_f32_array(_ptr(b), _ptr(y), b.size)
    return y


def to_f64(a) -> np.ndarray:
    """Values of an oracle input as float64."""
    if isinstance(a, BF16):
        return bf16_bits_to_f32(a.bits).astype(np.float64)
    return np.asarray(a).astype(np.float64)


# ---- attention -----------------------------------------------------------------------------

def flash_attention(q, k, v, mask=None, scale: float = -1.0, is_causal: bool = False, out_dtype=None,
                    nthreads: int = 0, return_lse: bool = False):
    """gt_flash_attention on dense inputs.  Output dtype = q's dtype unless `out_dtype` (a code)
    is given; float16/bfloat16 outputs come back as uint16 bit patterns."""
    qa, qc = _code(q)
    ka, kc = _code(k)
    va, vc = _code(v)
    B, H, L, D = qa.shape
    _, Hkv, S, Dv = va.shape
    oc = qc if out_dtype is None else out_dtype
    out = np.empty((B, H, L, Dv), dtype={F32: np.float32, F64: np.float64, F16: np.uint16, BF16_CODE: np.uint16}[oc])
    lse = np.empty((B, H, L), dtype=np.float64) if return_lse else None
    if mask is not None:
        ma, mc = _code(mask)
        mshape = (ctypes.c_int64 * 4)(*ma.shape, *([0] * (4 - ma.ndim)))
        mptr, mnd = _ptr(ma), ma.ndim
    else:
        ma, mc, mshape, mptr, mnd = None, 0, None, None, 0
    rc = lib().oracle_flash_attention(_ptr(qa), qc, _ptr(ka), kc, _ptr(va), vc, mptr, mc, mnd,
                                      ctypes.cast(mshape, ctypes.c_void_p) if mshape is not None else None,
                                      B, H, Hkv, L, S, D, Dv, float(scale), int(bool(is_causal)),
                                      _ptr(out), oc, _ptr(lse) if lse is not None else None, int(nthreads))
    if rc != 0:
        raise ValueError("oracle_flash_attention: inconsistent shapes")
    return (out, lse) if return_lse else out


def flash_attention_backward(dout, q, k, v, mask=None, scale: float = -1.0, is_causal: bool = False,
                             nthreads: int = 0):
    """FlashAttentionFn.backward in float64: returns (dq, dk, dv) as float64 arrays."""
    ga, gc = _code(dout)
    qa, qc = _code(q)
    ka, kc = _code(k)
    va, vc = _code(v)
    B, H, L, D = qa.shape
    _, Hkv, S, Dv = va.shape
    dq = np.empty((B, H, L, D), dtype=np.float64)
    dk = np.empty((B, Hkv, S, D), dtype=np.float64)
    dv = np.empty((B, Hkv, S, Dv), dtype=np.float64)
    if mask is not None:
        ma, mc = _code(mask)
        mshape = (ctypes.c_int64 * 4)(*ma.shape, *([0] * (4 - ma.ndim)))
        mptr, mnd = _ptr(ma), ma.ndim
    else:
        ma, mc, mshape, mptr, mnd = None, 0, None, None, 0
    rc = lib().oracle_flash_attention_backward(_ptr(ga), gc, _ptr(qa), qc, _ptr(ka), kc, _ptr(va), vc, mptr, mc, mnd,
                                               ctypes.cast(mshape, ctypes.c_void_p) if mshape is not None else None,
                                               B, H, Hkv, L, S, D, Dv, float(scale), int(bool(is_causal)),
                                               _ptr(dq), _ptr(dk), _ptr(dv), int(nthreads))
    if rc != 0:
        raise ValueError("oracle_flash_attention_backward: inconsistent shapes")
    return dq, dk, dv


# ---- dropout ---------------------------------------------------------------------------------

_PHILOX_M = (np.uint64(0xD2511F53), np.uint64(0xCD9E8D57))
_PHILOX_W = (0x9E3779B9, 0xBB67AE85)
_LO32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(counter, key) -> np.ndarray:
    """Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
    SC 2011): counter (N, 4) and key (N, 2) or (2,) of uint32 -> (N, 4) uint32 words.  Each round
    takes the two 32x32 -> 64-bit products M0 * c0 and M1 * c2 and maps
    (c0, c1, c2, c3) -> (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)); the key is
    bumped by the Weyl constants (W0, W1) between rounds."""
    c = np.array(counter, dtype=np.uint64).reshape(-1, 4)
    k = np.broadcast_to(np.array(key, dtype=np.uint64).reshape(-1, 2), (c.shape[0], 2)).copy()
    c0, c1, c2, c3 = (c[:, i].copy() for i in range(4))
    k0, k1 = k[:, 0], k[:, 1]
    for _ in range(10):
        p0 = _PHILOX_M[0] * c0
        p1 = _PHILOX_M[1] * c2
        c0, c1, c2, c3 = (p1 >> np.uint64(32)) ^ c1 ^ k0, p1 & _LO32, (p0 >> np.uint64(32)) ^ c3 ^ k1, p0 & _LO32
        k0 = (k0 + np.uint64(_PHILOX_W[0])) & _LO32
        k1 = (k1 + np.uint64(_PHILOX_W[1])) & _LO32
    return np.stack([c0, c1, c2, c3], axis=1).astype(np.uint32)


def dropout_threshold(p: float) -> int:
    """Keep when the element's word < floor((1 - p) * 2^32) (at most 2^32 - 1); 0 for p = 1."""
    return int(min(np.floor((1.0 - float(p)) * 4294967296.0), 4294967295.0))


def dropout_keep(B: int, H: int, L: int, S: int, p: float, seed: int, offset: int = 0) -> np.ndarray:
    """The dropout decisions (B, H, L, S) bool of the library's attention dropout: element
    (b, h, l, s) takes word s % 4 of Philox4x32-10 with counter (n mod 2^32, n / 2^32,
    offset mod 2^32, offset / 2^32), n = ((b*H + h)*L + l) * ceil(S/4) + s/4, and key (seed mod
    2^32, seed / 2^32); kept when the word is below dropout_threshold(p).  p = 0 keeps all."""
    if p == 0.0:
        return np.ones((B, H, L, S), dtype=bool)
    nb = (S + 3) // 4
    n = np.arange(B * H * L * nb, dtype=np.uint64)
    seed, offset = int(seed) & 0xFFFFFFFFFFFFFFFF, int(offset) & 0xFFFFFFFFFFFFFFFF
    ctr = np.stack([n & _LO32, n >> np.uint64(32), np.full_like(n, offset & 0xFFFFFFFF),
                    np.full_like(n, offset >> 32)], axis=1)
    words = philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32)).reshape(B * H * L, nb * 4)[:, :S]
    return (words < np.uint32(dropout_threshold(p)) if p < 1.0 else np.zeros_like(words, dtype=bool)).reshape(
        B, H, L, S)


def attention_dropout(q, k, v, keep, p: float, mask=None, scale: float = -1.0, is_causal: bool = False,
                      dout=None, out_dtype=None, nthreads: int = 0):
    """scaled_dot_product_attention with dropout (gguf_train/nn/functional.py:750-767) in float64
    for the keep mask `keep` (B,H,L,S bool).  Returns the output in q's dtype (or `out_dtype`;
    float16/bfloat16 as uint16 bits) and, when `dout` is given, (dq, dk, dv) float64."""
    qa, qc = _code(q)
    ka, kc = _code(k)
    va, vc = _code(v)
    B, H, L, D = qa.shape
    _, Hkv, S, Dv = va.shape
    kp = np.ascontiguousarray(keep, dtype=np.uint8)
    if kp.shape != (B, H, L, S):
        raise ValueError("oracle_attention_dropout: keep must be (B, H, L, S)")
    oc = qc if out_dtype is None else out_dtype
    out = np.empty((B, H, L, Dv), dtype={F32: np.float32, F64: np.float64, F16: np.uint16, BF16_CODE: np.uint16}[oc])
    if mask is not None:
        ma, mc = _code(mask)
        mshape = (ctypes.c_int64 * 4)(*ma.shape, *([0] * (4 - ma.ndim)))
        mptr, mnd = _ptr(ma), ma.ndim
    else:
        ma, mc, mshape, mptr, mnd = None, 0, None, None, 0
    if dout is not None:
        ga, gc = _code(dout)
        dq = np.empty((B, H, L, D), dtype=np.float64)
        dk = np.empty((B, Hkv, S, D), dtype=np.float64)
        dv = np.empty((B, Hkv, S, Dv), dtype=np.float64)
    else:
        ga, gc, dq, dk, dv = None, 0, None, None, None
    rc = lib().oracle_attention_dropout(_ptr(qa), qc, _ptr(ka), kc, _ptr(va), vc, mptr, mc, mnd,
                                        ctypes.cast(mshape, ctypes.c_void_p) if mshape is not None else None,
                                        _ptr(kp), float(p), _ptr(ga) if ga is not None else None, gc,
                                        B, H, Hkv, L, S, D, Dv, float(scale), int(bool(is_causal)), _ptr(out), oc,
                                        *(_ptr(x) if x is not None else None for x in (dq, dk, dv)), int(nthreads))
    if rc != 0:
        raise ValueError("oracle_attention_dropout: inconsistent shapes")
    return out if dout is None else (out, (dq, dk, dv))


# ---- Q8_0 ----------------------------------------------------------------------------------

def q8_0_quantize(x) -> np.ndarray:
    """float32 values (size a multiple of 32) -> ggml block_q8_0 bytes, shape (nblocks*34,)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if x.size % 32:
        raise ValueError("q8_0 needs a multiple of 32 values")
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib().oracle_q8_0_quantize(_ptr(x), _ptr(out), x.size // 32)
    return out


def q8_0_dequantize(blocks) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    n = b.size // 34
    y = np.empty(n * 32, dtype=np.float32)
    lib().oracle_q8_0_dequantize(_ptr(b), _ptr(y), n)
    return y


# ---- RoPE ----------------------------------------------------------------------------------

def rope(x, pos, n_dims=None, mode: int = 0, freq_base: float = 10000.0, freq_scale: float = 1.0,
         backward: bool = False):
    """gt_rope / gt_rope_backward on a dense (B, H, S, D) or (H, S, D) array: the result has x's
    dtype (float16/bfloat16 as uint16 bit patterns, BF16 in -> BF16 out)."""
    xa, xc = _code(x)
    shape = xa.shape
    if xa.ndim == 3:
        xa = xa.reshape((1,) + shape)
    B, H, S, D = xa.shape
    nd = D if n_dims is None else int(n_dims)
    p = np.ascontiguousarray(np.asarray(pos)[:S], dtype=np.int32)
    if p.size < S:
        raise ValueError("oracle rope: fewer positions than sequence elements")
    y = np.empty_like(xa)
    rc = lib().oracle_rope(_ptr(xa), xc, B, H, S, D, _ptr(p), nd, int(mode), float(freq_base), float(freq_scale),
                           int(bool(backward)), _ptr(y))
    if rc != 0:
        raise ValueError("oracle rope: bad n_dims or mode")
    y = y.reshape(shape)
    return BF16(y) if isinstance(x, BF16) else y


def max_threads() -> int:
    return int(lib().oracle_max_threads())


# ---- the reference's backward composition in float32 GEMMs (CPU baseline only) -------------

def backward_composition_f32(dout, q, k, v, mask=None, scale: float = -1.0, is_causal: bool = False):
    """FlashAttentionFn.backward as the reference composes it (gguf_train/_functions.py:1933-1965):
    full (B, H, L, S) scores, causal -1e9, additive mask, softmax, then dV = P^T dO,
    dP = dO V^T, dS = P (dP - rowsum(dP P)), dQ = dS K s, dK = dS^T Q s, GQA groups summed -
    with float32 numpy GEMMs (BLAS) standing in for ggml's float32 mul_mat.  Used only as the CPU
    baseline's timing of the training backward; the parity oracle is flash_attention_backward."""
    g, q, k, v = (to_f64(a).astype(np.float32) for a in (dout, q, k, v))
    B, H, L, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    s = np.float32(1.0 / np.sqrt(D) if scale <= 0 else scale)
    rep = H // Hkv
    ku = np.repeat(k, rep, axis=1) if rep > 1 else k
    vu = np.repeat(v, rep, axis=1) if rep > 1 else v
    scores = np.matmul(q, ku.transpose(0, 1, 3, 2)) * s
    if is_causal:
        scores += np.triu(np.full((L, S), -1e9, np.float32), k=1)
    if mask is not None:
        scores += to_f64(mask).astype(np.float32)
    scores -= scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p /= p.sum(axis=-1, keepdims=True)
    dv = np.matmul(p.transpose(0, 1, 3, 2), g)
    dp = np.matmul(g, vu.transpose(0, 1, 3, 2))
    ds = p * (dp - (dp * p).sum(axis=-1, keepdims=True))
    dq = np.matmul(ds, ku) * s
    dk = np.matmul(ds.transpose(0, 1, 3, 2), q) * s
    if rep > 1:
        dk = dk.reshape(B, Hkv, rep, S, D).sum(axis=2)
        dv = dv.reshape(B, Hkv, rep, S, v.shape[3]).sum(axis=2)
    return dq, dk, dv
