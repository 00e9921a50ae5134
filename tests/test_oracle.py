"""Pins the CPU oracle (oracle/) before the parity tests trust it.

Each oracle function is checked against something other than its own formula: numpy/torch
conversions over every bit pattern, the closed form softmax(QK^T*s + M).V evaluated by
torch.float64, hand-computed cases, the reference's rules (top-left causal, fully blocked row
-> 0, GQA = repeated heads), finite differences, torch.autograd, and for Q8_0 exactly
representable blocks, rounding ties and the reference's own accuracy checks
(tests/test_numpy_interop.py:443-454, tests/test_gguf_and_llama.py:65-79).
"""

import math

import numpy as np
import pytest
import torch

import oracle


# ---- float16 / bfloat16 conversions ----------------------------------------------------------

def test_f16_to_f32_matches_numpy_for_every_pattern():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def _f32_samples():
    rng = np.random.default_rng(7)
    halves = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    halves = halves[np.isfinite(halves)]
    # exact halfway points between neighbouring halves, and points just beside them
    mid = ((halves[:-1].astype(np.float64) + halves[1:].astype(np.float64)) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf))])
    wide = np.concatenate([rng.standard_normal(200_000).astype(np.float32) * s for s in (1e-9, 1e-6, 1e-3, 1, 1e3, 1e5)])
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.996, 65520, 1e38, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25,
                        2 ** -26, 1e-45], dtype=np.float32)
    return np.concatenate([halves, mid, near, wide, special])


def test_f32_to_f16_matches_numpy():
    x = _f32_samples()
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert (oracle.f32_to_f16_bits(x) == want).all()


def test_f32_to_bf16_matches_torch():
    x = _f32_samples()
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (oracle.f32_to_bf16_bits(x) == want).all()
    nan = np.array([np.nan], dtype=np.float32)
    assert np.isnan(oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(nan))).all()


# ---- forward -----------------------------------------------------------------------------------

def c_scale(D, scale=None):
    """The scale as the native code sees it: a float32 argument, 1.0f/sqrtf(D) in float32
    arithmetic when not given (csrc/gt_ops_nn.cpp:2433)."""
    if scale is None:
        return float(np.float32(1.0) / np.sqrt(np.float32(D)))
    return float(np.float32(scale))


def torch_attention(q, k, v, mask=None, scale=None, is_causal=False):
    """softmax(QK^T*s + M).V in float64 with explicit head repetition; bool mask True = attend."""
    q, k, v = (torch.from_numpy(np.asarray(a, dtype=np.float64)) for a in (q, k, v))
    H, Hkv = q.shape[1], k.shape[1]
    k = k.repeat_interleave(H // Hkv, dim=1)
    v = v.repeat_interleave(H // Hkv, dim=1)
    s = (q @ k.transpose(-1, -2)) * c_scale(q.shape[-1], scale)
    L, S = s.shape[-2:]
    if is_causal:
        s = s.masked_fill(torch.ones(L, S, dtype=torch.bool).triu(1), float("-inf"))
    if mask is not None:
        m = torch.from_numpy(np.array(mask))
        s = s.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else s + m.double()
    p = torch.softmax(s, -1)
    return (p @ v).numpy(), torch.logsumexp(s, -1).numpy()


def rand(shape, rng, dtype=np.float32, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(dtype)


@pytest.mark.parametrize("B,H,Hkv,L,S,D,Dv", [(2, 3, 3, 4, 5, 6, 6), (1, 4, 2, 7, 9, 8, 5), (2, 8, 1, 1, 33, 16, 16)])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_matches_closed_form(B, H, Hkv, L, S, D, Dv, causal):
    rng = np.random.default_rng(B * 100 + L)
    q, k, v = rand((B, H, L, D), rng), rand((B, Hkv, S, D), rng), rand((B, Hkv, S, Dv), rng)
    got, lse = oracle.flash_attention(q, k, v, is_causal=causal, out_dtype=oracle.F64, return_lse=True)
    want, wlse = torch_attention(q, k, v, is_causal=causal)
    assert np.abs(got - want).max() < 1e-12
    assert np.abs(lse - wlse).max() < 1e-12


MASK_SHAPES = [(2, 3, 4, 5), (2, 1, 4, 5), (1, 3, 4, 5), (4, 5), (1, 1, 1, 5), (2, 1, 1, 5), (1, 1, 4, 1), (2, 3, 1, 1)]


@pytest.mark.parametrize("mshape", MASK_SHAPES)
def test_forward_masks_broadcast_like_the_reference(mshape):
    rng = np.random.default_rng(11)
    q, k, v = rand((2, 3, 4, 6), rng), rand((2, 3, 5, 6), rng), rand((2, 3, 5, 6), rng)
    allowed = rng.random(mshape) < 0.6
    allowed[..., 0] = True
    got = oracle.flash_attention(q, k, v, mask=allowed, out_dtype=oracle.F64)
    want, _ = torch_attention(q, k, v, mask=np.broadcast_to(allowed, (2, 3, 4, 5)))
    assert np.abs(got - want).max() < 1e-12
    additive = np.where(allowed, 0.0, -1e9).astype(np.float32)
    got = oracle.flash_attention(q, k, v, mask=additive, out_dtype=oracle.F64)
    assert np.abs(got - want).max() < 1e-12
    bias = rand(mshape, rng)
    got = oracle.flash_attention(q, k, v, mask=bias, out_dtype=oracle.F64)
    want, _ = torch_attention(q, k, v, mask=np.broadcast_to(bias, (2, 3, 4, 5)))
    assert np.abs(got - want).max() < 1e-12


def test_forward_hand_computed():
    # scores 0 and ln 3 -> weights 1/4, 3/4 -> 1/4*1 + 3/4*5 = 4
    q = np.array([[[[1.0]]]])
    k = np.array([[[[0.0], [math.log(3.0)]]]])
    v = np.array([[[[1.0], [5.0]]]])
    got = oracle.flash_attention(q, k, v, scale=1.0)
    assert got.shape == (1, 1, 1, 1) and abs(got[0, 0, 0, 0] - 4.0) < 1e-15


def test_causal_is_top_left_aligned_and_blocked_rows_are_zero():
    rng = np.random.default_rng(3)
    q, k, v = rand((1, 1, 3, 4), rng, np.float64), rand((1, 1, 5, 4), rng, np.float64), rand((1, 1, 5, 4), rng, np.float64)
    got = oracle.flash_attention(q, k, v, is_causal=True)
    assert np.array_equal(got[0, 0, 0], v[0, 0, 0])  # row 0 sees key 0 only, whatever S is
    blocked = np.ones((3, 5), dtype=bool)
    blocked[1] = False  # row 1 sees nothing
    got, lse = oracle.flash_attention(q, k, v, mask=blocked, return_lse=True)
    assert np.array_equal(got[0, 0, 1], np.zeros(4)) and np.isinf(lse[0, 0, 1]) and lse[0, 0, 1] > 0
    neg = np.where(blocked, 0.0, -np.inf)
    got2 = oracle.flash_attention(q, k, v, mask=neg)
    assert np.array_equal(got2[0, 0, 1], np.zeros(4))


def test_gqa_equals_repeated_heads():
    rng = np.random.default_rng(5)
    q, k, v = rand((2, 6, 5, 8), rng), rand((2, 2, 7, 8), rng), rand((2, 2, 7, 8), rng)
    got = oracle.flash_attention(q, k, v, out_dtype=oracle.F64)
    want = oracle.flash_attention(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1), out_dtype=oracle.F64)
    assert np.array_equal(got, want)


def test_outputs_round_through_float32():
    rng = np.random.default_rng(9)
    q, k, v = rand((1, 2, 8, 16), rng), rand((1, 2, 8, 16), rng), rand((1, 2, 8, 16), rng)
    exact = oracle.flash_attention(q, k, v, out_dtype=oracle.F64)
    h = oracle.flash_attention(q, k, v, out_dtype=oracle.F16)
    assert np.array_equal(h, exact.astype(np.float32).astype(np.float16).view(np.uint16))
    b = oracle.flash_attention(q, k, v, out_dtype=oracle.BF16_CODE)
    want = torch.from_numpy(exact.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(b, want)


def test_reads_half_and_bfloat16_inputs_by_value():
    rng = np.random.default_rng(13)
    q, k, v = rand((1, 2, 4, 8), rng), rand((1, 2, 6, 8), rng), rand((1, 2, 6, 8), rng)
    qh, kh, vh = (a.astype(np.float16) for a in (q, k, v))
    got = oracle.flash_attention(qh, kh, vh, out_dtype=oracle.F64)
    want, _ = torch_attention(qh.astype(np.float64), kh.astype(np.float64), vh.astype(np.float64))
    assert np.abs(got - want).max() < 1e-12
    qb, kb, vb = (oracle.BF16(oracle.f32_to_bf16_bits(a)) for a in (q, k, v))
    got = oracle.flash_attention(qb, kb, vb, out_dtype=oracle.F64)
    want, _ = torch_attention(*(oracle.to_f64(a) for a in (qb, kb, vb)))
    assert np.abs(got - want).max() < 1e-12


# ---- backward ----------------------------------------------------------------------------------

def torch_grads(q, k, v, dout, mask=None, is_causal=False):
    q, k, v = (torch.tensor(np.asarray(a, dtype=np.float64), requires_grad=True) for a in (q, k, v))
    H, Hkv = q.shape[1], k.shape[1]
    ku, vu = k.repeat_interleave(H // Hkv, 1), v.repeat_interleave(H // Hkv, 1)
    s = (q @ ku.transpose(-1, -2)) * c_scale(q.shape[-1])
    L, S = s.shape[-2:]
    if is_causal:
        s = s.masked_fill(torch.ones(L, S, dtype=torch.bool).triu(1), float("-inf"))
    if mask is not None:
        m = torch.from_numpy(np.array(mask))
        s = s.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else s + m.double()
    out = torch.softmax(s, -1) @ vu
    out.backward(torch.from_numpy(np.asarray(dout, dtype=np.float64)))
    return q.grad.numpy(), k.grad.numpy(), v.grad.numpy()


@pytest.mark.parametrize("Hkv", [4, 2, 1])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_autograd(Hkv, causal):
    rng = np.random.default_rng(17 + Hkv)
    q, k, v = rand((2, 4, 6, 8), rng), rand((2, Hkv, 7, 8), rng), rand((2, Hkv, 7, 5), rng)
    dout = rand((2, 4, 6, 5), rng)
    mask = rng.random((2, 1, 1, 7)) < 0.8
    mask[..., 0] = True
    got = oracle.flash_attention_backward(dout, q, k, v, mask=mask, is_causal=causal)
    want = torch_grads(q, k, v, dout, mask=mask, is_causal=causal)
    for g, w in zip(got, want):
        assert np.abs(g - w).max() < 1e-10


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(23)
    q, k, v = rand((1, 2, 3, 4), rng, np.float64), rand((1, 1, 5, 4), rng, np.float64), rand((1, 1, 5, 3), rng, np.float64)
    dout = rand((1, 2, 3, 3), rng, np.float64)
    bias = rand((1, 1, 3, 5), rng, np.float64)
    dq, dk, dv = oracle.flash_attention_backward(dout, q, k, v, mask=bias, is_causal=True)

    def loss(qq, kk, vv):
        return float((oracle.flash_attention(qq, kk, vv, mask=bias, is_causal=True) * dout).sum())

    eps = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            a1, a2 = arr.copy(), arr.copy()
            a1[idx] += eps
            a2[idx] -= eps
            args1 = [a1 if x is arr else x for x in (q, k, v)]
            args2 = [a2 if x is arr else x for x in (q, k, v)]
            num[idx] = (loss(*args1) - loss(*args2)) / (2 * eps)
        assert np.abs(num - grad).max() < 1e-7


# ---- Q8_0 --------------------------------------------------------------------------------------

def blocks_of(b):
    b = b.reshape(-1, 34)
    d = b[:, :2].copy().view(np.uint16).reshape(-1)
    qs = b[:, 2:].view(np.int8)
    return d, qs


def test_q8_0_exact_block():
    # amax = 127 -> d = 1, every integer is represented exactly
    x = np.arange(-127, -127 + 32, dtype=np.float32)
    x[5] = 127.0
    b = oracle.q8_0_quantize(x)
    d, qs = blocks_of(b)
    assert d[0] == np.float16(1.0).view(np.uint16)
    assert np.array_equal(qs[0].astype(np.float32), x)
    assert np.array_equal(oracle.q8_0_dequantize(b), x)


def test_q8_0_zero_block_and_ties_round_away_from_zero():
    z = oracle.q8_0_quantize(np.zeros(32, np.float32))
    assert np.array_equal(z, np.zeros(34, np.uint8))
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0
    x[1:5] = [2.5, -2.5, 0.5, -0.5]  # d = 1: ties go away from zero (roundf), not to even
    _, qs = blocks_of(oracle.q8_0_quantize(x))
    assert list(qs[0, 1:5]) == [3, -3, 1, -1]


def test_q8_0_scale_is_fp16_of_amax_over_127():
    for amax in (1.0, 3.7, 1e-3, 65000.0):
        x = np.zeros(32, dtype=np.float32)
        x[7] = -amax
        d, qs = blocks_of(oracle.q8_0_quantize(x))
        assert d[0] == np.float16(np.float32(amax) / np.float32(127)).view(np.uint16)
        assert qs[0, 7] == -127


def test_q8_0_reference_accuracy_checks():
    # tests/test_numpy_interop.py:443-454: arange(64)/64 round trip within 0.01
    x = (np.arange(64) / 64).astype(np.float32)
    assert np.abs(oracle.q8_0_dequantize(oracle.q8_0_quantize(x)) - x).max() < 0.01
    # tests/test_gguf_and_llama.py:65-79: cosine similarity > 0.85 on normal data
    rng = np.random.default_rng(29)
    y = rng.standard_normal(4096).astype(np.float32)
    r = oracle.q8_0_dequantize(oracle.q8_0_quantize(y))
    assert float(y @ r / np.linalg.norm(y) / np.linalg.norm(r)) > 0.85


def test_q8_0_error_bound_and_idempotence():
    rng = np.random.default_rng(31)
    x = (rng.standard_normal(32 * 512) * rng.choice([1e-3, 1, 30], 32 * 512)).astype(np.float32)
    b = oracle.q8_0_quantize(x)
    y = oracle.q8_0_dequantize(b)
    d, qs = blocks_of(b)
    df = d.view(np.float16).astype(np.float32)
    # dequantized value is exactly qs * d in float32
    assert np.array_equal(y.reshape(-1, 32), qs.astype(np.float32) * df[:, None])
    # every value lies within half a step (plus the fp16 rounding of d) of the input
    step = np.repeat(df, 32)
    amax = np.repeat(np.abs(x.reshape(-1, 32)).max(1), 32)
    assert (np.abs(y - x) <= 0.5 * step + 127 * np.abs(step - amax / 127) + 1e-7).all()
    assert np.array_equal(oracle.q8_0_quantize(y), b)
