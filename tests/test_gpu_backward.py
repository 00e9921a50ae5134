"""Backward parity: gt_flash_attention_backward against the float64 oracle restatement of
FlashAttentionFn.backward (gguf_train/_functions.py:1933-1965) on the same rounded inputs, the
kernel's float32 gradients compared before the autograd engine casts them; plus gradcheck in
float64 (tests/test_autograd.py:137-140) and the autograd wiring."""

import math

import numpy as np
import pytest
import torch

import gguf_train_amd as g
import oracle
from gguf_train_amd.nn import functional as F

from _util import assert_close, randn, to_oracle

pytestmark = pytest.mark.gpu


def oracle_grads(dout, q, k, v, mask=None, is_causal=False, scale=-1.0):
    return oracle.flash_attention_backward(to_oracle(dout), to_oracle(q), to_oracle(k), to_oracle(v),
                                           mask=None if mask is None else to_oracle(mask), scale=scale,
                                           is_causal=is_causal)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,Hkv,L,S,D", [(2, 4, 4, 20, 20, 64), (1, 4, 2, 13, 29, 32), (2, 2, 1, 33, 17, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_native_backward_matches_oracle(dev, dtype, B, H, Hkv, L, S, D, causal):
    seed = 7 * B + L + S
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    dout = randn((B, H, L, D), seed + 3, dtype)
    # key padding, as the training configuration: valid length per sequence, -inf beyond
    lens = np.random.default_rng(seed).integers(S // 2 + 1, S + 1, size=B)
    mask = torch.zeros(B, 1, 1, S)
    for b, n in enumerate(lens):
        mask[b, ..., n:] = float("-inf")
    out, lse, out32 = g.flash_attention_train(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, causal)
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                                            out if out32 is None else out32, lse, 0.0, causal)
    assert dq.dtype == dk.dtype == dv.dtype == torch.float32
    wq, wk, wv = oracle_grads(dout, q, k, v, mask=mask, is_causal=causal)
    tol_dtype = torch.float32 if dtype == torch.float32 else torch.bfloat16
    assert_close(dq, wq, tol_dtype, "dq", out_dtype=torch.float32)
    assert_close(dk, wk, tol_dtype, "dk", out_dtype=torch.float32)
    assert_close(dv, wv, tol_dtype, "dv", out_dtype=torch.float32)


def _full_mask(kind, shape, seed):
    rng = np.random.default_rng(seed)
    if kind == "bool":
        m = torch.from_numpy(rng.random(shape) < 0.8)
        m[..., 0] = True  # every row sees a key
        return m
    return torch.from_numpy((rng.standard_normal(shape) * 0.7).astype(np.float32))


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float16, 128)])
@pytest.mark.parametrize("kind", ["bool", "float"])
@pytest.mark.parametrize("mshape", ["LS", "BHLS"])
@pytest.mark.parametrize("L,S", [(160, 256), (150, 150)])
@pytest.mark.parametrize("causal", [False, True])
def test_mfma_backward_with_per_element_masks(dev, dtype, D, kind, mshape, L, S, causal):
    # S % 4 == 0 with contiguous keys: the dQ kernel's 4-key mask loads; 150 keys: per element
    B, H, Hkv = 2, 4, 2
    seed = L + S + D
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    dout = randn((B, H, L, D), seed + 3, dtype)
    mask = _full_mask(kind, (L, S) if mshape == "LS" else (B, H, L, S), seed)
    md = mask.to(dev)
    out, lse, out32 = g.flash_attention_train(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal)
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), md, out32, lse, 0.0, causal)
    m4 = mask.reshape((1, 1) + tuple(mask.shape)) if mask.ndim == 2 else mask
    wq, wk, wv = oracle_grads(dout, q, k, v, mask=m4, is_causal=causal)
    for name, got, want in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv)):
        assert_close(got, want, torch.bfloat16, f"{name} {kind} {mshape}", out_dtype=torch.float32)


@pytest.mark.parametrize("kind", ["bool", "float"])
def test_backward_mask_loads_of_every_layout_give_the_same_bits(dev, kind):
    # the contiguous mask (4-key loads in dQ) and the same values strided by 2 or at an unaligned
    # base (per-element loads) give identical gradients
    B, H, L, S, D, dtype = 2, 4, 128, 192, 64, torch.bfloat16
    q, k, v, dout = (randn(sh, i, dtype).to(dev) for i, sh in enumerate([(B, H, L, D), (B, H, S, D), (B, H, S, D),
                                                                         (B, H, L, D)]))
    m = _full_mask(kind, (L, S), 3).to(dev)
    wide = torch.zeros((L, 2 * S), dtype=m.dtype, device=dev)
    wide[:, ::2] = m
    flat = torch.zeros(L * S + 1, dtype=m.dtype, device=dev)
    flat[1:] = m.reshape(-1)

    def grads(mask):
        out, lse, out32 = g.flash_attention_train(q, k, v, mask, 0.0, True)
        return g.flash_attention_backward(dout, q, k, v, mask, out32, lse, 0.0, True)

    ref = grads(m)
    for other in (wide[:, ::2], flat[1:].view(L, S)):
        for a, b in zip(grads(other), ref):
            assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("D,Dv", [(64, 96), (256, 256), (200, 160), (16, 8), (300, 40), (1, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_generic_backward_chunk_and_value_shapes(dev, dtype, D, Dv, causal):
    # the generic backward's chunk sizes (64 / 32 / 16 keys or query rows staged per workgroup),
    # 1, 2 or 4 output blocks of 64 with a partial last one, the unstaged kernels (D > 256),
    # GQA, 150 keys / 37 rows (partial chunks), key padding plus scattered float mask values
    B, H, Hkv, L, S = 1, 4, 2, 37, 150
    seed = D * 17 + Dv
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, Dv), seed + 2, dtype)
    dout = randn((B, H, L, Dv), seed + 3, dtype)
    rng = np.random.default_rng(seed)
    mask = torch.from_numpy(rng.standard_normal((L, S)) * 0.5).to(dtype)
    mask[:, 120:] = float("-inf")
    out, lse, out32 = g.flash_attention_train(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, causal)
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), mask.to(dev),
                                            out if out32 is None else out32, lse, 0.0, causal)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    wq, wk, wv = oracle_grads(dout, q, k, v, mask=mask, is_causal=causal)
    assert_close(dq, wq, dtype, f"dq D={D} Dv={Dv}")
    assert_close(dk, wk, dtype, f"dk D={D} Dv={Dv}")
    assert_close(dv, wv, dtype, f"dv D={D} Dv={Dv}")
    # keys 120.. are never visible: their gradients are exactly zero
    assert not dk[:, :, 120:].any() and not dv[:, :, 120:].any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("given", ["rounded_out", "nothing", "rounded_out_no_lse"])
def test_backward_from_the_rounded_output(dev, dtype, D, given):
    # the C ABI also takes the forward's output in the input dtype (not the float32 copy the
    # training forward keeps), or no output / log-sum-exp at all: the float32 output is then
    # recomputed, so rowsum(dO * O) carries no output rounding
    B, H, Hkv, L, S = 2, 4, 2, 70, 70
    seed = D + (3 if dtype == torch.float16 else 5)
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    dout = randn((B, H, L, D), seed + 3, dtype)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), None, 0.0, True)
    assert out.dtype == dtype
    o_arg = None if given == "nothing" else out
    l_arg = lse if given == "rounded_out" else None
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), None, o_arg, l_arg, 0.0, True)
    wq, wk, wv = oracle_grads(dout, q, k, v, is_causal=True)
    assert_close(dq, wq, torch.bfloat16, "dq", out_dtype=torch.float32)
    assert_close(dk, wk, torch.bfloat16, "dk", out_dtype=torch.float32)
    assert_close(dv, wv, torch.bfloat16, "dv", out_dtype=torch.float32)


def test_gradcheck_float64(dev):
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 2, 4, 8, dtype=torch.float64, device=dev, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(lambda a, b, c: F.scaled_dot_product_attention(a, b, c, is_causal=True),
                                    (q, k, v), eps=1e-6, atol=1e-5, rtol=1e-3)


def test_autograd_wiring_and_grad_dtypes(dev):
    q = randn((2, 4, 16, 64), 1, torch.bfloat16).to(dev).requires_grad_()
    k = randn((2, 2, 16, 64), 2, torch.bfloat16).to(dev).requires_grad_()
    v = randn((2, 2, 16, 64), 3, torch.bfloat16).to(dev).requires_grad_()
    out = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    dout = randn((2, 4, 16, 64), 4, torch.bfloat16).to(dev)
    out.backward(dout)
    assert q.grad.dtype == k.grad.dtype == v.grad.dtype == torch.bfloat16
    wq, wk, wv = oracle_grads(dout, q, k, v, is_causal=True)
    for got, want in ((q.grad, wq), (k.grad, wk), (v.grad, wv)):
        # bf16 rounding of the gradient itself on top of the kernel tolerance
        err = np.abs(got.float().cpu().numpy() - want) / np.maximum(1.0, np.abs(want))
        assert err.max() < 2e-3 + 2 ** -8


def test_backward_without_saved_lse(dev):
    q, k, v = randn((1, 2, 9, 16), 5), randn((1, 2, 9, 16), 6), randn((1, 2, 9, 16), 7)
    dout = randn((1, 2, 9, 16), 8)
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), None, None, None, 0.0, True)
    wq, wk, wv = oracle_grads(dout, q, k, v, is_causal=True)
    assert_close(dq, wq, torch.float32, "dq")
    assert_close(dk, wk, torch.float32, "dk")
    assert_close(dv, wv, torch.float32, "dv")
