"""Autocast lowering and view invariance of the attention path, ported from the reference's tests:

- tests/test_autocast.py:208-214: inside an autocast block scaled_dot_product_attention (with and
  without dropout) and MultiheadAttention return the autocast dtype, float32 outside; the
  operands are cast (gguf_train/_tensor.py:261-283, policy gguf_train/amp.py:8-10) and the
  gradients come back to float32 leaves in float32 (gguf_train/_autograd_engine.py:325-326);
- tests/test_views_and_fast_paths.py:334-336 (check_views, :90-140): the same values and the same
  gradients, at 2e-4 * max(1, |w|), whether each argument is fresh storage, a contiguous view
  at an offset into a larger storage or a strided view, and whether the incoming gradient is
  plain, a slice of a larger one or strided.  Run at the reference's shape (float32, D = 4: the
  generic kernels) and at a shape that takes the MFMA kernels (bf16 / fp16, D = 64)."""

import math

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd.nn import MultiheadAttention
from gguf_train_amd.nn import functional as F

from _util import assert_close, randn, to_oracle
import oracle

pytestmark = pytest.mark.gpu

JUNK = 99.0


# ---- autocast ----------------------------------------------------------------------------------

@pytest.mark.parametrize("device_type", ["cuda", "cpu"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_runs_in_the_autocast_dtype(dev, device_type, dtype):
    d = dev if device_type == "cuda" else torch.device("cpu")
    torch.manual_seed(0)
    heads = torch.randn(2, 2, 5, 4, device=d)
    seq = torch.randn(2, 5, 8, device=d)
    mha = MultiheadAttention(8, 2, batch_first=True).to(d)
    cases = {
        "attention": lambda: F.scaled_dot_product_attention(heads, heads, heads),
        "attention with dropout": lambda: F.scaled_dot_product_attention(heads, heads, heads, dropout_p=0.1),
        "nn.MultiheadAttention": lambda: mha(seq, seq, seq)[0],
    }
    with torch.autocast(device_type, dtype=dtype):
        for name, fn in cases.items():
            assert fn().dtype == dtype, name
    for name, fn in cases.items():
        assert fn().dtype == torch.float32, name + " (no autocast)"
    assert not torch.is_autocast_enabled(device_type)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_autocast_casts_operands_and_mask_and_returns_float32_grads(dev, dtype):
    # the result equals the training forward (the one the autograd function runs) on the operands
    # cast to `dtype` (a float mask too), and the float32 leaves receive float32 gradients of those
    # cast operands
    B, H, L, D = 2, 4, 70, 64
    q, k, v = (randn((B, H, L, D), s).to(dev).requires_grad_() for s in (1, 2, 3))
    mask = torch.from_numpy(np.random.default_rng(4).standard_normal((L, L)).astype(np.float32) * 0.3).to(dev)
    with torch.autocast("cuda", dtype=dtype):
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=True)
    assert out.dtype == dtype
    qc, kc, vc, mc = (t.detach().to(dtype) for t in (q, k, v, mask))
    want = g.flash_attention_train(qc, kc, vc, mc.reshape(1, 1, L, L), 1 / math.sqrt(D), True)[0]
    assert torch.equal(out.detach(), want)
    dout = randn((B, H, L, D), 5, dtype).to(dev)
    out.backward(dout)
    assert q.grad.dtype == k.grad.dtype == v.grad.dtype == torch.float32
    wq, wk, wv = oracle.flash_attention_backward(to_oracle(dout), to_oracle(qc), to_oracle(kc), to_oracle(vc),
                                                 mask=to_oracle(mc), is_causal=True)
    # the engine rounds each gradient to the dtype of the cast operand, then widens it back to
    # float32 for the leaf: one rounding to `dtype`
    assert_close(q.grad, wq, torch.bfloat16, "dq", out_dtype=dtype)
    assert_close(k.grad, wk, torch.bfloat16, "dk", out_dtype=dtype)
    assert_close(v.grad, wv, torch.bfloat16, "dv", out_dtype=dtype)


# ---- views -------------------------------------------------------------------------------------

def _fresh(t):
    return t.detach().clone().contiguous()


def _as_offset(t):
    """A contiguous view that starts in the middle of a larger storage."""
    pad = torch.full((3,) + tuple(t.shape[1:]), JUNK, dtype=t.dtype, device=t.device)
    view = torch.cat([pad, t], dim=0)[3:]
    assert view.is_contiguous() and view.storage_offset() > 0
    return view


def _as_strided(t):
    """A non-contiguous view with the same values."""
    last = t.ndim - 1
    view = t.transpose(0, last).contiguous().transpose(0, last)
    assert not view.is_contiguous()
    return view


KINDS = {"offset": _as_offset, "strided": _as_strided}


def _run(fn, tensors, which=None, kind=None, grad="plain"):
    leaves = [_fresh(t).requires_grad_(True) for t in tensors]
    args = [KINDS[kind](leaf) if (kind is not None and (which is None or i == which)) else leaf
            for i, leaf in enumerate(leaves)]
    out = fn(*args)
    weights = (torch.arange(out.numel(), dtype=torch.float32, device=out.device).reshape(out.shape) * 0.01 + 0.5)
    weights = weights.to(out.dtype)
    if grad == "plain":
        loss = (out * weights).float().sum()
    elif grad == "offset":
        # downstream cat: the gradient that arrives is a slice of a larger one
        loss = (torch.cat([out * 0.0, out], dim=0) * torch.cat([weights, weights], dim=0)).float().sum()
    else:
        # downstream transpose: the gradient that arrives is strided
        last = out.ndim - 1
        loss = (out.transpose(0, last) * weights.transpose(0, last)).float().sum()
    loss.backward()
    return out.detach(), [leaf.grad for leaf in leaves]


def _close(got, want, tol, msg):
    got, want = got.double(), want.double()
    bound = tol * torch.clamp(want.abs(), min=1.0)
    assert got.shape == want.shape, msg
    assert bool(((got - want).abs() <= bound).all()), f"{msg}: max diff {(got - want).abs().max().item():.3e}"


@pytest.mark.parametrize("dtype,shape", [(torch.float32, (2, 2, 5, 4)), (torch.bfloat16, (2, 4, 70, 64)),
                                         (torch.float16, (1, 4, 130, 64))])
@pytest.mark.parametrize("causal", [False, True])
def test_values_and_gradients_do_not_depend_on_views(dev, dtype, shape, causal):
    torch.manual_seed(sum(shape))
    tensors = [torch.randn(shape, device=dev).to(dtype) for _ in range(3)]

    def fn(q, k, v):
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal)

    want, want_grads = _run(fn, tensors)
    variants = [(None, kind, "plain") for kind in KINDS]
    variants += [(i, kind, "plain") for i in range(3) for kind in KINDS]
    variants += [(None, None, "offset"), (None, None, "strided")]
    # the reference's bar is 2e-4 relative for float32; a bf16 / fp16 result differs from
    # another run of the same kernel only by the order of float32 sums, then one rounding
    tol = 2e-4 if dtype == torch.float32 else 2e-3
    for which, kind, grad in variants:
        label = f"{'every argument' if which is None else f'argument {which}'} as {kind or 'fresh'}, {grad} gradient"
        got, got_grads = _run(fn, tensors, which, kind, grad)
        _close(got, want, tol, f"forward ({label})")
        for i, (gg, w) in enumerate(zip(got_grads, want_grads)):
            assert gg is not None and gg.dtype == dtype, label
            _close(gg, w, tol, f"gradient of argument {i} ({label})")
