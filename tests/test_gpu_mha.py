"""MultiheadAttention on the GPU against the reference test's explicit implementation
(tests/test_pooling_and_attention.py:176-260): every layout, need_weights on/off, nine mask
combinations."""

import itertools
import math

import pytest
import torch

from gguf_train_amd.nn import MultiheadAttention

pytestmark = pytest.mark.gpu
NEG_INF = float("-inf")


def mha_reference(m, q, k, v, key_padding_mask=None, attn_mask=None):
    E, H = m.embed_dim, m.num_heads
    D = E // H
    B, L, _ = q.shape
    S = k.shape[1]

    def project(x, i):
        y = x.matmul(m.in_proj_weight[i * E:(i + 1) * E].transpose(0, 1)) + m.in_proj_bias[i * E:(i + 1) * E]
        return y.reshape(B, x.shape[1], H, D).transpose(1, 2)

    scores = project(q, 0).matmul(project(k, 1).transpose(-2, -1)) / math.sqrt(D)
    for mask, shape in ((attn_mask, None), (key_padding_mask, (B, 1, 1, S))):
        if mask is None:
            continue
        if shape is None:
            shape = (1, 1, L, S) if mask.ndim == 2 else (B, H, L, S)
        mask = mask.reshape(shape)
        scores = scores.masked_fill(mask, NEG_INF) if mask.dtype == torch.bool else scores + mask
    weights = torch.softmax(scores, dim=-1)
    out = weights.matmul(project(v, 2)).transpose(1, 2).reshape(B, L, E)
    return out.matmul(m.out_proj.weight.transpose(0, 1)) + m.out_proj.bias, weights


def masks(batch, L, S, H, dev):
    kpm = torch.zeros(batch, S, dtype=torch.bool)
    kpm[:, -1] = True
    if batch > 1:
        kpm[1, 1] = True
    causal = torch.triu(torch.ones(L, S), diagonal=1).bool()
    per_head = torch.rand(batch * H, L, S) < 0.3
    per_head[:, :, 0] = False
    d = {
        "none": (None, None),
        "bool kpm": (kpm, None),
        "float kpm": (torch.zeros(batch, S).masked_fill(kpm, NEG_INF), None),
        "bool attn": (None, causal),
        "float attn": (None, torch.zeros(L, S).masked_fill(causal, NEG_INF)),
        "3D bool attn": (None, per_head),
        "bool kpm + bool attn": (kpm, causal),
        "bool kpm + float attn": (kpm, torch.zeros(L, S).masked_fill(causal, NEG_INF)),
        "float kpm + 3D bool attn": (torch.zeros(batch, S).masked_fill(kpm, NEG_INF), per_head),
    }
    return {n: tuple(None if t is None else t.to(dev) for t in pair) for n, pair in d.items()}


def test_matches_the_reference_in_every_layout(dev):
    E, H, B, L, S = 8, 2, 3, 4, 5
    torch.manual_seed(0)
    for batch_first, batched, need_weights in itertools.product((False, True), (True, False), (True, False)):
        m = MultiheadAttention(E, H, batch_first=batch_first).to(dev)
        with torch.no_grad():
            m.in_proj_bias.copy_(torch.randn(3 * E) * 0.1)
        m.eval()
        batch = B if batched else 1
        q, k, v = (torch.randn(batch, n, E, device=dev) for n in (L, S, S))

        def layout(x):
            if not batched:
                return x[0]
            return x if batch_first else x.transpose(0, 1)

        for name, (kpm, am) in masks(batch, L, S, H, dev).items():
            with torch.no_grad():
                want, weights = mha_reference(m, q, k, v, kpm, am)
                out, got_w = m(layout(q), layout(k), layout(v), key_padding_mask=kpm if (batched or kpm is None) else kpm[0],
                               attn_mask=am, need_weights=need_weights)
            assert (out - layout(want)).abs().max().item() < 1e-4, name
            if need_weights:
                avg = weights.mean(dim=1)
                assert (got_w - (avg if batched else avg[0])).abs().max().item() < 1e-4, name
            else:
                assert got_w is None


def test_gradients_reach_every_parameter(dev):
    torch.manual_seed(4)
    m = MultiheadAttention(8, 2, batch_first=True).to(dev)
    x = torch.randn(2, 4, 8, device=dev)
    kpm = torch.tensor([[False, False, False, True], [False, False, True, True]], device=dev)
    causal = torch.triu(torch.ones(4, 4, device=dev), diagonal=1).bool()
    for need_weights in (True, False):
        m.zero_grad()
        out, _ = m(x, x, x, key_padding_mask=kpm, attn_mask=causal, need_weights=need_weights)
        out.sum().backward()
        for name, p in m.named_parameters():
            assert p.grad is not None and torch.isfinite(p.grad).all(), name


def test_half_precision_with_a_head_size_the_kernels_pad(dev):
    # head size 96: the fused kernels run with heads zero-padded to 128 (forward and backward)
    torch.manual_seed(5)
    E, H, B, L = 384, 4, 2, 40
    m = MultiheadAttention(E, H, batch_first=True).to(dev).half()
    x = (torch.randn(B, L, E, device=dev) * 0.5).half().requires_grad_()
    causal = torch.triu(torch.ones(L, L, device=dev), diagonal=1).bool()
    out, _ = m(x, x, x, attn_mask=causal, need_weights=False)
    m32 = MultiheadAttention(E, H, batch_first=True).to(dev)
    m32.load_state_dict({k: t.float() for k, t in m.state_dict().items()})
    with torch.no_grad():
        want, _ = mha_reference(m32, x.float(), x.float(), x.float(), None, causal)
    err = ((out.float() - want).abs() / want.abs().clamp_min(1.0)).max().item()
    assert err < 5e-3, err
    out.float().sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    for name, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), name


@pytest.mark.parametrize("dtype,tol", [(torch.float16, 5e-3), (torch.bfloat16, 3e-2)])
def test_reduced_precision_masks_and_weights(dev, dtype, tol):
    # every mask kind with float16 / bfloat16 parameters and inputs, with and without the
    # returned weights, against the float32 composition on the same rounded values
    torch.manual_seed(6)
    E, H, B, L, S = 256, 4, 2, 24, 30
    m = MultiheadAttention(E, H, batch_first=True).to(dev).to(dtype)
    m32 = MultiheadAttention(E, H, batch_first=True).to(dev)
    m32.load_state_dict({k: t.float() for k, t in m.state_dict().items()})
    q = (torch.randn(B, L, E, device=dev) * 0.5).to(dtype)
    kv = (torch.randn(B, S, E, device=dev) * 0.5).to(dtype)
    for name, (kpm, am) in masks(B, L, S, H, dev).items():
        for need_weights in (False, True):
            with torch.no_grad():
                want, weights = mha_reference(m32, q.float(), kv.float(), kv.float(), kpm, am)
                out, got_w = m(q, kv, kv, key_padding_mask=kpm, attn_mask=am, need_weights=need_weights)
            err = ((out.float() - want).abs() / want.abs().clamp_min(1.0)).max().item()
            assert err < tol, (name, need_weights, err)
            if need_weights:
                assert (got_w.float() - weights.mean(dim=1)).abs().max().item() < tol, (name, "weights")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_reduced_precision_training_with_dropout(dev, dtype):
    torch.manual_seed(7)
    E, H, B, L = 256, 4, 2, 24
    m = MultiheadAttention(E, H, dropout=0.1, batch_first=True).to(dev).to(dtype)
    m.train()
    x = (torch.randn(B, L, E, device=dev) * 0.5).to(dtype).requires_grad_()
    kpm = torch.zeros(B, L, dtype=torch.bool, device=dev)
    kpm[:, -3:] = True
    for need_weights in (False, True):
        m.zero_grad()
        x.grad = None
        out, w = m(x, x, x, key_padding_mask=kpm, need_weights=need_weights)
        assert out.shape == (B, L, E) and torch.isfinite(out.float()).all()
        if need_weights:
            assert w.shape == (B, L, L) and torch.isfinite(w.float()).all()
        out.float().sum().backward()
        assert torch.isfinite(x.grad.float()).all()
        for name, p in m.named_parameters():
            assert p.grad is not None and torch.isfinite(p.grad.float()).all(), name


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fully_padded_sequence_is_the_same_under_autocast(dev, dtype):
    # a sequence whose every key is padded: the boolean key_padding_mask becomes -1e9 in the
    # scores' dtype as in the reference (transformer.py:187-188), i.e. -inf in float16 and a
    # finite -1e9 in bfloat16; either way the sequence's rows have nothing visible and give 0,
    # so its outputs are the out_proj bias; the module run under autocast (which lowers the
    # mask with q/k/v) equals the module cast to `dtype`, for need_weights on and off
    torch.manual_seed(5)
    m = MultiheadAttention(64, 4, batch_first=True).to(dev)
    x = torch.randn(2, 8, 64, device=dev)
    kpm = torch.zeros(2, 8, dtype=torch.bool, device=dev)
    kpm[0] = True
    kpm[1, 5:] = True
    half = MultiheadAttention(64, 4, batch_first=True).to(dev)
    half.load_state_dict(m.state_dict())
    half = half.to(dtype)
    for need_weights in (False, True):
        with torch.no_grad():
            with torch.autocast("cuda", dtype=dtype):
                got, w_got = m(x, x, x, key_padding_mask=kpm, need_weights=need_weights)
            want, w_want = half(x.to(dtype), x.to(dtype), x.to(dtype), key_padding_mask=kpm, need_weights=need_weights)
        assert got.dtype == want.dtype == dtype
        assert torch.isfinite(got).all() and torch.isfinite(want).all()
        tol = 2e-2 if dtype == torch.bfloat16 else 2e-3
        assert torch.allclose(got.float(), want.float(), atol=tol, rtol=tol), (need_weights, (got - want).abs().max())
        assert torch.equal(want[0], half.out_proj.bias.expand(8, 64)), need_weights
        if need_weights:
            assert not w_got[0].any() and not w_want[0].any()
