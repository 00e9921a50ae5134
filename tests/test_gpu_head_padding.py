"""Float16/bfloat16 attention with head sizes other than 64 and 128 (up to 128, more than one query
row) runs on the MFMA kernels with the heads zero-padded: forward (output, float32 output,
log-sum-exp) and backward against the float64 oracle on the same rounded inputs, with masks, GQA,
causal / not, dropout, D != Dv, and a timing-independent check that padding is what ran (the
result equals the unpadded kernels' on explicitly zero-padded inputs, bit for bit)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as tF

import gguf_train_amd as g
import oracle

from _util import assert_close, oracle_forward, randn, to_oracle

pytestmark = pytest.mark.gpu


CASES = [
    # dtype, B, H, Hkv, L, S, D, Dv, causal, mask
    (torch.float16, 2, 4, 2, 150, 150, 96, 96, True, None),
    (torch.bfloat16, 1, 4, 4, 129, 200, 80, 80, False, "pad"),
    (torch.float16, 2, 2, 1, 64, 64, 32, 32, True, "bool"),
    (torch.bfloat16, 1, 2, 2, 100, 77, 48, 48, False, "add"),
    (torch.float16, 1, 4, 2, 90, 90, 112, 112, True, None),
    (torch.bfloat16, 2, 2, 2, 70, 70, 96, 64, False, None),
]


def _mask(kind, B, H, L, S, seed):
    rng = np.random.default_rng(seed)
    if kind is None:
        return None
    if kind == "bool":
        m = torch.from_numpy(rng.random((L, S)) < 0.8)
        m[:, 0] = True
        return m
    if kind == "add":
        return torch.from_numpy(rng.standard_normal((B, H, L, S)).astype(np.float32))
    m = torch.zeros(B, 1, 1, S)
    m[0, ..., S - S // 3:] = float("-inf")
    return m


@pytest.mark.parametrize("dtype,B,H,Hkv,L,S,D,Dv,causal,mkind", CASES)
def test_padded_heads_match_the_oracle(dev, dtype, B, H, Hkv, L, S, D, Dv, causal, mkind):
    seed = L + S + D + Dv
    q, k = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype)
    v, dout = randn((B, Hkv, S, Dv), seed + 2, dtype), randn((B, H, L, Dv), seed + 3, dtype)
    mask = _mask(mkind, B, H, L, S, seed)
    md = None if mask is None else mask.to(dev)
    out, lse, out32 = g.flash_attention_train(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal)
    assert out.shape == (B, H, L, Dv) and out32.shape == (B, H, L, Dv)
    want, want_lse = oracle_forward(q, k, v, mask=mask, is_causal=causal, return_lse=True)
    assert_close(out, want, dtype, "out")
    assert_close(out32, want, dtype, "out32", out_dtype=torch.float32)
    # float16: the row sum adds the float16-rounded probabilities that also weight V (each within
    # 2^-11 relative), so the log-sum-exp is within log(1 + 2^-11) < 2^-11; bfloat16 sums float32
    assert np.abs(lse.cpu().double().numpy() - want_lse).max() < (2.0 ** -11 if dtype == torch.float16 else 1e-4)
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), md, out32, lse, 0.0, causal)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    wq, wk, wv = oracle.flash_attention_backward(to_oracle(dout), to_oracle(q), to_oracle(k), to_oracle(v),
                                                 mask=None if mask is None else to_oracle(mask), is_causal=causal)
    for name, got, ref in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv)):
        assert_close(got, ref, torch.bfloat16, name, out_dtype=torch.float32)


# D % 8 == 0: the 8-element pad / unpad copies; 100 and 36: the one-element copies
@pytest.mark.parametrize("dtype,D", [(torch.float16, 96), (torch.bfloat16, 40), (torch.float16, 100),
                                     (torch.bfloat16, 36)])
def test_padding_is_the_unpadded_kernel_on_zero_padded_heads(dev, dtype, D):
    B, H, L, S = 2, 4, 130, 130
    Dp = 64 if D <= 64 else 128
    q, k, v, dout = (randn((B, H, n, D), i, dtype).to(dev) for i, n in enumerate((L, S, S, L)))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))  # the default scale, 1 / sqrt(D) in float32
    out, lse, out32 = g.flash_attention_train(q, k, v, None, 0.0, True)
    pad = lambda t: tF.pad(t, (0, Dp - D))
    ref, ref_lse, ref32 = g.flash_attention_train(pad(q), pad(k), pad(v), None, scale, True)
    assert torch.equal(out, ref[..., :D]) and torch.equal(out32, ref32[..., :D]) and torch.equal(lse, ref_lse)
    grads = g.flash_attention_backward(dout, q, k, v, None, out32, lse, 0.0, True)
    ref_grads = g.flash_attention_backward(pad(dout), pad(q), pad(k), pad(v), None, ref32, ref_lse, scale, True)
    for a, b in zip(grads, ref_grads):
        assert torch.equal(a, b[..., :D])
        assert not b[..., D:].any()


def test_padded_heads_with_dropout(dev):
    B, H, L, S, D, p, seed = 1, 2, 96, 96, 80, 0.3, 17
    q, k, v, dout = (randn((B, H, n, D), i + 5, torch.bfloat16) for i, n in enumerate((L, S, S, L)))
    out, lse, out32 = g.flash_attention_dropout(q.to(dev), k.to(dev), v.to(dev), None, 0.0, True, p, seed)
    dq, dk, dv = g.flash_attention_dropout_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), None, out32, lse,
                                                    0.0, True, p, seed)
    keep = oracle.dropout_keep(B, H, L, S, p, seed)
    ref, (rq, rk, rv) = oracle.attention_dropout(to_oracle(q), to_oracle(k), to_oracle(v), keep, p, is_causal=True,
                                                 dout=to_oracle(dout), out_dtype=oracle.F64)
    assert_close(out32, ref, torch.bfloat16, "out32", out_dtype=torch.float32)
    for name, got, want in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert_close(got, want, torch.bfloat16, name, out_dtype=torch.float32)


def test_padded_heads_read_strided_views(dev):
    # (B, L, H, D) storage viewed as (B, H, L, D): the padding copy reads the strides
    B, H, L, D = 2, 4, 90, 80
    base = [randn((B, L, H, D), 30 + i, torch.float16).to(dev) for i in range(4)]
    views = [t.transpose(1, 2) for t in base]
    dense = [t.contiguous() for t in views]
    assert not views[0].is_contiguous()
    out, lse, out32 = g.flash_attention_train(views[0], views[1], views[2], None, 0.0, True)
    ref, ref_lse, ref32 = g.flash_attention_train(dense[0], dense[1], dense[2], None, 0.0, True)
    assert torch.equal(out, ref) and torch.equal(out32, ref32) and torch.equal(lse, ref_lse)
    grads = g.flash_attention_backward(views[3], views[0], views[1], views[2], None, out32, lse, 0.0, True)
    ref_grads = g.flash_attention_backward(dense[3], dense[0], dense[1], dense[2], None, ref32, ref_lse, 0.0, True)
    for a, b in zip(grads, ref_grads):
        assert torch.equal(a, b)
