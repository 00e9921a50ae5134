"""Dropout of the attention probabilities on the GPU against the oracle.

The reference composes scaled_dot_product_attention with dropout_p > 0 from explicit ops
(gguf_train/nn/functional.py:750-767; MultiheadAttention likewise on its weights,
transformer.py:153-166); the oracle restates that composition in float64 for a given keep mask
(tests/test_oracle_dropout.py pins it against torch.autograd), and the keep mask is the oracle's
Philox4x32-10 layout (pinned against rocRAND and the Random123 known answers).  Here:
* the library's decisions (gt_attention_dropout_mask) equal the oracle's bit for bit;
* the fused forward (output, float32 output, log-sum-exp) and backward (dQ, dK, dV) equal the
  oracle's composition under those decisions, on the MFMA kernels (float16/bfloat16, head size
  64/128: several key tiles, causal, bool / additive / key-padding masks, GQA, L = 1) and the
  generic ones (float32, float64, odd head sizes), p from 0.1 to 1;
* scaled_dot_product_attention and MultiheadAttention draw their seed from torch's generator:
  torch.manual_seed reproduces them, checkpoint's recomputation gives the same gradients, and
  MultiheadAttention's returned weights are the dropped ones.
Tolerances as the other parity tests (tests/_util.py); rows always see at least one key (the
reference's -1e9 fill would average V over a fully blocked row, where the library gives 0)."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
import oracle
from gguf_train_amd._functions import draw_dropout_seed
from gguf_train_amd.nn import functional as F

from _util import assert_close, randn, to_oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,H,L,S", [(1, 1, 1, 1), (2, 3, 5, 7), (1, 2, 33, 1000), (2, 1, 4, 4), (1, 1, 3, 130)])
@pytest.mark.parametrize("p,seed,offset", [(0.1, 1, 0), (0.5, 2 ** 64 - 1, 2 ** 40 + 3), (0.9, 12345, 7),
                                           (1.0, 3, 0), (0.0, 4, 0)])
def test_decisions_match_the_oracle(dev, B, H, L, S, p, seed, offset):
    got = g.attention_dropout_mask((B, H, L, S), p, seed, offset, device=dev)
    assert got.dtype == torch.bool and got.shape == (B, H, L, S)
    want = oracle.dropout_keep(B, H, L, S, p, seed, offset)
    assert np.array_equal(got.cpu().numpy(), want)


def _mask(kind, B, H, L, S, lens, seed):
    gen = np.random.default_rng(seed)
    if kind is None:
        return None
    if kind == "bool":
        m = torch.from_numpy(gen.random((L, S)) > 0.3)
        m[:, 0] = True
        return m
    if kind == "add":
        return torch.from_numpy(gen.standard_normal((B, H, L, S)).astype(np.float32))
    m = torch.zeros(B, 1, 1, S)  # "pad": key padding (a float mask that does not depend on the row)
    for b, n in enumerate(lens):
        m[b, ..., int(n):] = float("-inf")
    return m


CASES = [
    # dtype, B, H, Hkv, L, S, D, causal, mask, key lengths, p
    (torch.bfloat16, 2, 4, 2, 300, 300, 64, True, "pad", (300, 211), 0.1),
    (torch.float16, 1, 4, 4, 257, 257, 128, False, None, (), 0.5),
    (torch.bfloat16, 1, 2, 2, 200, 333, 128, True, "bool", (), 0.3),
    (torch.float16, 2, 2, 1, 130, 260, 64, False, "add", (), 0.2),
    (torch.bfloat16, 1, 2, 2, 1024, 1024, 64, True, "pad", (1024,), 0.1),
    (torch.float16, 2, 8, 2, 1, 500, 128, False, "pad", (500, 317), 0.3),
    (torch.float32, 2, 2, 2, 70, 90, 64, True, None, (), 0.25),
    (torch.float64, 1, 3, 1, 33, 47, 40, False, "add", (), 0.6),
    (torch.float16, 1, 2, 2, 40, 41, 40, True, "bool", (), 0.4),
    (torch.bfloat16, 1, 2, 2, 64, 64, 64, True, None, (), 1.0),
    (torch.float32, 1, 2, 1, 20, 30, 300, True, None, (), 0.3),        # generic kernels without LDS staging
    (torch.float16, 1, 2, 2, 50, 61, 256, False, "bool", (), 0.5),     # generic, LDS-staged, 4 blocks of 64 dims
    (torch.bfloat16, 2, 4, 4, 96, 130, 128, True, "pad", (130, 67), 0.05),
    # per-element masks whose keys come in whole 4-key groups (S % 4 == 0): the 4-key mask loads
    # of the forward and dQ kernels (bool: mode 5, float: mode 6) together with dropout
    (torch.float16, 1, 2, 2, 256, 256, 64, True, "bool", (), 0.3),
    (torch.float16, 1, 2, 2, 256, 256, 64, False, "bool", (), 0.2),
    (torch.bfloat16, 1, 2, 1, 192, 320, 128, True, "bool", (), 0.1),
    (torch.bfloat16, 1, 2, 2, 128, 192, 128, True, "add", (), 0.15),
    # few keys per row with fp16: a random-shape sweep found dK at 1.23x the bar while the fp16
    # dropout forward fed P.V single fp16 probabilities (its float32 output forms rowsum(dO.O))
    (torch.float16, 1, 4, 2, 141, 3, 128, False, "bool", (), 0.5),
]


@pytest.mark.parametrize("dtype,B,H,Hkv,L,S,D,causal,mkind,lens,p", CASES)
def test_forward_and_backward_match_the_oracle(dev, dtype, B, H, Hkv, L, S, D, causal, mkind, lens, p):
    s0 = L + 7 * S + D + H
    q, k, v = randn((B, H, L, D), s0, dtype), randn((B, Hkv, S, D), s0 + 1, dtype), randn((B, Hkv, S, D), s0 + 2, dtype)
    dout = randn((B, H, L, D), s0 + 3, dtype)
    mask = _mask(mkind, B, H, L, S, lens, s0)
    if mask is not None and mask.dtype != torch.bool:
        mask = mask.to(torch.float64 if dtype == torch.float64 else torch.float32)
    seed, offset = 1000 + s0, 3
    md = None if mask is None else mask.to(dev)
    out, lse, out32 = g.flash_attention_dropout(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal, p, seed, offset)
    dq, dk, dv = g.flash_attention_dropout_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), md,
                                                    out if out32 is None else out32, lse, 0.0, causal, p, seed,
                                                    offset)
    keep = oracle.dropout_keep(B, H, L, S, p, seed, offset)
    ref, (rdq, rdk, rdv) = oracle.attention_dropout(to_oracle(q), to_oracle(k), to_oracle(v), keep, p,
                                                    mask=None if mask is None else to_oracle(mask),
                                                    is_causal=causal, dout=to_oracle(dout), out_dtype=oracle.F64)
    print(f"[dropout] {dtype} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} mask={mkind} p={p}", flush=True)
    worst = [assert_close(out, ref, dtype, "out")]
    if out32 is not None:
        worst.append(assert_close(out32, ref, dtype, "out32", out_dtype=torch.float32))
    # the log-sum-exp is that of the undropped scores
    _, want_lse = oracle.flash_attention(to_oracle(q), to_oracle(k), to_oracle(v),
                                         mask=None if mask is None else to_oracle(mask), is_causal=causal,
                                         out_dtype=oracle.F64, return_lse=True)
    assert np.abs(lse.cpu().double().numpy() - want_lse).max() < (1e-10 if dtype == torch.float64 else 1e-4)
    gd = torch.float32 if dtype in (torch.float16, torch.bfloat16) else None
    for name, got, want in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        worst.append(assert_close(got, want, dtype, name, out_dtype=gd))
    print(f"[dropout-ratio] worst {max(worst):.3f}", flush=True)
    if p == 1.0:
        assert not out.any() and not dq.any() and not dk.any() and not dv.any()


@pytest.mark.parametrize("dtype,D,S", [(torch.bfloat16, 64, 300), (torch.float16, 128, 257)])
def test_backward_without_the_decision_buffer_gives_the_same_bits(dev, monkeypatch, dtype, D, S):
    # past GT_ATTN_DROPOUT_BITS_MAX bytes the dK/dV kernel draws the decisions itself
    B, H, L, p, seed = 2, 4, 200, 0.2, 31
    q, k, v, dout = (randn(shape, i, dtype).to(dev) for i, shape in
                     enumerate([(B, H, L, D), (B, 2, S, D), (B, 2, S, D), (B, H, L, D)]))
    mask = _mask("pad", B, H, L, S, (S, S - 77), 1).to(dev)
    out, lse, out32 = g.flash_attention_dropout(q, k, v, mask, 0.0, True, p, seed)
    with_buffer = g.flash_attention_dropout_backward(dout, q, k, v, mask, out32, lse, 0.0, True, p, seed)
    monkeypatch.setenv("GT_ATTN_DROPOUT_BITS_MAX", "0")
    drawn = g.flash_attention_dropout_backward(dout, q, k, v, mask, out32, lse, 0.0, True, p, seed)
    for a, b in zip(with_buffer, drawn):
        assert torch.equal(a, b)


def test_same_seed_same_bits_other_offset_other_mask(dev):
    q, k, v = (randn((2, 4, 128, 64), i, torch.bfloat16).to(dev) for i in range(3))
    a = g.flash_attention_dropout(q, k, v, None, 0.0, True, 0.2, 77, 0)[0]
    b = g.flash_attention_dropout(q, k, v, None, 0.0, True, 0.2, 77, 0)[0]
    c = g.flash_attention_dropout(q, k, v, None, 0.0, True, 0.2, 77, 1)[0]
    assert torch.equal(a, b) and not torch.equal(a, c)


@pytest.mark.parametrize("dtype,D,avg", [(torch.float16, 64, False), (torch.bfloat16, 128, True),
                                         (torch.float32, 40, False)])
def test_weights_are_the_dropped_probabilities(dev, dtype, D, avg):
    B, H, L, S, p, seed = 2, 3, 37, 70, 0.3, 555
    q, k, v = randn((B, H, L, D), 1, dtype), randn((B, H, S, D), 2, dtype), randn((B, H, S, D), 3, dtype)
    mask = _mask("pad", B, H, L, S, (70, 41), 0)
    out, lse, _ = g.flash_attention_dropout(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, True, p, seed)
    w = g.attention_weights_dropout(q.to(dev), k.to(dev), mask.to(dev), lse, 0.0, True, avg, p, seed)
    keep = torch.from_numpy(oracle.dropout_keep(B, H, L, S, p, seed))
    qd, kd = q.double(), k.double()
    sc = qd.matmul(kd.transpose(-2, -1)) * float(np.float32(1 / np.sqrt(D)))
    sc = sc + torch.ones(L, S, dtype=torch.float64).triu(1) * (-1e9) + mask.double()
    want = torch.softmax(sc, dim=-1) * keep.double() / (1 - p)
    if avg:
        want = want.mean(dim=1)
    assert_close(w, want.numpy(), dtype, "weights")


def test_sdpa_follows_torch_seed_and_checkpoint(dev):
    q0, k0, v0 = (randn((2, 4, 96, 64), i + 10, torch.bfloat16).to(dev) for i in range(3))
    torch.manual_seed(123)
    a = F.scaled_dot_product_attention(q0, k0, v0, dropout_p=0.25, is_causal=True)
    torch.manual_seed(123)
    seed = draw_dropout_seed()
    b = g.flash_attention_dropout(q0, k0, v0, None, 0.0, True, 0.25, seed)[0]
    assert torch.equal(a, b)

    def run(use_ckpt):
        q, k, v = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
        torch.manual_seed(9)
        fn = lambda x, y, z: F.scaled_dot_product_attention(x, y, z, dropout_p=0.25, is_causal=True)
        if use_ckpt:
            out = torch.utils.checkpoint.checkpoint(fn, q, k, v, use_reentrant=False)
        else:
            out = fn(q, k, v)
        out.float().sum().backward()
        return out, q.grad, k.grad, v.grad

    plain, ck = run(False), run(True)
    for x, y in zip(plain, ck):
        assert torch.equal(x, y)


def test_multihead_attention_returns_the_dropped_weights(dev):
    torch.manual_seed(0)
    mha = g.nn.MultiheadAttention(64, 4, dropout=0.2, batch_first=True).to(dev)
    mha.train()
    x = torch.randn(2, 50, 64, device=dev)
    torch.manual_seed(5)
    out, w = mha(x, x, x, need_weights=True, average_attn_weights=False)
    torch.manual_seed(5)
    seed = draw_dropout_seed()
    with torch.no_grad():
        # the same projections the module makes, then the weights' definition
        qkv = torch.nn.functional.linear(x, mha.in_proj_weight, mha.in_proj_bias)
        q, k, v = (t.reshape(2, 50, 4, 16).transpose(1, 2).double() for t in qkv.chunk(3, dim=-1))
        keep = torch.from_numpy(oracle.dropout_keep(2, 4, 50, 50, 0.2, seed)).to(dev)
        pw = torch.softmax(q.matmul(k.transpose(-2, -1)) * float(np.float32(0.25)), dim=-1) * keep / 0.8
        # the output is the dropped weights applied to V, through the output projection
        ref = torch.nn.functional.linear(pw.matmul(v).transpose(1, 2).reshape(2, 50, 64).float(), mha.out_proj.weight,
                                         mha.out_proj.bias)
    assert_close(w, pw.cpu().numpy(), torch.float32, "weights")
    assert_close(out, ref.cpu().numpy(), torch.float32, "out")
    out.sum().backward()
    assert mha.in_proj_weight.grad is not None and torch.isfinite(mha.in_proj_weight.grad).all()
