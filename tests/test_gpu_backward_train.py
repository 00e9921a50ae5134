"""Backward parity at the training workload's shapes: bf16 L = S = 1024, D = 64, causal plus an
additive key-padding mask (gguf_train/_functions.py:1933-1965 restated by the oracle in
float64), so that every key tile of the dK/dV kernel (128 keys each), the causal start of the
query walk and the fast paths for blocks where every (query, key) pair is visible all run; the
same for fp16 D = 128 with GQA groups of 2 and 4 heads; and rows with nothing to attend to, whose
gradient is zero (the reference's composition gives NaN there for -inf masks).

The kernel's float32 gradients are compared before any cast, at 2e-3 * max(1, |ref|) per
element (no output-rounding allowance: the gradients are float32)."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
import oracle

from _util import assert_close, randn, to_oracle

pytestmark = pytest.mark.gpu


def _grads(dev, q, k, v, dout, mask, causal):
    out, lse, out32 = g.flash_attention_train(q.to(dev), k.to(dev), v.to(dev),
                                              None if mask is None else mask.to(dev), 0.0, causal)
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev),
                                            None if mask is None else mask.to(dev),
                                            out if out32 is None else out32, lse, 0.0, causal)
    assert dq.dtype == dk.dtype == dv.dtype == torch.float32
    return out, dq, dk, dv


def _oracle(dout, q, k, v, mask, causal):
    return oracle.flash_attention_backward(to_oracle(dout), to_oracle(q), to_oracle(k), to_oracle(v),
                                           mask=None if mask is None else to_oracle(mask), is_causal=causal)


def _key_padding(B, S, lens):
    mask = torch.zeros(B, 1, 1, S)
    for b, n in enumerate(lens):
        mask[b, ..., int(n):] = float("-inf")
    return mask


CASES = [
    # dtype, B, H, Hkv, L, S, D, causal, valid key lengths
    (torch.bfloat16, 2, 2, 2, 1024, 1024, 64, True, (1024, 717)),   # the training workload's shape
    (torch.bfloat16, 2, 2, 2, 1024, 1024, 64, True, (512, 1000)),
    (torch.bfloat16, 1, 4, 4, 1024, 1024, 64, False, (843,)),
    (torch.float16, 1, 4, 2, 384, 384, 128, True, (333,)),           # GQA 2, key tiles 0..2
    (torch.float16, 2, 4, 1, 300, 400, 128, False, (400, 350)),      # GQA 4, L != S
    (torch.bfloat16, 1, 8, 2, 320, 320, 128, True, (257,)),
    (torch.float16, 2, 4, 2, 520, 520, 64, True, (520, 301)),
    # caught by a random-shape sweep while fp16 used single operands: early causal keys collect the
    # P of every row (dV 1.27x the bar), and two visible keys per row left the forward's fp16 row
    # sum 1.6e-4 off in the log-sum-exp (dV 1.01x)
    (torch.float16, 2, 4, 2, 155, 155, 128, True, (155, 61)),
    (torch.float16, 1, 4, 2, 285, 16, 64, False, (2,)),
]


@pytest.mark.parametrize("dtype,B,H,Hkv,L,S,D,causal,lens", CASES)
def test_backward_at_training_shapes(dev, dtype, B, H, Hkv, L, S, D, causal, lens):
    seed = L + 3 * S + D + H
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    dout = randn((B, H, L, D), seed + 3, dtype)
    mask = _key_padding(B, S, lens)
    _, dq, dk, dv = _grads(dev, q, k, v, dout, mask, causal)
    wq, wk, wv = _oracle(dout, q, k, v, mask, causal)
    what = f"{dtype} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} lens={lens}"
    worst = [assert_close(got, want, torch.bfloat16, f"{name} {what}", out_dtype=torch.float32)
             for name, got, want in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv))]
    print(f"[bwd-ratio] {what}: dq {worst[0]:.3f} dk {worst[1]:.3f} dv {worst[2]:.3f}", flush=True)
    # keys past a sequence's valid length are never visible: exactly zero
    for b, n in enumerate(lens):
        assert not dk[b, :, n:].any() and not dv[b, :, n:].any()


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float16, 128)])
def test_sequence_with_no_valid_key_has_zero_gradient(dev, dtype, D):
    # key padding with a valid length of 0: every row of sequence 0 has nothing to attend to.
    # Its output and all of its gradients are 0; sequence 1 matches the oracle run on it alone.
    B, H, Hkv, L, S = 2, 4, 2, 200, 200
    q, k, v = randn((B, H, L, D), 21, dtype), randn((B, Hkv, S, D), 22, dtype), randn((B, Hkv, S, D), 23, dtype)
    dout = randn((B, H, L, D), 24, dtype)
    mask = _key_padding(B, S, (0, 150))
    out, dq, dk, dv = _grads(dev, q, k, v, dout, mask, True)
    assert not out[0].any()
    assert not dq[0].any() and not dk[0].any() and not dv[0].any()
    wq, wk, wv = _oracle(dout[1:], q[1:], k[1:], v[1:], mask[1:], True)
    assert_close(dq[1:], wq, torch.bfloat16, "dq", out_dtype=torch.float32)
    assert_close(dk[1:], wk, torch.bfloat16, "dk", out_dtype=torch.float32)
    assert_close(dv[1:], wv, torch.bfloat16, "dv", out_dtype=torch.float32)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float16, 128)])
@pytest.mark.parametrize("kind", ["additive", "bool"])
@pytest.mark.parametrize("causal", [False, True])
def test_fully_masked_query_row_has_zero_gradient(dev, dtype, D, kind, causal):
    # a per-element (L, S) mask whose last query row blocks every key: that row's output and dq
    # are 0 and it adds nothing to dk / dv, so the other gradients equal the oracle's on the
    # inputs without that row (the last row: removing it moves no causal boundary)
    B, H, Hkv, L, S = 1, 4, 2, 160, 300
    q, k, v = randn((B, H, L, D), 31, dtype), randn((B, Hkv, S, D), 32, dtype), randn((B, Hkv, S, D), 33, dtype)
    dout = randn((B, H, L, D), 34, dtype)
    rng = np.random.default_rng(35)
    allowed = torch.from_numpy(rng.random((L, S)) < 0.7)
    allowed[:, 0] = True
    allowed[L - 1] = False
    mask = allowed if kind == "bool" else torch.zeros(L, S).masked_fill(~allowed, float("-inf"))
    out, dq, dk, dv = _grads(dev, q, k, v, dout, mask, causal)
    assert not out[:, :, L - 1].any() and not dq[:, :, L - 1].any()
    assert not torch.isnan(dk).any() and not torch.isnan(dv).any()
    wq, wk, wv = _oracle(dout[:, :, :-1], q[:, :, :-1], k, v, mask[:-1], causal)
    assert_close(dq[:, :, :-1], wq, torch.bfloat16, "dq", out_dtype=torch.float32)
    assert_close(dk, wk, torch.bfloat16, "dk", out_dtype=torch.float32)
    assert_close(dv, wv, torch.bfloat16, "dv", out_dtype=torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_training_forward_float32_output_without_rounding_allowance(dev, dtype, D):
    # the training forward's float32 output (before rounding to the input dtype) against the
    # float64 oracle at 2e-3 * max(1, |ref|), with no allowance for output rounding: the
    # kernel's own error
    B, H, Hkv, L, S = 2, 4, 2, 1024, 1024
    seed = 40 + D
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    mask = _key_padding(B, S, (1024, 611))
    _, _, out32 = g.flash_attention_train(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, True)
    want = oracle.flash_attention(to_oracle(q), to_oracle(k), to_oracle(v), mask=to_oracle(mask), is_causal=True,
                                  out_dtype=oracle.F64)
    worst = assert_close(out32, want, torch.bfloat16, "out32", out_dtype=torch.float32)
    print(f"[fwd32-ratio] {dtype} D{D}: {worst:.3f}", flush=True)
