"""Explicit attention weights over float32 q/k (attn_weights_f32_kernel: head sizes 64 and 128,
S^T on v_mfma_f32_32x32x2_f32) against the float64 oracle's softmax at the float32 bar
(max-abs 1e-4): GQA, causal or not, key counts that are and are not multiples of 4 (16-byte or
4-byte stores), per head or averaged over the heads, key-padding, bool and float per-element
masks, the invariant sum_s P[l, s] v[s] = the oracle's output row, and the launch log naming the
kernel (other head sizes: the generic kernel)."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C, _ops

import oracle
from _util import assert_close, oracle_forward, randn, to_oracle
from test_gpu_attention_weights import oracle_weights

pytestmark = pytest.mark.gpu


def _weights(dev, q, k, v, mask, causal, average):
    md = None if mask is None else mask.to(dev)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal)
    w = _ops.attention_weights(q.to(dev), k.to(dev), md, lse, 0.0, causal, average)
    return w, _C.last_launch()


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal,L,S", [(False, 70, 200), (True, 150, 150), (False, 129, 66), (True, 200, 257)])
@pytest.mark.parametrize("average", [False, True])
def test_float32_weights_match_the_oracle(dev, D, causal, L, S, average):
    B, H, Hkv = 2, 4, 2
    seed = D + L + S + (7 if causal else 0)
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    mask = torch.zeros(B, 1, 1, S)
    mask[1, ..., S - 9:] = float("-inf")
    w, launch = _weights(dev, q, k, v, mask, causal, average)
    what = f"D={D} causal={causal} L={L} S={S} average={average}"
    assert launch == f"weights mfma f32 D={D}", (what, launch)
    assert w.dtype == torch.float32 and w.shape == ((B, L, S) if average else (B, H, L, S))
    want = oracle_weights(q, k, mask, causal, 1.0 / np.sqrt(D))
    assert_close(w, want.mean(axis=1) if average else want, torch.float32, what)
    if not average:
        # the weights reproduce the attention output
        vd = np.repeat(oracle.to_f64(to_oracle(v)), H // Hkv, axis=1)
        pv = np.einsum("bhls,bhsd->bhld", w.double().cpu().numpy(), vd)
        assert_close(pv, oracle_forward(q, k, v, mask=mask, is_causal=causal), torch.float32, "P.V " + what)


@pytest.mark.parametrize("average", [False, True])
def test_float32_weights_with_per_element_masks(dev, average):
    B, H, L, S, D = 2, 4, 90, 130, 64
    q, k, v = randn((B, H, L, D), 20), randn((B, H, S, D), 21), randn((B, H, S, D), 22)
    allowed = torch.from_numpy(np.random.default_rng(6).random((L, S)) < 0.6)
    allowed[:, 0] = True
    w, launch = _weights(dev, q, k, v, allowed, False, average)
    assert launch == "weights mfma f32 D=64", launch
    bias = torch.zeros(L, S).masked_fill(~allowed, float("-inf"))
    want = oracle_weights(q, k, bias, False, 1.0 / np.sqrt(D))
    assert_close(w, want.mean(axis=1) if average else want, torch.float32, "bool mask")
    add = torch.from_numpy((np.random.default_rng(7).standard_normal((B, H, L, S)) * 2).astype(np.float32))
    w, launch = _weights(dev, q, k, v, add, True, average)
    assert launch == "weights mfma f32 D=64", launch
    want = oracle_weights(q, k, add, True, 1.0 / np.sqrt(D))
    assert_close(w, want.mean(axis=1) if average else want, torch.float32, "float mask, causal")


def test_other_head_sizes_keep_the_generic_weights_kernel(dev):
    B, H, L, S, D = 1, 2, 33, 47, 32
    q, k, v = randn((B, H, L, D), 30), randn((B, H, S, D), 31), randn((B, H, S, D), 32)
    w, launch = _weights(dev, q, k, v, None, True, False)
    assert launch == "weights generic f32 D=32", launch
    assert_close(w, oracle_weights(q, k, None, True, 1.0 / np.sqrt(D)), torch.float32, "generic f32 weights")
