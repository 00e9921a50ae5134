"""Explicit attention weights (gt_attention_weights, MultiheadAttention need_weights=True) on
the GPU: softmax(q.k^T*scale + mask) with the causal mask, recomputed from the forward's
log-sum-exp, against the float64 oracle: P = exp(scores - lse) with the oracle's own lse, and
the invariant sum_s P[l, s] v[s] = the oracle's output row."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _ops

from _util import assert_close, oracle_forward, randn, to_oracle
import oracle

pytestmark = pytest.mark.gpu


def oracle_weights(q, k, mask, causal, scale):
    """float64 softmax weights from the oracle's lse (GQA: kv head h // (H // Hkv))."""
    _, lse = oracle_forward(q, k, k, mask=mask, scale=scale, is_causal=causal, return_lse=True)
    qd, kd = oracle.to_f64(to_oracle(q)), oracle.to_f64(to_oracle(k))
    B, H, L, D = qd.shape
    Hkv, S = kd.shape[1], kd.shape[2]
    kd = np.repeat(kd, H // Hkv, axis=1)
    sc = np.einsum("bhld,bhsd->bhls", qd, kd) * scale
    if mask is not None:
        sc = sc + np.broadcast_to(mask.double().numpy(), sc.shape)
    if causal:
        sc = np.where(np.triu(np.ones((L, S), bool), 1), -np.inf, sc)
    with np.errstate(invalid="ignore", over="ignore"):
        p = np.exp(sc - np.asarray(lse, np.float64)[..., None])
    return np.nan_to_num(p, nan=0.0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal,L,S", [(False, 70, 200), (True, 150, 150)])
@pytest.mark.parametrize("average", [False, True])
def test_weights_match_the_oracle(dev, dtype, D, causal, L, S, average):
    B, H, Hkv = 2, 4, 2
    q, k, v = randn((B, H, L, D), 1, dtype), randn((B, Hkv, S, D), 2, dtype), randn((B, Hkv, S, D), 3, dtype)
    mask = torch.zeros(B, 1, 1, S)
    mask[1, ..., S - 9:] = float("-inf")
    scale = 1.0 / np.sqrt(D)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, causal)
    w = _ops.attention_weights(q.to(dev), k.to(dev), mask.to(dev), lse, 0.0, causal, average)
    want = oracle_weights(q, k, mask, causal, scale)
    assert w.dtype == dtype and w.shape == ((B, L, S) if average else (B, H, L, S))
    assert_close(w, want.mean(axis=1) if average else want, dtype, "weights")
    if not average:
        # the weights reproduce the attention output, up to the rounding of each weight to the
        # output format (one ulp of a weight times |v| per term)
        vd = np.repeat(oracle.to_f64(to_oracle(v)), H // Hkv, axis=1)
        wd = w.double().cpu().numpy()
        pv = np.einsum("bhls,bhsd->bhld", wd, vd)
        o = np.asarray(oracle_forward(q, k, v, mask=mask, is_causal=causal), np.float64)
        ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
        bound = 2e-3 * np.maximum(1.0, np.abs(o)) + ulp * np.einsum("bhls,bhsd->bhld", np.abs(wd), np.abs(vd))
        assert (np.abs(pv - o) <= bound).all(), float(np.max(np.abs(pv - o) / bound))


def test_weights_float32_and_bool_mask(dev):
    B, H, L, S, D = 1, 2, 33, 47, 16
    q, k = randn((B, H, L, D), 4), randn((B, H, S, D), 5)
    allowed = torch.from_numpy(np.random.default_rng(6).random((L, S)) < 0.6)
    allowed[:, 0] = True
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), k.to(dev), allowed.to(dev), 0.5, False)
    w = _ops.attention_weights(q.to(dev), k.to(dev), allowed.to(dev), lse, 0.5, False, False)
    bias = torch.zeros(L, S).masked_fill(~allowed, float("-inf"))
    assert_close(w, oracle_weights(q, k, bias, False, 0.5), torch.float32, "fp32 weights")
