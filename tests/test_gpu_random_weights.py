"""Seeded random explicit attention weights (gt_attention_weights: MultiheadAttention with
need_weights=True) against the float64 oracle's softmax, one case per seed: float16, bfloat16
and float32, head sizes 64 and 128 (the MFMA kernels) and 32 / 80 (the generic kernel), per head
or averaged over the heads (key tiles split over the grid), GQA, causal or not, no mask, a
key-padding row, a bool or float (L, S) mask, key counts that are and are not multiples of 8 and
4 (16-byte or narrower stores).  The kernel each case took is printed with it."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C, _ops

from _util import assert_close, randn
from test_gpu_attention_weights import oracle_weights

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(9000 + seed)
    dt = (torch.float16, torch.bfloat16, torch.float32)[seed % 3]
    D = int(rng.choice([64, 128, 64, 128, 32, 80]))
    B = int(rng.integers(1, 3)); Hkv = int(rng.choice([1, 2, 4])); H = Hkv * int(rng.choice([1, 2, 4]))
    L = int(rng.integers(1, 260)); S = int(rng.integers(1, 300))
    causal = bool(rng.random() < 0.4)
    average = bool(rng.random() < 0.5)
    kind = int(rng.integers(0, 4))
    mask = None
    if kind == 1:
        mask = torch.zeros(B, 1, 1, S)
        for b in range(B):
            mask[b, ..., int(rng.integers(1, S + 1)):] = float("-inf")
    elif kind == 2:
        mask = torch.from_numpy(rng.random((L, S)) < 0.7)
        mask[:, 0] = True
    elif kind == 3:
        mask = torch.from_numpy((rng.standard_normal((L, S)) * 2).astype(np.float32))
    q, k = randn((B, H, L, D), 9000 + seed, dt, 0.5), randn((B, Hkv, S, D), 9100 + seed, dt, 0.5)
    what = f"{dt} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} average={average} mask kind {kind}"
    return dt, q, k, mask, causal, average, what


@pytest.mark.parametrize("seed", range(36))
def test_random_weights_against_the_oracle(dev, seed):
    dt, q, k, mask, causal, average, what = _case(seed)
    md = None if mask is None else mask.to(dev)
    _, lse = g.flash_attention_lse(q.to(dev), k.to(dev), k.to(dev), md, 0.0, causal)
    w = _ops.attention_weights(q.to(dev), k.to(dev), md, lse, 0.0, causal, average)
    print(f"[random-weights] seed {seed}: {what} -> {_C.last_launch()}", flush=True)
    # the oracle's weights take an additive mask: a bool mask as its -inf bias
    bias = mask
    if mask is not None and mask.dtype == torch.bool:
        bias = torch.zeros(mask.shape).masked_fill(~mask, float("-inf"))
    want = oracle_weights(q, k, bias, causal, 1.0 / np.sqrt(q.shape[3]))
    assert w.dtype == dt
    assert_close(w, want.mean(axis=1) if average else want, dt, what)
