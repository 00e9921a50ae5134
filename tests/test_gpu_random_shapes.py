"""Seeded random shapes against the float64 oracle, one case per seed: fp16/bf16 decode (head
groups of 1 to 32 query heads, 1 to 6000 keys, every split count and both grid orders the
decode launcher picks), Q8_0 decode (the streaming kernel for 16-byte slices, the register
kernel otherwise), and prefill (ragged L and S, GQA, both head sizes), each with no mask, a
key-padding row, a per-head bool mask or a float (L, S) mask, causal or not.  These fill the
gaps between the hand-picked cases of the other files."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C
import oracle

from _util import assert_close, oracle_forward

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    fam = ("decode", "q8", "prefill")[seed % 3]
    D = int(rng.choice([64, 128]))
    if fam == "prefill":
        B = int(rng.integers(1, 4)); Hkv = int(rng.choice([1, 2, 4])); H = Hkv * int(rng.choice([1, 2, 3]))
        L = int(rng.integers(2, 701)); S = int(rng.integers(2, 901))
        dt = torch.float16 if rng.random() < 0.5 else torch.bfloat16
    else:
        B = int(rng.integers(1, 13)); Hkv = int(rng.choice([1, 2, 3, 5, 8]))
        H = Hkv * int(rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16, 20, 32]))
        L, S = 1, int(rng.integers(1, 6001))
        dt = torch.float16 if fam == "q8" or rng.random() < 0.5 else torch.bfloat16
    causal = bool(rng.random() < 0.3)
    kind = int(rng.integers(0, 4))
    mask = None
    if kind == 1:
        mask = torch.zeros(B, 1, 1, S)
        for b in range(B):
            mask[b, ..., int(rng.integers(1, S + 1)):] = float("-inf")
    elif kind == 2:
        mask = torch.from_numpy(rng.random((B, H, L, S)) < 0.6)
        mask[..., 0] = True
    elif kind == 3:
        mask = torch.from_numpy((rng.standard_normal((B, 1, L, S)) * 2).astype(np.float32))
    t = lambda shape, s=1.0: torch.from_numpy((rng.standard_normal(shape) * s).astype(np.float32))
    q = t((B, H, L, D), 0.5).to(dt)
    if fam == "q8":
        k, v = t((B, Hkv, S, D)), t((B, Hkv, S, D))
    else:
        k, v = t((B, Hkv, S, D), 0.5).to(dt), t((B, Hkv, S, D)).to(dt)
    what = f"{fam} {dt} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} mask kind {kind}"
    return fam, dt, q, k, v, mask, causal, what


@pytest.mark.parametrize("seed", range(96))
def test_random_shape_against_the_oracle(dev, seed):
    fam, dt, q, k, v, mask, causal, what = _case(seed)
    m = None if mask is None else mask.to(dev)
    if fam == "q8":
        kb, vb = oracle.q8_0_quantize(k.numpy()), oracle.q8_0_quantize(v.numpy())
        kq = g.QuantizedTensor(torch.from_numpy(kb).to(dev), tuple(k.shape))
        vq = g.QuantizedTensor(torch.from_numpy(vb).to(dev), tuple(v.shape))
        got = g.flash_attention(q.to(dev), kq, vq, m, 0.0, causal)
        k = torch.from_numpy(oracle.q8_0_dequantize(kb).reshape(k.shape))
        v = torch.from_numpy(oracle.q8_0_dequantize(vb).reshape(v.shape))
    else:
        got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), m, 0.0, causal)
    launch = _C.last_launch()
    print(f"[random] seed {seed}: {what} -> {launch}", flush=True)
    assert launch.startswith("prefill" if fam == "prefill" else "decode q8_0" if fam == "q8" else "decode")
    assert_close(got, oracle_forward(q, k, v, mask=mask, is_causal=causal), dt, what)
