"""Dropout on the float32 MFMA kernels (prefill_f32_kernel, bwd_dq_f32_kernel and
bwd_dkdv_f32_kernel with DROP: head sizes 64 and 128, padded heads, key padding or per-element
masks) against the oracle's composition under the oracle's Philox4x32-10 decisions, at the float32
bar: forward output and the undropped log-sum-exp, dQ, dK, dV; several key tiles, causal or not,
GQA, p from 0.05 to 1, tiled and small-grid kernels, the launch log naming the kernels, and the
generic backward when the decision buffer would exceed GT_ATTN_DROPOUT_BITS_MAX (the float32
dK/dV kernels read the dQ kernel's decisions and do not draw their own)."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C
import oracle

from _util import assert_close, randn, to_oracle

pytestmark = pytest.mark.gpu

CASES = [
    # B, H, Hkv, L, S, D, causal, key lengths (key padding) or a per-element mask, p (below 128
    # dQ workgroups of the tiled kernels, B * H * ceil(L / 128): the small-grid kernels)
    (2, 16, 8, 300, 300, 64, True, (300, 211), 0.1),
    (1, 32, 32, 257, 257, 128, False, (), 0.5),
    (2, 16, 4, 130, 260, 64, False, (260, 100), 0.2),
    (1, 32, 8, 200, 333, 128, True, (), 0.3),
    (2, 16, 16, 96, 130, 128, True, (130, 67), 0.05),
    (1, 32, 32, 64, 64, 64, True, (), 1.0),
    (2, 16, 16, 16, 50, 64, False, (), 0.4),
    (2, 16, 8, 100, 120, 80, True, (), 0.3),  # heads padded to 128
    # per-element masks with dropout (bool: one workgroup per CU for head size 64's dK/dV)
    (2, 16, 8, 130, 200, 64, True, "bool", 0.2),
    (1, 32, 16, 96, 131, 128, False, "add", 0.3),
    # tiny grids (the small-grid kernels, 4 dQ workgroups of the tiled ones)
    (1, 4, 4, 128, 128, 64, True, (), 0.2),
    (1, 2, 1, 40, 300, 128, False, (211,), 0.3),
    (1, 4, 2, 12, 77, 64, True, "bool", 0.5),
]


def _run(dev, q, k, v, dout, mask, causal, p, seed, offset=3):
    md = None if mask is None else mask.to(dev)
    out, lse, out32 = g.flash_attention_dropout(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal, p, seed, offset)
    fwd = _C.last_launch()
    assert out32 is None  # float32: the output is already exact
    grads = g.flash_attention_dropout_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), md, out, lse, 0.0,
                                               causal, p, seed, offset)
    return out, lse, grads, fwd, _C.last_launch()


def _check(q, k, v, dout, mask, causal, p, seed, out, lse, grads, what, offset=3):
    B, H, L, _ = q.shape
    S = k.shape[2]
    keep = oracle.dropout_keep(B, H, L, S, p, seed, offset)
    ref, (rdq, rdk, rdv) = oracle.attention_dropout(to_oracle(q), to_oracle(k), to_oracle(v), keep, p,
                                                    mask=None if mask is None else to_oracle(mask),
                                                    is_causal=causal, dout=to_oracle(dout), out_dtype=oracle.F64)
    assert_close(out, ref, torch.float32, "out " + what)
    _, want_lse = oracle.flash_attention(to_oracle(q), to_oracle(k), to_oracle(v),
                                         mask=None if mask is None else to_oracle(mask), is_causal=causal,
                                         out_dtype=oracle.F64, return_lse=True)
    assert np.abs(lse.cpu().double().numpy() - want_lse).max() < 1e-4, what  # undropped scores
    for name, got, want in zip(("dq", "dk", "dv"), grads, (rdq, rdk, rdv)):
        assert_close(got, want, torch.float32, f"{name} {what}")


@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal,lens,p", CASES)
def test_float32_dropout_matches_the_oracle(dev, B, H, Hkv, L, S, D, causal, lens, p):
    s0 = L + 7 * S + D + H
    q, k, v = randn((B, H, L, D), s0), randn((B, Hkv, S, D), s0 + 1), randn((B, Hkv, S, D), s0 + 2)
    dout = randn((B, H, L, D), s0 + 3)
    mask = None
    rng = np.random.default_rng(s0)
    if lens == "bool":
        mask = torch.from_numpy(rng.random((L, S)) < 0.7)
        mask[:, 0] = True
    elif lens == "add":
        mask = torch.from_numpy((rng.standard_normal((B, H, L, S)) * 2).astype(np.float32))
    elif lens:
        mask = torch.zeros(B, 1, 1, S)
        for b, n in enumerate(lens):
            mask[b, ..., int(n):] = float("-inf")
    seed = 1000 + s0
    out, lse, grads, fwd, bwd = _run(dev, q, k, v, dout, mask, causal, p, seed)
    Dp = 64 if D <= 64 else 128
    what = f"B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} lens={lens} p={p}"
    assert fwd.startswith(f"prefill f32 D={Dp} "), (what, fwd)
    small = B * H * ((L + 127) // 128) < 128  # the small-grid kernels
    assert bwd == f"backward mfma f32 D={Dp}" + (" split" if small else ""), (what, bwd)
    _check(q, k, v, dout, mask, causal, p, seed, out, lse, grads, what)
    if p == 1.0:
        assert not out.any() and not any(t.any() for t in grads)


def test_float32_dropout_without_the_decision_buffer_takes_the_generic_backward(dev, monkeypatch):
    B, H, L, S, D, p, seed = 2, 16, 200, 300, 64, 0.2, 31
    q, k, v, dout = (randn(shape, 50 + i) for i, shape in
                     enumerate([(B, H, L, D), (B, 4, S, D), (B, 4, S, D), (B, H, L, D)]))
    monkeypatch.setenv("GT_ATTN_DROPOUT_BITS_MAX", "0")
    out, lse, grads, fwd, bwd = _run(dev, q, k, v, dout, None, True, p, seed)
    assert fwd.startswith("prefill f32 D=64 ") and bwd == "backward generic f32", (fwd, bwd)
    _check(q, k, v, dout, None, True, p, seed, out, lse, grads, "generic backward")
