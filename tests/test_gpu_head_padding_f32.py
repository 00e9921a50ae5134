"""Float32 attention with head sizes other than 64 and 128 (up to 128) on the float32 MFMA
kernels with the heads zero-padded: forward (output, log-sum-exp) and backward against the
float64 oracle at the float32 bar, GQA, causal or not, key padding, D != Dv, the 8-element and
one-element pad copies, the launch log naming the padded kernels, a check that padding is what
ran (the result equals the unpadded kernels' on explicitly zero-padded inputs, bit for bit), and
the calls the float32 kernels do not take (fewer than 16 query rows), which stay unpadded on the
generic kernels; per-element masks and small backward grids are padded."""

import numpy as np
import pytest
import torch
import torch.nn.functional as tF

import gguf_train_amd as g
from gguf_train_amd import _C
import oracle

from _util import assert_close, oracle_forward, randn, to_oracle

pytestmark = pytest.mark.gpu

CASES = [
    # B, H, Hkv, L, S, D, Dv, causal, key padding (B * H * ceil(L / 128) >= 32: the MFMA backward)
    (2, 16, 8, 150, 150, 96, 96, True, False),
    (1, 32, 32, 129, 200, 80, 80, False, True),
    (2, 16, 4, 64, 64, 32, 32, True, True),
    (2, 16, 16, 100, 77, 48, 48, False, False),
    (1, 32, 8, 90, 90, 112, 112, True, False),
    (2, 16, 16, 70, 70, 96, 64, False, True),
    (2, 16, 8, 130, 130, 100, 100, True, False),
    (2, 16, 8, 40, 300, 36, 36, False, True),
]


def _keypad(B, S, seed):
    m = torch.zeros(B, 1, 1, S)
    m[0, ..., S - S // 3:] = float("-inf")
    return m


@pytest.mark.parametrize("B,H,Hkv,L,S,D,Dv,causal,kp", CASES)
def test_float32_padded_heads_match_the_oracle(dev, B, H, Hkv, L, S, D, Dv, causal, kp):
    seed = L + S + D + Dv
    q, k = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1)
    v, dout = randn((B, Hkv, S, Dv), seed + 2), randn((B, H, L, Dv), seed + 3)
    mask = _keypad(B, S, seed) if kp else None
    md = None if mask is None else mask.to(dev)
    Dp = 64 if max(D, Dv) <= 64 else 128
    what = f"B{B} H{H}/{Hkv} L{L} S{S} D{D} Dv{Dv} causal={causal} keypad={kp}"
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal)
    assert _C.last_launch().startswith(f"prefill f32 D={Dp} "), (what, _C.last_launch())
    assert out.shape == (B, H, L, Dv)
    want, want_lse = oracle_forward(q, k, v, mask=mask, is_causal=causal, return_lse=True)
    assert_close(out, want, torch.float32, "out " + what)
    fin = np.isfinite(want_lse)
    assert np.abs(lse.cpu().double().numpy()[fin] - want_lse[fin]).max() < 1e-4, what
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), md, out, lse, 0.0, causal)
    small = B * H * ((L + 127) // 128) < 128  # the small-grid kernels
    assert _C.last_launch() == f"backward mfma f32 D={Dp}" + (" split" if small else ""), (what, _C.last_launch())
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    wq, wk, wv = oracle.flash_attention_backward(to_oracle(dout), to_oracle(q), to_oracle(k), to_oracle(v),
                                                 mask=None if mask is None else to_oracle(mask), is_causal=causal)
    for name, got, ref in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv)):
        assert_close(got, ref, torch.float32, f"{name} {what}")


# D % 8 == 0: the 8-element pad / unpad copies; 100 and 36: the one-element copies
@pytest.mark.parametrize("D", [96, 40, 100, 36])
def test_float32_padding_is_the_unpadded_kernel_on_zero_padded_heads(dev, D):
    B, H, L, S = 2, 16, 130, 130
    Dp = 64 if D <= 64 else 128
    q, k, v, dout = (randn((B, H, n, D), i).to(dev) for i, n in enumerate((L, S, S, L)))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))  # the default scale, 1 / sqrt(D) in float32
    out, lse = g.flash_attention_lse(q, k, v, None, 0.0, True)
    pad = lambda t: tF.pad(t, (0, Dp - D))
    ref, ref_lse = g.flash_attention_lse(pad(q), pad(k), pad(v), None, scale, True)
    assert torch.equal(out, ref[..., :D]) and torch.equal(lse, ref_lse)
    grads = g.flash_attention_backward(dout, q, k, v, None, out, lse, 0.0, True)
    ref_grads = g.flash_attention_backward(pad(dout), pad(q), pad(k), pad(v), None, ref, ref_lse, scale, True)
    for a, b in zip(grads, ref_grads):
        assert torch.equal(a, b[..., :D])
        assert not b[..., D:].any()


def test_float32_padding_of_short_rows_masks_and_small_grids(dev):
    B, H, S, D = 1, 4, 90, 96
    k, v = randn((B, H, S, D), 41).to(dev), randn((B, H, S, D), 42).to(dev)
    # 15 query rows: the generic forward
    q = randn((B, H, 15, D), 40)
    out = g.flash_attention(q.to(dev), k, v, None, 0.0, False)
    assert _C.last_launch() == "generic f32", _C.last_launch()
    assert_close(out, oracle_forward(q, k.cpu(), v.cpu()), torch.float32, "L=15")
    # a per-element bool mask: the padded MFMA forward
    L = 40
    q, dout = randn((B, H, L, D), 43), randn((B, H, L, D), 44)
    m = torch.from_numpy(np.random.default_rng(8).random((L, S)) < 0.7)
    m[:, 0] = True
    out = g.flash_attention(q.to(dev), k, v, m.to(dev), 0.0, False)
    assert _C.last_launch().startswith("prefill f32 D=128 "), _C.last_launch()
    assert_close(out, oracle_forward(q, k.cpu(), v.cpu(), mask=m), torch.float32, "bool mask")
    # 4 dQ workgroups: the padded small-grid kernels, forward and backward
    out, lse = g.flash_attention_lse(q.to(dev), k, v, None, 0.0, True)
    assert _C.last_launch().startswith("prefill f32 D=128 "), _C.last_launch()
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k, v, None, out, lse, 0.0, True)
    assert _C.last_launch() == "backward mfma f32 D=128 split", _C.last_launch()
    wq, wk, wv = oracle.flash_attention_backward(to_oracle(dout), to_oracle(q), to_oracle(k.cpu()), to_oracle(v.cpu()),
                                                 is_causal=True)
    for name, got, ref in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv)):
        assert_close(got, ref, torch.float32, name + " small grid")
