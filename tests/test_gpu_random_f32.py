"""Seeded random float32 shapes against the float64 oracle, one case per seed, filling the gaps
between the hand-picked cases of the float32 files: decode (head groups of 1 to 32 query heads,
1 to 6000 keys, every split count the launcher picks, masks) and prefill + backward (ragged L
and S, GQA, head sizes 32 to 128 with and without padding, no mask, a key-padding row, a per-head
bool mask or a float (L, S) mask, causal or not, dropout or not, backward grids on both sides of
the 32-workgroup threshold).  Forward output, log-sum-exp and dQ/dK/dV at the float32 bar; the
kernel each call took is printed with the case."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C
import oracle

from _util import assert_close, oracle_forward, to_oracle

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(5000 + seed)
    fam = "decode" if seed % 4 == 0 else "prefill"
    if fam == "decode":
        D = int(rng.choice([64, 128]))
        B = int(rng.integers(1, 9)); Hkv = int(rng.choice([1, 2, 3, 8]))
        H = Hkv * int(rng.choice([1, 2, 3, 4, 5, 8, 12, 32]))
        L, S = 1, int(rng.integers(1, 6001))
        p = 0.0
    else:
        D = int(rng.choice([32, 48, 64, 80, 96, 100, 128]))
        B = int(rng.integers(1, 3)); Hkv = int(rng.choice([1, 2, 4])); H = Hkv * int(rng.choice([1, 2, 4]))
        H = H * int(rng.choice([1, 4]))
        L = int(rng.integers(16, 301)); S = int(rng.integers(8, 401))
        p = float(rng.choice([0.0, 0.0, 0.1, 0.4]))
    causal = bool(rng.random() < 0.35)
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
        mask = torch.from_numpy((rng.standard_normal((L, S)) * 2).astype(np.float32))
    t = lambda shape, s=1.0: torch.from_numpy((rng.standard_normal(shape) * s).astype(np.float32))
    q, k, v = t((B, H, L, D), 0.5), t((B, Hkv, S, D), 0.5), t((B, Hkv, S, D))
    dout = t((B, H, L, D))
    what = f"{fam} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} mask kind {kind} p={p}"
    return fam, q, k, v, dout, mask, causal, p, what


@pytest.mark.parametrize("seed", range(48))
def test_random_float32_shape_against_the_oracle(dev, seed):
    fam, q, k, v, dout, mask, causal, p, what = _case(seed)
    md = None if mask is None else mask.to(dev)
    if p == 0.0:
        out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal)
    else:
        out, lse, _ = g.flash_attention_dropout(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal, p, seed)
    fwd = _C.last_launch()
    print(f"[random-f32] seed {seed}: {what} -> {fwd}", flush=True)
    want, want_lse = oracle_forward(q, k, v, mask=mask, is_causal=causal, return_lse=True)
    fin = np.isfinite(want_lse)
    assert np.array_equal(np.isinf(lse.cpu().numpy()), ~fin), what
    assert np.abs(lse.cpu().double().numpy()[fin] - want_lse[fin]).max(initial=0.0) < 1e-4, what
    if fam == "decode":
        assert fwd.startswith("decode f32"), (what, fwd)
        assert_close(out, want, torch.float32, what)
        return
    if p == 0.0:
        assert_close(out, want, torch.float32, what)
        dq, dk, dv = g.flash_attention_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), md, out, lse, 0.0,
                                                causal)
        ref = oracle.flash_attention_backward(to_oracle(dout), to_oracle(q), to_oracle(k), to_oracle(v),
                                              mask=None if mask is None else to_oracle(mask), is_causal=causal)
    else:
        dq, dk, dv = g.flash_attention_dropout_backward(dout.to(dev), q.to(dev), k.to(dev), v.to(dev), md, out, lse,
                                                        0.0, causal, p, seed)
        B, H, L, _ = q.shape
        keep = oracle.dropout_keep(B, H, L, k.shape[2], p, seed, 0)
        ref_o, ref = oracle.attention_dropout(to_oracle(q), to_oracle(k), to_oracle(v), keep, p,
                                              mask=None if mask is None else to_oracle(mask), is_causal=causal,
                                              dout=to_oracle(dout), out_dtype=oracle.F64)
        assert_close(out, ref_o, torch.float32, what)
    print(f"[random-f32] seed {seed}: backward -> {_C.last_launch()}", flush=True)
    for name, got, w in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        assert_close(got, w, torch.float32, f"{name} {what}")
