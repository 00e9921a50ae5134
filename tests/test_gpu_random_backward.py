"""Seeded random shapes for the training path against the float64 oracle, one case per seed:
the training forward + backward (flash_attention_train / flash_attention_backward) and the
dropout pair, fp16 / bf16 / fp32, head sizes 48 (padded), 64 and 128, GQA, ragged L and S, no
mask / key padding / per-element bool / float masks, causal or not.  Random shapes of this kind
found the fp16 gradients leaving the bar where a key collects the probabilities of many rows
(causal key padding) or a row sees only a few keys; these keep that covered."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C
import oracle

from _util import assert_close, to_oracle

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(5000 + seed)
    drop = seed % 2 == 1
    dt = (torch.float16, torch.bfloat16, torch.float32)[(seed // 2) % 3]
    D = int(rng.choice([48, 64, 128]))
    B = int(rng.integers(1, 3)); Hkv = int(rng.choice([1, 2])); H = Hkv * int(rng.choice([1, 2, 3]))
    L = int(rng.integers(2, 300)); S = L if rng.random() < 0.5 else int(rng.integers(2, 350))
    causal = bool(rng.random() < 0.5)
    kind = int(rng.integers(0, 4))
    mask = None
    if kind == 1:
        mask = torch.zeros(B, 1, 1, S)
        for b in range(B):
            mask[b, ..., int(rng.integers(1, S + 1)):] = float("-inf")
    elif kind == 2:
        mask = torch.from_numpy(rng.random((B, 1, L, S)) < 0.6)
        mask[..., 0] = True
    elif kind == 3:
        mask = torch.from_numpy((rng.standard_normal((B, 1, L, S)) * 2).astype(np.float32))
    t = lambda shape, s=1.0: torch.from_numpy((rng.standard_normal(shape) * s).astype(np.float32)).to(dt)
    q, k, v, do = t((B, H, L, D), 0.5), t((B, Hkv, S, D), 0.5), t((B, Hkv, S, D)), t((B, H, L, D))
    p = float(rng.choice([0.1, 0.4])) if drop else 0.0
    seed_, off = int(rng.integers(1, 1 << 40)), int(rng.integers(0, 9))
    what = (f"{'dropout ' if drop else ''}{dt} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} mask kind {kind}"
            + (f" p={p}" if drop else ""))
    return drop, dt, q, k, v, do, mask, causal, p, seed_, off, what


@pytest.mark.parametrize("seed", range(48))
def test_random_training_shape_against_the_oracle(dev, seed):
    drop, dt, q, k, v, do, mask, causal, p, s, off, what = _case(seed)
    qd, kd, vd, dod = (x.to(dev) for x in (q, k, v, do))
    md = None if mask is None else mask.to(dev)
    if drop:
        out, lse, out32 = g.flash_attention_dropout(qd, kd, vd, md, 0.0, causal, p, s, off)
        dq, dk, dv = g.flash_attention_dropout_backward(dod, qd, kd, vd, md, out if out32 is None else out32, lse,
                                                        0.0, causal, p, s, off)
        keep = oracle.dropout_keep(*q.shape[:3], k.shape[2], p, s, off)
        ref, want = oracle.attention_dropout(to_oracle(q), to_oracle(k), to_oracle(v), keep, p,
                                             mask=None if mask is None else to_oracle(mask), is_causal=causal,
                                             dout=to_oracle(do), out_dtype=oracle.F64)
    else:
        out, lse, out32 = g.flash_attention_train(qd, kd, vd, md, 0.0, causal)
        dq, dk, dv = g.flash_attention_backward(dod, qd, kd, vd, md, out if out32 is None else out32, lse, 0.0, causal)
        ref = oracle.flash_attention(to_oracle(q), to_oracle(k), to_oracle(v),
                                     mask=None if mask is None else to_oracle(mask), is_causal=causal,
                                     out_dtype=oracle.F64)
        want = oracle.flash_attention_backward(to_oracle(do), to_oracle(q), to_oracle(k), to_oracle(v),
                                               mask=None if mask is None else to_oracle(mask), is_causal=causal)
    print(f"[random-train] seed {seed}: {what} -> {_C.last_launch()}", flush=True)
    gd = torch.float32 if dt in (torch.float16, torch.bfloat16) else None
    assert_close(out, ref, dt, "out " + what)
    if out32 is not None:
        assert_close(out32, ref, dt, "out32 " + what, out_dtype=torch.float32)
    for name, got, w in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert_close(got, w, dt, f"{name} {what}", out_dtype=gd)
