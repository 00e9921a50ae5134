"""Seeded random prefill shapes at the benchmark's scale (L and S from 700 to 2300, up to 32
query heads over 8 kv heads, batches up to 4), so that the grid takes several rounds of the
chip and the per-XCD head partition is exercised with and without causal skipping.  The float64
oracle is too slow for every (batch, head) unit at this size, so each case checks the first and
last unit and two seeded ones; the unit order inside the grid is what a wrong partition would
break, and those four land on different XCDs."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C

from _util import assert_close, oracle_forward

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(9000 + seed)
    dt = torch.float16 if seed % 2 == 0 else torch.bfloat16
    D = int(rng.choice([64, 128]))
    B = int(rng.integers(1, 5)); Hkv = int(rng.choice([1, 2, 4, 8])); H = Hkv * int(rng.choice([1, 2, 4]))
    L = int(rng.integers(700, 2300)); S = L if rng.random() < 0.6 else int(rng.integers(600, 2600))
    causal = bool(rng.random() < 0.6)
    mask = None
    if rng.random() < 0.3:
        mask = torch.zeros(B, 1, 1, S)
        for b in range(B):
            mask[b, ..., int(rng.integers(1, S + 1)):] = float("-inf")
    t = lambda shape, s=1.0: torch.from_numpy((rng.standard_normal(shape) * s).astype(np.float32)).to(dt)
    q, k, v = t((B, H, L, D), 0.5), t((B, Hkv, S, D), 0.5), t((B, Hkv, S, D))
    units = sorted({0, B * H - 1, int(rng.integers(0, B * H)), int(rng.integers(0, B * H))})
    what = f"{dt} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} mask={mask is not None}"
    return dt, q, k, v, mask, causal, units, what


@pytest.mark.parametrize("seed", range(8))
def test_random_large_prefill_against_the_oracle(dev, seed):
    dt, q, k, v, mask, causal, units, what = _case(seed)
    out = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None if mask is None else mask.to(dev), 0.0, causal)
    launch = _C.last_launch()
    print(f"[random-large] seed {seed}: {what} units {units} -> {launch}", flush=True)
    assert launch.startswith("prefill")
    H, G = q.shape[1], q.shape[1] // k.shape[1]
    out = out.cpu()
    for u in units:
        b, h = divmod(u, H)
        want = oracle_forward(q[b:b + 1, h:h + 1], k[b:b + 1, h // G:h // G + 1], v[b:b + 1, h // G:h // G + 1],
                              mask=None if mask is None else mask[b:b + 1], is_causal=causal)
        assert_close(out[b:b + 1, h:h + 1], want, dt, f"{what} unit {u}")
