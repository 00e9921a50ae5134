"""Float32 attention on v_mfma_f32_32x32x2_f32 (prefill_f32_kernel: head sizes 64 and 128, no
mask, a key-padding row or a per-element mask, 16 query rows or more) against the float64 oracle at the float32 bar
(max-abs 1e-4): ragged query and key counts around the 128-row query tiles and 32-key K/V
tiles, one key, GQA, causal or not, key padding and per-element bool / additive masks (4-key and
one-key loads), the log-sum-exp and the training forward's float32 output, and the launch log
naming the kernel.  One query row takes the decode kernel; 2 to 15 rows the small-grid kernel on
small grids, else the generic kernel."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C

from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu

CASES = [
    # B, H, Hkv, L, S, D, causal, key padding
    (1, 2, 2, 128, 128, 64, True, False),
    (2, 4, 2, 300, 300, 128, True, False),
    (1, 2, 1, 37, 257, 128, False, False),
    (2, 2, 2, 129, 33, 64, False, True),
    (1, 3, 1, 1, 640, 128, False, False),
    (2, 2, 2, 16, 300, 64, True, True),
    (2, 2, 1, 257, 1, 64, False, False),
    (1, 2, 2, 200, 31, 128, True, True),
    (2, 4, 4, 513, 513, 64, True, True),
]


def _keypad(B, S, seed):
    rng = np.random.default_rng(seed)
    m = torch.zeros(B, 1, 1, S)
    for b in range(B):
        m[b, ..., int(rng.integers(1, S + 1)):] = float("-inf")
    return m


@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal,kp", CASES)
def test_float32_prefill_against_the_oracle(dev, B, H, Hkv, L, S, D, causal, kp):
    seed = B + 10 * H + L + 7 * S + D
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    mask = _keypad(B, S, seed) if kp else None
    md = None if mask is None else mask.to(dev)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), md, 0.0, causal)
    launch = _C.last_launch()
    what = f"B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} keypad={kp}"
    # one query row takes the float32 decode kernel; 2 to 15 rows stay on the generic kernel
    # (measured as fast or faster there)
    want_kernel = f"prefill f32 D={D}" if L >= 16 else f"decode f32 D={D}" if L == 1 else "generic f32"
    assert launch.startswith(want_kernel), (what, launch)
    want = oracle_forward(q, k, v, mask=mask, is_causal=causal)
    assert_close(out, want, torch.float32, what)
    # the log-sum-exp: natural log of the row's sum of exp(score) (scores scaled), +inf with nothing visible
    s = torch.einsum("bhld,bhsd->bhls", q.double(), k.double().repeat_interleave(H // Hkv, dim=1)) / np.sqrt(D)
    if mask is not None:
        s = s + mask.double()
    if causal:
        s = s.masked_fill(torch.ones(L, S, dtype=torch.bool).triu(1), float("-inf"))
    want_lse = torch.logsumexp(s, dim=-1)
    got_lse = lse.cpu().double()
    fin = torch.isfinite(want_lse)
    assert torch.equal(torch.isinf(got_lse), ~fin), what
    assert (got_lse[fin] - want_lse[fin]).abs().max().item() < 1e-4, what


def test_float32_training_forward_writes_the_float32_output(dev):
    B, H, L, D = 2, 4, 150, 64
    q, k, v = (randn((B, H, L, D), 40 + i) for i in range(3))
    mask = _keypad(B, L, 3)
    out, lse, out32 = g.flash_attention_train(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, True)
    assert _C.last_launch().startswith("prefill f32 D=64")
    assert out32 is None or torch.equal(out32, out)
    assert_close(out, oracle_forward(q, k, v, mask=mask, is_causal=True), torch.float32, "train forward f32")


def _elem_mask(kind, B, H, L, S, seed):
    rng = np.random.default_rng(seed)
    if kind == "bool":
        m = torch.from_numpy(rng.random((L, S)) < 0.7)
        m[:, 0] = True
        return m
    return torch.from_numpy((rng.standard_normal((B, H, L, S)) * 2).astype(np.float32))


# per-element masks: S % 4 == 0 reads 4 keys per load (modes 5, 6), other S one key (modes 1, 2)
@pytest.mark.parametrize("kind", ["bool", "add"])
@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal", [(1, 2, 2, 70, 92, 64, False), (2, 2, 1, 130, 131, 128, True),
                                                  (1, 4, 2, 200, 256, 128, False), (2, 2, 2, 40, 33, 64, True)])
def test_float32_prefill_with_per_element_masks(dev, kind, B, H, Hkv, L, S, D, causal):
    seed = L + S + D
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    m = _elem_mask(kind, B, H, L, S, seed)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), m.to(dev), 0.0, causal)
    what = f"{kind} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal}"
    assert _C.last_launch().startswith(f"prefill f32 D={D}"), (what, _C.last_launch())
    want, want_lse = oracle_forward(q, k, v, mask=m, is_causal=causal, return_lse=True)
    assert_close(out, want, torch.float32, what)
    fin = np.isfinite(want_lse)
    assert np.array_equal(np.isinf(lse.cpu().numpy()), ~fin), what
    assert np.abs(lse.cpu().double().numpy()[fin] - want_lse[fin]).max() < 1e-4, what


# small grids (at most 64 workgroups of the tiled kernel, B * H * query-tile pairs, and at most
# 4096 keys; no mask, no dropout): the split kernel, whose 4 wavefronts split a 32-row group's key
# tiles and merge; larger grids or longer key ranges: the tiled kernel
@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal,split", [
    (1, 4, 4, 128, 128, 64, True, True), (1, 16, 16, 1024, 1024, 64, True, True),
    (1, 17, 17, 1024, 1024, 64, True, False), (2, 3, 1, 33, 300, 128, False, True),
    (1, 2, 2, 16, 1, 128, False, True), (2, 2, 2, 100, 77, 128, True, True),
    (1, 1, 1, 500, 700, 64, False, True), (1, 2, 1, 40, 4097, 64, False, False)])
def test_float32_split_kernel_for_small_grids(dev, B, H, Hkv, L, S, D, causal, split):
    seed = 7 * L + S + D
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), None, 0.0, causal)
    launch = _C.last_launch()
    what = f"B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal}"
    assert launch.startswith(f"prefill f32 D={D} ") and launch.endswith(" split") == split, (what, launch)
    want, want_lse = oracle_forward(q, k, v, is_causal=causal, return_lse=True)
    assert_close(out, want, torch.float32, what)
    assert np.abs(lse.cpu().double().numpy() - want_lse).max() < 1e-4, what


# the split kernel with every mask mode (key padding 4; bool 5 / 1 and float 6 / 2 with S a
# multiple of 4 or not) and with dropout (against the oracle's composition under its decisions)
@pytest.mark.parametrize("kind,S", [("pad", 77), ("bool", 128), ("bool", 77), ("add", 128), ("add", 77)])
@pytest.mark.parametrize("causal", [False, True])
def test_float32_split_kernel_with_masks(dev, kind, S, causal):
    B, H, Hkv, L, D = 2, 2, 1, 100, 128
    seed = S + (3 if causal else 0) + len(kind)
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    if kind == "pad":
        m = _keypad(B, S, seed)
    else:
        m = _elem_mask(kind, B, H, L, S, seed)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), m.to(dev), 0.0, causal)
    launch = _C.last_launch()
    what = f"{kind} S{S} causal={causal}"
    assert launch.endswith(" split"), (what, launch)
    want, want_lse = oracle_forward(q, k, v, mask=m, is_causal=causal, return_lse=True)
    assert_close(out, want, torch.float32, what)
    fin = np.isfinite(want_lse)
    assert np.array_equal(np.isinf(lse.cpu().numpy()), ~fin), what
    assert np.abs(lse.cpu().double().numpy()[fin] - want_lse[fin]).max() < 1e-4, what


@pytest.mark.parametrize("masked", [False, True])
def test_float32_split_kernel_with_dropout(dev, masked):
    import oracle
    from _util import to_oracle
    B, H, L, S, D, p, seed = 1, 4, 128, 128, 64, 0.3, 11
    q, k, v = randn((B, H, L, D), 20), randn((B, H, S, D), 21), randn((B, H, S, D), 22)
    m = _keypad(B, S, 5) if masked else None
    out, lse, _ = g.flash_attention_dropout(q.to(dev), k.to(dev), v.to(dev), None if m is None else m.to(dev), 0.0,
                                            True, p, seed)
    assert _C.last_launch().endswith(" split"), _C.last_launch()
    keep = oracle.dropout_keep(B, H, L, S, p, seed, 0)
    ref = oracle.attention_dropout(to_oracle(q), to_oracle(k), to_oracle(v), keep, p,
                                   mask=None if m is None else to_oracle(m), is_causal=True, out_dtype=oracle.F64)
    assert_close(out, ref, torch.float32, f"dropout masked={masked}")


# 2 to 15 query rows on a small grid (e.g. draft tokens against a cache): the split kernel; on a
# large grid: the generic kernel
@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal,kp,split", [
    (1, 8, 2, 4, 1000, 128, False, False, True), (2, 4, 4, 8, 300, 64, True, True, True),
    (1, 4, 1, 2, 77, 64, False, True, True), (1, 2, 2, 15, 130, 128, True, False, True),
    (17, 8, 8, 3, 64, 64, False, False, False)])
def test_float32_few_query_rows(dev, B, H, Hkv, L, S, D, causal, kp, split):
    seed = 11 * L + S + D
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    mask = _keypad(B, S, seed) if kp else None
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), None if mask is None else mask.to(dev), 0.0,
                                     causal)
    launch = _C.last_launch()
    what = f"B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} keypad={kp}"
    assert launch == (f"prefill f32 D={D} B={B} H={H} L={L} S={S} split" if split else "generic f32"), (what, launch)
    want, want_lse = oracle_forward(q, k, v, mask=mask, is_causal=causal, return_lse=True)
    assert_close(out, want, torch.float32, what)
    fin = np.isfinite(want_lse)
    assert np.abs(lse.cpu().double().numpy()[fin] - want_lse[fin]).max() < 1e-4, what
