"""Float32 backward on v_mfma_f32_32x32x2_f32 (bwd_dq_f32_kernel, then bwd_dkdv_f32_kernel: head
sizes 64 and 128, any mask, 16 query rows or more; dropout in test_gpu_dropout_f32.py) against
the float64 oracle's gradients at the float32 bar (max-abs 1e-4): ragged query and key counts around
the dQ kernel's 128-row query tiles and 32-key K/V tiles and the dK/dV kernel's 128-key tiles and
64-row query steps, one key, GQA and MQA, causal or not, keys no query sees (causal, S > L),
fully padded rows, per-element bool / additive masks, and the launch log naming the kernel.
Grids of fewer than 128 dQ workgroups of the tiled kernels take the small-grid kernels
(bwd_dq_f32s_kernel, bwd_dkdv_f32s_kernel: 4 wavefronts per workgroup splitting the key tiles or
query steps), fewer than 16 query rows included; larger grids with fewer than 16 rows keep the
generic kernels."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C

import oracle
from _util import assert_close, randn, to_oracle

pytestmark = pytest.mark.gpu

CASES = [
    # B, H, Hkv, L, S, D, causal, key padding (B * H * ceil(L / 128) dQ workgroups of the tiled
    # kernels: fewer than 128 take the small-grid kernels, see _want)
    (1, 32, 32, 128, 128, 64, True, False),
    (2, 32, 8, 300, 300, 128, True, True),
    (2, 16, 1, 37, 257, 128, False, False),
    (4, 32, 32, 129, 33, 64, False, True),
    (2, 16, 16, 16, 300, 64, True, True),
    (2, 16, 16, 257, 1, 64, False, False),
    (1, 16, 16, 200, 31, 128, True, True),
    (2, 16, 16, 513, 513, 64, True, True),
    (4, 8, 2, 65, 200, 64, True, False),
    (2, 16, 4, 96, 160, 128, False, True),
]


def _want(B, H, L, S, D):
    """The launch log of a float32 backward without dropout: the small-grid kernels below 128 dQ
    workgroups of the tiled ones (and at most 4096 query rows and keys), else the tiled kernels."""
    small = B * H * ((L + 127) // 128) < 128 and L <= 4096 and S <= 4096
    return f"backward mfma f32 D={D}" + (" split" if small else "")


def _keypad(B, S, seed, empty_row=False):
    rng = np.random.default_rng(seed)
    m = torch.zeros(B, 1, 1, S)
    for b in range(B):
        m[b, ..., int(rng.integers(1, S + 1)):] = float("-inf")
    if empty_row:
        m[B - 1] = float("-inf")  # the last sequence sees no key at all
    return m


def _grads(dev, q, k, v, dout, mask, causal, with_residuals=True):
    md = None if mask is None else mask.to(dev)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = lse = None
    if with_residuals:
        out, lse = g.flash_attention_lse(qd, kd, vd, md, 0.0, causal)
    dq, dk, dv = g.flash_attention_backward(dout.to(dev), qd, kd, vd, md, out, lse, 0.0, causal)
    return dq, dk, dv, _C.last_launch()


def _oracle_grads(dout, q, k, v, mask, causal):
    return oracle.flash_attention_backward(to_oracle(dout), to_oracle(q), to_oracle(k), to_oracle(v),
                                           mask=None if mask is None else to_oracle(mask), is_causal=causal)


@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal,kp", CASES)
def test_float32_backward_against_the_oracle(dev, B, H, Hkv, L, S, D, causal, kp):
    seed = 3 * B + 11 * H + L + 5 * S + D
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    dout = randn((B, H, L, D), seed + 3)
    mask = _keypad(B, S, seed) if kp else None
    dq, dk, dv, launch = _grads(dev, q, k, v, dout, mask, causal)
    what = f"B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal} keypad={kp}"
    assert launch == _want(B, H, L, S, D), (what, launch)
    assert dq.dtype == dk.dtype == dv.dtype == torch.float32
    wq, wk, wv = _oracle_grads(dout, q, k, v, mask, causal)
    assert_close(dq, wq, torch.float32, "dq " + what)
    assert_close(dk, wk, torch.float32, "dk " + what)
    assert_close(dv, wv, torch.float32, "dv " + what)


def test_one_key_seen_by_every_query_of_an_mqa_group(dev):
    # dV of the single key sums dO over all 16 x 257 query rows of the group (P = 1) in one
    # float32 accumulator: values of magnitude ~60, where a sequential float32 sum of 4112 normal
    # terms is itself off by up to 2.5e-4 (64 trials); it is held to 1e-4 relative to
    # max(1, |ref|).  The softmax over one key is constant, so dQ and dK are 0 up to rounding and
    # keep the absolute bar.
    B, H, L, D = 2, 16, 257, 64
    q, k, v, dout = randn((B, H, L, D), 90), randn((B, 1, 1, D), 91), randn((B, 1, 1, D), 92), randn((B, H, L, D), 93)
    dq, dk, dv, launch = _grads(dev, q, k, v, dout, None, False)
    assert launch == _want(B, H, L, 1, D), launch
    wq, wk, wv = _oracle_grads(dout, q, k, v, None, False)
    assert_close(dq, wq, torch.float32, "dq one key")
    assert_close(dk, wk, torch.float32, "dk one key")
    got = dv.double().cpu().numpy()
    assert np.abs(wv).max() > 10  # the long sums this test is about
    worst = (np.abs(got - wv) / (1e-4 * np.maximum(1.0, np.abs(wv)))).max()
    assert worst <= 1.0, f"dv one key: {worst:.3f}x the bound"


def test_float32_backward_without_residuals_and_with_an_empty_row(dev):
    # no output or log-sum-exp given: the forward is recomputed; the last sequence's rows see no
    # key (log-sum-exp +inf), so its gradients are zero
    B, H, L, D = 2, 16, 70, 128
    q, k, v, dout = (randn((B, H, L, D), 60 + i) for i in range(4))
    mask = _keypad(B, L, 9, empty_row=True)
    dq, dk, dv, launch = _grads(dev, q, k, v, dout, mask, False, with_residuals=False)
    # the log names the recomputed forward first
    assert launch.startswith("prefill f32 D=128") and launch.endswith("; " + _want(B, H, L, L, D)), launch
    for got, want, name in zip((dq, dk, dv), _oracle_grads(dout, q, k, v, mask, False), ("dq", "dk", "dv")):
        assert_close(got, want, torch.float32, name + " empty row")
        assert torch.count_nonzero(got[B - 1]).item() == 0, name


def test_small_grids_take_the_split_backward(dev):
    # 15 and 3 query rows: the small-grid kernels (32-row groups); the same rows on a grid of 128
    # or more tiled workgroups: the generic kernels
    S, D = 90, 64
    for B, H, L, want_launch in ((1, 32, 15, "backward mfma f32 D=64 split"), (2, 8, 3, "backward mfma f32 D=64 split"),
                                 (4, 32, 15, "backward generic f32")):
        q, k, v, dout = randn((B, H, L, D), 70), randn((B, H, S, D), 71), randn((B, H, S, D), 72), randn((B, H, L, D), 73)
        dq, dk, dv, launch = _grads(dev, q, k, v, dout, None, L == 3)
        assert launch == want_launch, (B, H, L, launch)
        for got, want, name in zip((dq, dk, dv), _oracle_grads(dout, q, k, v, None, L == 3), ("dq", "dk", "dv")):
            assert_close(got, want, torch.float32, f"{name} B{B} H{H} L={L}")
    # 127 dQ workgroups of the tiled kernels (B * H * ceil(L / 128)): the small-grid kernels; 128: tiled
    for H2, want_launch in ((127, "backward mfma f32 D=64 split"), (128, "backward mfma f32 D=64")):
        q2, k2, v2, g2 = (randn((1, H2, 128, D), 80 + i) for i in range(4))
        dq, dk, dv, launch = _grads(dev, q2, k2, v2, g2, None, True)
        assert launch == want_launch, (H2, launch)
        for got, want, name in zip((dq, dk, dv), _oracle_grads(g2, q2, k2, v2, None, True), ("dq", "dk", "dv")):
            assert_close(got, want, torch.float32, f"{name} H={H2}")


# per-element masks: S % 4 == 0 reads 4 keys per load in dQ (modes 5, 6), other S one key; dK/dV
# reads one element per (query, key)
@pytest.mark.parametrize("kind", ["bool", "add"])
@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal", [(1, 32, 16, 70, 92, 64, False), (4, 32, 8, 130, 131, 128, True),
                                                  (4, 32, 32, 40, 256, 128, False), (2, 16, 4, 100, 33, 64, True)])
def test_float32_backward_with_per_element_masks(dev, kind, B, H, Hkv, L, S, D, causal):
    seed = L + S + D + 1
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    dout = randn((B, H, L, D), seed + 3)
    rng = np.random.default_rng(seed)
    if kind == "bool":
        m = torch.from_numpy(rng.random((L, S)) < 0.7)
        m[:, 0] = True
    else:
        m = torch.from_numpy((rng.standard_normal((B, H, L, S)) * 2).astype(np.float32))
    dq, dk, dv, launch = _grads(dev, q, k, v, dout, m, causal)
    what = f"{kind} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal}"
    assert launch == _want(B, H, L, S, D), (what, launch)
    for got, want, name in zip((dq, dk, dv), _oracle_grads(dout, q, k, v, m, causal), ("dq", "dk", "dv")):
        assert_close(got, want, torch.float32, f"{name} {what}")


# small grids: the split kernels (32 query rows or keys per workgroup, 4 wavefronts splitting the
# key tiles / query steps, partials summed through LDS), every mask kind
@pytest.mark.parametrize("kind", [None, "pad", "bool", "add"])
@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal", [(1, 4, 4, 128, 128, 64, True), (1, 2, 1, 1024, 1024, 64, True),
                                                  (2, 3, 1, 70, 133, 128, False), (1, 4, 2, 200, 61, 128, True),
                                                  (1, 1, 1, 16, 300, 64, False)])
def test_float32_split_backward_for_small_grids(dev, kind, B, H, Hkv, L, S, D, causal):
    seed = 5 * L + S + D + 3
    q, k, v = randn((B, H, L, D), seed), randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    dout = randn((B, H, L, D), seed + 3)
    rng = np.random.default_rng(seed)
    m = None
    if kind == "pad":
        m = _keypad(B, S, seed)
    elif kind == "bool":
        m = torch.from_numpy(rng.random((L, S)) < 0.7)
        m[:, 0] = True
    elif kind == "add":
        m = torch.from_numpy((rng.standard_normal((B, H, L, S)) * 2).astype(np.float32))
    dq, dk, dv, launch = _grads(dev, q, k, v, dout, m, causal)
    what = f"{kind} B{B} H{H}/{Hkv} L{L} S{S} D{D} causal={causal}"
    assert launch == f"backward mfma f32 D={D} split", (what, launch)
    for got, want, name in zip((dq, dk, dv), _oracle_grads(dout, q, k, v, m, causal), ("dq", "dk", "dv")):
        assert_close(got, want, torch.float32, f"{name} {what}")
