"""The MFMA prefill kernel (fp16/bf16, head size 64/128): ragged lengths (not multiples of
the 128-row query tile or the 64-row key tile), L != S with the top-left causal rule, every
mask form, rows with nothing to attend to, GQA, and one full-length (L = S = 2048, D = 128)
head pair against the oracle."""

import math

import numpy as np
import pytest
import torch

import gguf_train_amd as g

from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("L,S", [(2, 2), (129, 129), (200, 77), (77, 300), (256, 256), (65, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_ragged(dev, dtype, D, L, S, causal):
    B, H, Hkv = 2, 4, 2
    seed = L * 31 + S + D
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None, 0.0, causal)
    assert_close(got, oracle_forward(q, k, v, is_causal=causal), dtype, f"L={L} S={S} D={D} causal={causal}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mshape", [(2, 4, 150, 150), (2, 1, 1, 150), (150, 150), (1, 4, 150, 1), (2, 1, 150, 150),
                                    (2, 4, 160, 160), (160, 160), (2, 1, 1, 160), (1, 4, 160, 160)])
def test_prefill_masks(dev, dtype, mshape):
    # 150 keys: per-element mask loads; 160 (whole 4-key groups, contiguous): 4-key loads
    B, H, L, D = 2, 4, mshape[-2] if mshape[-2] > 1 else mshape[-1], 64
    q, k, v = randn((B, H, L, D), 1, dtype), randn((B, H, L, D), 2, dtype), randn((B, H, L, D), 3, dtype)
    rng = np.random.default_rng(4)
    allowed = torch.from_numpy(rng.random(mshape) < 0.7)
    allowed[..., 0] = True
    m4 = allowed.reshape((1,) * (4 - allowed.ndim) + tuple(allowed.shape))
    want = oracle_forward(q, k, v, mask=m4)
    assert_close(g.flash_attention(q.to(dev), k.to(dev), v.to(dev), allowed.to(dev)), want, dtype, f"bool {mshape}")
    add = torch.zeros(mshape).masked_fill(~allowed, float("-inf"))
    assert_close(g.flash_attention(q.to(dev), k.to(dev), v.to(dev), add.to(dev)), want, dtype, f"-inf {mshape}")
    bias = randn(mshape, 5)
    assert_close(g.flash_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), 0.0, True),
                 oracle_forward(q, k, v, mask=bias, is_causal=True), dtype, f"bias {mshape}")


@pytest.mark.parametrize("dtype,D", [(torch.float16, 128), (torch.bfloat16, 64)])
@pytest.mark.parametrize("kind", ["bool", "float"])
def test_mask_loads_of_every_layout_give_the_same_bits(dev, dtype, D, kind):
    # a contiguous (L, S) mask takes 4-key loads; the same values as a view with a key stride of
    # 2, or at a base that is not 16-byte aligned, take per-element loads: identical outputs
    B, H, L, S = 2, 4, 192, 256
    q, k, v = randn((B, H, L, D), 7, dtype), randn((B, H, S, D), 8, dtype), randn((B, H, S, D), 9, dtype)
    rng = np.random.default_rng(11)
    vals = rng.random((L, S)) < 0.8 if kind == "bool" else rng.standard_normal((L, S)).astype(np.float32)
    m = torch.from_numpy(vals).to(dev)
    wide = torch.zeros((L, 2 * S), dtype=m.dtype, device=dev)
    wide[:, ::2] = m
    shifted = torch.zeros(L * S + 1, dtype=m.dtype, device=dev)
    shifted[1:] = m.reshape(-1)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    for causal in (False, True):
        ref = g.flash_attention(qd, kd, vd, m, 0.0, causal)
        for other in (wide[:, ::2], shifted[1:].view(L, S)):
            assert torch.equal(g.flash_attention(qd, kd, vd, other, 0.0, causal), ref)
        want = oracle_forward(q, k, v, mask=m.cpu().reshape(1, 1, L, S), is_causal=causal)
        assert_close(ref, want, dtype, f"{kind} causal={causal}")


def test_prefill_key_padding_training_shape(dev):
    # causal + additive key padding (B,1,1,S), -inf beyond each sequence's valid length
    B, H, L, D = 4, 4, 1024, 64
    dtype = torch.bfloat16
    q, k, v = randn((B, H, L, D), 6, dtype), randn((B, H, L, D), 7, dtype), randn((B, H, L, D), 8, dtype)
    lens = [1024, 512, 777, 600]
    mask = torch.zeros(B, 1, 1, L)
    for b, n in enumerate(lens):
        mask[b, ..., n:] = float("-inf")
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, True)
    assert_close(got, oracle_forward(q, k, v, mask=mask, is_causal=True), dtype, "key padding")


def test_prefill_blocked_rows_and_explicit_scale(dev):
    B, H, L, D = 1, 2, 140, 128
    q, k, v = randn((B, H, L, D), 9, torch.float16), randn((B, H, L, D), 10, torch.float16), randn((B, H, L, D), 11, torch.float16)
    allowed = torch.ones(L, L, dtype=torch.bool)
    allowed[5] = False
    allowed[139] = False
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), allowed.to(dev), 0.3, False)
    assert torch.equal(got[:, :, 5].cpu(), torch.zeros(B, H, D, dtype=torch.float16))
    assert torch.equal(got[:, :, 139].cpu(), torch.zeros(B, H, D, dtype=torch.float16))
    assert_close(got, oracle_forward(q, k, v, mask=allowed, scale=0.3), torch.float16, "blocked rows")


def test_prefill_full_length_heads(dev):
    # two heads of the L = S = 2048, D = 128 causal fp16 workload, inputs 0.5 * N(0,1)
    q = randn((1, 2, 2048, 128), 12, torch.float16, 0.5)
    k = randn((1, 2, 2048, 128), 13, torch.float16, 0.5)
    v = randn((1, 2, 2048, 128), 14, torch.float16, 0.5)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None, 0.0, True)
    assert_close(got, oracle_forward(q, k, v, is_causal=True), torch.float16, "2048 causal")


def test_prefill_lse_matches_oracle(dev):
    q, k, v = randn((2, 2, 300, 64), 15, torch.bfloat16), randn((2, 2, 300, 64), 16, torch.bfloat16), randn((2, 2, 300, 64), 17, torch.bfloat16)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), None, 0.0, True)
    want_o, want_l = oracle_forward(q, k, v, is_causal=True, return_lse=True)
    assert_close(out, want_o, torch.bfloat16, "out")
    assert np.abs(lse.cpu().numpy() - want_l).max() < 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("mshape", [(2, 1, 1, 96), (96, 96)])
def test_huge_finite_mask_values(dev, dtype, mshape):
    # float32 masks of -1e9 (a finite value far below the scores): rows where it covers only
    # some keys match the oracle; rows where it covers every key put the softmax reference
    # point near -1.4e9 (an ulp of 128 in float32) and must stay finite: every probability
    # underflows there, which gives 0 (the rule for a row with nothing visible)
    B, H, L, S, D = 2, 4, 96, 96, 64
    q, k, v = randn((B, H, L, D), 21, dtype), randn((B, H, S, D), 22, dtype), randn((B, H, S, D), 23, dtype)
    blocked = torch.zeros(mshape, dtype=torch.bool)
    blocked[..., 40:] = True
    if len(mshape) == 2:
        blocked[10] = True  # query row 10: every key blocked
    else:
        blocked[1] = True   # sequence 1: every key blocked
    mask = torch.zeros(mshape).masked_fill(blocked, -1e9)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev)).cpu()
    assert torch.isfinite(got).all()
    full = blocked.all(-1).reshape((1,) * (4 - blocked.ndim) + tuple(blocked.shape[:-1])).expand(B, H, L)
    assert not got[full].any()
    m4 = mask.reshape((1,) * (4 - mask.ndim) + tuple(mask.shape))
    want = oracle_forward(q, k, v, mask=m4)
    keep = ~full
    assert_close(got[keep], want[keep.numpy()], dtype, f"-1e9 mask {mshape}")
