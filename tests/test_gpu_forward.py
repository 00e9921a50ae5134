"""Forward parity of gt_flash_attention on the GPU against the CPU oracle, same inputs."""

import math

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd.nn import functional as F

from _util import TOL, assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


def test_fp32_causal_parity_configuration(dev):
    # B=1 H=4 L=S=128 D=64, causal, N(0,1), default scale: max-abs <= 1e-4 against fp64
    q, k, v = (randn((1, 4, 128, 64), s) for s in (1, 2, 3))
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), is_causal=True)
    assert out.dtype == torch.float32 and out.shape == (1, 4, 128, 64)
    want = oracle_forward(q, k, v, scale=1 / math.sqrt(64), is_causal=True)
    assert_close(out, want, torch.float32, "fp32 causal")


@pytest.mark.parametrize("shape", [(2, 3, 4, 5), (2, 1, 4, 5), (1, 3, 4, 5), (3, 4, 5), (4, 5), (5,), (1, 5), (4, 1)])
def test_masks_broadcast_from_the_right(dev, shape):
    # tests/test_pooling_and_attention.py:357-373 on the GPU
    q, k, v = randn((2, 3, 4, 6), 6), randn((2, 3, 5, 6), 7), randn((2, 3, 5, 6), 8)
    rng = np.random.default_rng(9)
    allowed = torch.from_numpy(rng.random(shape) < 0.6)
    allowed[..., 0] = True
    m4 = allowed.reshape((1,) * (4 - allowed.ndim) + tuple(allowed.shape))
    want = oracle_forward(q, k, v, mask=m4, scale=1 / math.sqrt(6))
    got = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), attn_mask=allowed.to(dev))
    assert_close(got, want, torch.float32, f"bool mask {shape}")
    additive = torch.zeros(shape).masked_fill(~allowed, -1e9)
    got = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), attn_mask=additive.to(dev))
    assert_close(got, want, torch.float32, f"additive mask {shape}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
@pytest.mark.parametrize("B,H,Hkv,L,S,D", [(2, 4, 4, 33, 33, 64), (1, 8, 2, 17, 40, 128), (2, 6, 3, 5, 70, 32),
                                            (1, 2, 1, 64, 64, 80), (3, 4, 2, 1, 100, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_dtypes_shapes_gqa(dev, dtype, B, H, Hkv, L, S, D, causal):
    seed = B * 1000 + L * 7 + S
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None, 0.0, causal)
    assert got.dtype == dtype
    want = oracle_forward(q, k, v, is_causal=causal)
    assert_close(got, want, dtype, f"{dtype} {(B, H, Hkv, L, S, D)} causal={causal}")


def test_rows_with_nothing_to_attend_are_zero(dev):
    q, k, v = randn((1, 2, 6, 16), 11), randn((1, 2, 9, 16), 12), randn((1, 2, 9, 16), 13)
    allowed = torch.ones(6, 9, dtype=torch.bool)
    allowed[2] = False
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), allowed.to(dev), 0.0, False)
    assert torch.equal(got[:, :, 2].cpu(), torch.zeros(1, 2, 16))
    neg = torch.zeros(6, 9).masked_fill(~allowed, float("-inf"))
    got2 = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), neg.to(dev), 0.0, False)
    assert torch.equal(got2[:, :, 2].cpu(), torch.zeros(1, 2, 16))
    assert_close(got2, oracle_forward(q, k, v, mask=neg), torch.float32, "blocked rows")


def test_causal_is_top_left_aligned(dev):
    q, k, v = randn((1, 1, 3, 8), 14), randn((1, 1, 7, 8), 15), randn((1, 1, 7, 8), 16)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None, 0.0, True).cpu()
    assert torch.allclose(got[0, 0, 0], v[0, 0, 0], atol=1e-6, rtol=0)
    assert_close(got, oracle_forward(q, k, v, is_causal=True), torch.float32, "L<S causal")


def test_empty_and_keyless_inputs(dev):
    q = torch.randn(1, 2, 3, 8, device=dev)
    empty_k = torch.empty(1, 2, 0, 8, device=dev)
    out = g.flash_attention(q, empty_k, empty_k)
    assert out.shape == (1, 2, 3, 8) and torch.equal(out.cpu(), torch.zeros(1, 2, 3, 8))
    out = g.flash_attention(torch.empty(0, 2, 3, 8, device=dev), torch.empty(0, 2, 4, 8, device=dev),
                            torch.empty(0, 2, 4, 8, device=dev))
    assert out.shape == (0, 2, 3, 8)


def test_strided_views_give_the_same_result(dev):
    # MultiheadAttention hands (B, L, H, D) memory viewed as (B, H, L, D)
    B, L, S, H, D = 2, 19, 23, 4, 64
    for dtype in (torch.float32, torch.float16):
        qb, kb, vb = randn((B, L, H, D), 20, dtype), randn((B, S, H, D), 21, dtype), randn((B, S, H, D), 22, dtype)
        q, k, v = (t.to(dev).transpose(1, 2) for t in (qb, kb, vb))
        got = g.flash_attention(q, k, v, None, 0.0, True)
        ref = g.flash_attention(q.contiguous(), k.contiguous(), v.contiguous(), None, 0.0, True)
        assert torch.equal(got, ref)
        assert_close(got, oracle_forward(q, k, v, is_causal=True), dtype, f"strided {dtype}")
        # an offset view (x[1:]) too
        got = g.flash_attention(q[1:], k[1:], v[1:], None, 0.0, True)
        assert torch.equal(got, ref[1:])


def test_host_tensors_round_trip_through_the_device(dev):
    q, k, v = randn((1, 2, 5, 16), 30), randn((1, 2, 7, 16), 31), randn((1, 2, 7, 16), 32)
    got = g.flash_attention(q, k, v, None, 0.0, True)
    assert got.device.type == "cpu"
    assert_close(got, oracle_forward(q, k, v, is_causal=True), torch.float32, "host io")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("D,Dv", [(64, 96), (256, 256), (200, 160), (1, 1), (300, 40), (48, 130), (16, 8)])
@pytest.mark.parametrize("causal", [False, True])
def test_generic_kernel_chunk_and_value_shapes(dev, dtype, D, Dv, causal):
    # head sizes that select each chunk size of the generic forward (64 / 32 / 16 keys staged per
    # workgroup), 1, 2 or 4 value blocks of 64 with a partial last block, and the unstaged path
    # (D > 256); 150 keys = several chunks with a partial last one, 37 rows = a partial row block
    B, H, Hkv, L, S = 1, 4, 2, 37, 150
    seed = D * 31 + Dv
    q, k, v = randn((B, H, L, D), seed, dtype), randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, Dv), seed + 2, dtype)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None, 0.0, causal)
    assert got.shape == (B, H, L, Dv) and got.dtype == dtype
    want = oracle_forward(q, k, v, is_causal=causal)
    assert_close(got, want, dtype, f"{dtype} D={D} Dv={Dv} causal={causal}")
    # a float mask blocking scattered keys (and every key of row 5) on top
    rng = np.random.default_rng(seed)
    mask = torch.from_numpy(np.where(rng.random((L, S)) < 0.3, -np.inf, rng.standard_normal((L, S)))).to(dtype)
    mask[5] = -math.inf
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), 0.0, causal)
    want = oracle_forward(q, k, v, mask=mask, is_causal=causal)
    assert_close(got, want, dtype, f"{dtype} D={D} Dv={Dv} causal={causal} masked")
    assert torch.equal(got[:, :, 5].cpu(), torch.zeros(B, H, Dv, dtype=dtype))


def test_mixed_dtypes_compute_in_the_wider_type(dev):
    q = randn((1, 2, 9, 32), 40, torch.float16)
    k = randn((1, 2, 11, 32), 41, torch.float32)
    v = randn((1, 2, 11, 32), 42, torch.bfloat16)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None, 0.0, False)
    assert got.dtype == torch.float16
    assert_close(got, oracle_forward(q, k, v), torch.float16, "mixed")


def test_float_mask_dtypes(dev):
    q, k, v = randn((2, 2, 8, 16), 50), randn((2, 2, 12, 16), 51), randn((2, 2, 12, 16), 52)
    bias = randn((2, 1, 1, 12), 53)
    want = oracle_forward(q, k, v, mask=bias)
    for mdt in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        m = bias.to(mdt)
        got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), m.to(dev), 0.0, False)
        assert_close(got, oracle_forward(q, k, v, mask=m), torch.float32, f"mask {mdt}")
    assert want.shape == (2, 2, 8, 16)
