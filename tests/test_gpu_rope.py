"""RoPE on the GPU (gt_rope / gt_rope_backward, F.rope, RoPEFn, KVCache.append(rope=...)).

Parity: every result against the oracle's restatement of ggml_rope_ext (float32 angle chain and
rotation) on the same inputs: float32 max-abs <= 1e-4, float16/bfloat16 within 2e-3 relative
plus the output's half ulp, float64 computed in float32 as the reference does.  The reference's
own RoPE tests (tests/test_losses_and_rope.py:268-391) are ported: values, dtypes kept through
autograd, the backward as the inverse rotation, strided views and position tables.  RoPE on
append: the cache holds bit for bit what rope() then append() stores (Q8_0: the same bytes)."""

import math

import numpy as np
import pytest
import torch

import gguf_train_amd as g
import oracle
from gguf_train_amd.nn import functional as F

from _util import assert_close, oracle_forward, randn, to_oracle

pytestmark = pytest.mark.gpu


def oracle_rope(x, pos, n_dims=None, mode=0, freq_base=10000.0, freq_scale=1.0, backward=False):
    """The oracle on exactly x's values, as float64: for float16/bfloat16 inputs its float32 result
    before the final rounding (the tests' half-ulp allowance covers that rounding; against the
    oracle's own rounded output, a float32 result that lands on the other side of a rounding
    boundary would count a whole ulp)."""
    xo = to_oracle(x.float()) if x.dtype in (torch.float16, torch.bfloat16) else to_oracle(x)
    y = oracle.rope(xo, np.asarray(pos.cpu() if isinstance(pos, torch.Tensor) else pos),
                    n_dims=n_dims, mode=mode, freq_base=freq_base, freq_scale=freq_scale, backward=backward)
    return np.asarray(y).astype(np.float64)


def closed_form(x, positions, n_dims=None, neox=False, freq_base=10000.0, freq_scale=1.0):
    # the reference test's rope_reference (tests/test_losses_and_rope.py:254-265), one head
    d = len(x[0])
    n_dims = d if n_dims is None else n_dims
    out = [list(row) for row in x]
    for s, row in enumerate(x):
        for i in range(n_dims // 2):
            theta = positions[s] * freq_scale * freq_base ** (-2.0 * i / n_dims)
            a, b = (i, i + n_dims // 2) if neox else (2 * i, 2 * i + 1)
            out[s][a] = row[a] * math.cos(theta) - row[b] * math.sin(theta)
            out[s][b] = row[a] * math.sin(theta) + row[b] * math.cos(theta)
    return out


def head(seq=3, dim=6):
    return [[0.5 + 0.25 * s - 0.125 * d + 0.03 * s * d for d in range(dim)] for s in range(seq)]


# ---- the reference's own tests -----------------------------------------------------------------

@pytest.mark.parametrize("on_device", [True, False])
@pytest.mark.parametrize("kwargs", [{}, {"n_dims": 4}, {"neox": True}, {"n_dims": 2, "neox": True},
                                    {"freq_base": 100.0}, {"freq_scale": 0.5}])
def test_values(dev, kwargs, on_device):
    x = head()
    pos = [0, 1, 7]
    call = dict(kwargs)
    mode = 2 if call.pop("neox", False) else 0
    want = np.array(closed_form(x, pos, **kwargs))
    t = torch.tensor([x, x])
    p = torch.tensor(pos)
    if on_device:
        t, p = t.to(dev), p.to(dev)
    got = F.rope(t, p, mode=mode, **call)
    assert tuple(got.shape) == (2, 3, 6) and got.device == t.device
    np.testing.assert_allclose(got[0].cpu().numpy(), want, atol=5e-5)
    np.testing.assert_allclose(got[1].cpu().numpy(), want, atol=5e-5)
    got4 = F.rope(t.reshape(1, 2, 3, 6), p, mode=mode, **call)
    np.testing.assert_allclose(got4[0, 1].cpu().numpy(), want, atol=5e-5)


@pytest.mark.parametrize("dtype,atol", [(torch.float32, 1e-5), (torch.float64, 1e-5), (torch.float16, 1e-2),
                                        (torch.bfloat16, 1e-1)])
def test_result_keeps_the_dtype_of_the_input(dev, dtype, atol):
    x = head()
    want = np.array(closed_form(x, [0, 1, 2]))
    t = torch.tensor([x], dtype=dtype, device=dev, requires_grad=True)
    out = F.rope(t, torch.arange(3, device=dev))
    assert out.dtype == dtype
    np.testing.assert_allclose(out[0].detach().double().cpu().numpy(), want, atol=atol)
    out.sum().backward()
    assert t.grad.dtype == dtype


@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("n_dims", [8, 4])
def test_backward_is_the_inverse_rotation(dev, mode, n_dims):
    x = randn((2, 3, 5, 8), 11).to(dev)
    y = randn((2, 3, 5, 8), 12).to(dev)
    pos = torch.tensor([4, 0, 9, 2, 2], device=dev)
    xr = x.clone().requires_grad_(True)
    out = F.rope(xr, pos, n_dims=n_dims, mode=mode)
    (out * y).sum().backward()
    assert abs((out * y).sum().item() - (x * xr.grad).sum().item()) < 1e-3
    assert abs((out * out).sum().item() - (x * x).sum().item()) < 1e-3
    assert abs((xr.grad * xr.grad).sum().item() - (y * y).sum().item()) < 1e-3
    # and it is the oracle's backward
    assert_close(xr.grad, oracle_rope(y, pos, n_dims=n_dims, mode=mode, backward=True), torch.float32, "grad")


def test_views_and_other_layouts(dev):
    x = head(seq=3, dim=4)
    wide = torch.tensor([[v for value in row for v in (value, -1.0)] for row in x], device=dev).reshape(1, 3, 8)
    got = F.rope(wide[..., ::2], torch.arange(3, device=dev))
    np.testing.assert_allclose(got[0].cpu().numpy(), closed_form(x, [0, 1, 2]), atol=5e-5)
    want = np.array(closed_form(x, [3, 5, 7]))
    t = torch.tensor([x], device=dev)
    np.testing.assert_allclose(F.rope(t, torch.tensor([3, 5, 7], dtype=torch.int32, device=dev))[0].cpu().numpy(),
                               want, atol=5e-5)
    np.testing.assert_allclose(F.rope(t, torch.tensor([3, 0, 5, 0, 7, 0], device=dev)[::2])[0].cpu().numpy(), want,
                               atol=5e-5)
    np.testing.assert_allclose(F.rope(t, torch.tensor([3.0, 5.0, 7.0], device=dev))[0].cpu().numpy(), want,
                               atol=5e-5)
    # a longer position table: the first seq_len entries are used
    np.testing.assert_allclose(F.rope(t, torch.tensor([3, 5, 7, 100, 200], device=dev))[0].cpu().numpy(), want,
                               atol=5e-5)


def test_errors_on_device_tensors(dev):
    x = torch.ones(1, 3, 4, device=dev)
    with pytest.raises(RuntimeError, match="a position for each of the 3 sequence elements"):
        F.rope(x, torch.arange(2, device=dev))
    with pytest.raises(RuntimeError, match="n_dims must be an even number"):
        F.rope(x, torch.arange(3, device=dev), n_dims=3)
    out = F.rope(torch.ones(1, 2, 0, 4, device=dev, dtype=torch.float16), torch.arange(0, device=dev))
    assert tuple(out.shape) == (1, 2, 0, 4) and out.dtype == torch.float16 and out.is_cuda


# ---- parity with the oracle ---------------------------------------------------------------------

CASES = [
    # (shape, dtype, n_dims, mode, freq_base, freq_scale)
    ((2, 4, 33, 64), torch.float32, None, 0, 10000.0, 1.0),
    ((2, 4, 33, 64), torch.float32, None, 2, 10000.0, 1.0),
    ((3, 17, 128), torch.float32, 96, 2, 500000.0, 0.25),
    ((1, 8, 40, 128), torch.float16, None, 0, 10000.0, 1.0),
    ((1, 8, 40, 128), torch.float16, 64, 2, 10000.0, 1.0),
    ((2, 2, 19, 80), torch.bfloat16, 32, 0, 1e6, 1.0),
    ((2, 2, 19, 80), torch.bfloat16, None, 2, 10000.0, 0.5),
    ((1, 3, 9, 10), torch.float64, 6, 0, 10000.0, 1.0),
    ((1, 3, 9, 6), torch.float16, 6, 2, 10000.0, 1.0),  # odd half: single-element groups
]


@pytest.mark.parametrize("backward", [False, True])
@pytest.mark.parametrize("case", CASES)
def test_parity_with_the_oracle(dev, case, backward):
    shape, dtype, n_dims, mode, base, fs = case
    x = randn(shape, 21, dtype).to(dev)
    S = shape[-2]
    pos = torch.from_numpy(np.random.default_rng(22).integers(0, 70000, S)).to(dev)
    got = g.rope(x, pos, n_dims if n_dims is not None else shape[-1], mode, 0, base, fs, backward=backward)
    assert got.dtype == dtype and tuple(got.shape) == shape
    want = oracle_rope(x, pos, n_dims=n_dims, mode=mode, freq_base=base, freq_scale=fs, backward=backward)
    if dtype == torch.float64:
        # computed in float32 like the reference: the float32 tolerance applies
        assert_close(got, want, torch.float32, "rope f64")
    else:
        assert_close(got, want, dtype, "rope")


@pytest.mark.parametrize("mode", [0, 2])
def test_strided_views_equal_the_dense_input(dev, mode):
    # MultiheadAttention-style (B, L, H, D) memory viewed as (B, H, L, D), and an offset view
    base = randn((2, 50, 8, 128), 31, torch.float16).to(dev)
    x = base.transpose(1, 2)
    pos = torch.arange(50, device=dev) + 1000
    got = F.rope(x, pos, mode=mode)
    want = F.rope(x.contiguous(), pos, mode=mode)
    assert torch.equal(got, want)
    off = base[:, 1:, 1:7].transpose(1, 2)
    assert torch.equal(F.rope(off, pos[:49], mode=mode), F.rope(off.contiguous(), pos[:49], mode=mode))


def test_prefill_shape(dev):
    # the prefill workload's q: B=4 H=32 L=2048 D=128 float16, positions 0..2047
    x = randn((4, 32, 2048, 128), 41, torch.float16).to(dev)
    pos = torch.arange(2048, device=dev)
    got = F.rope(x, pos, mode=2)
    sl = (slice(None), slice(0, 32, 7))
    assert_close(got[sl], oracle_rope(x[sl], pos, mode=2), torch.float16, "rope prefill shape")


# ---- RoPE on append into the KV cache -------------------------------------------------------------

@pytest.mark.parametrize("mode,n_dims", [(0, None), (2, None), (2, 64)])
@pytest.mark.parametrize("cache_dtype,src_dtype", [(torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                                                   (torch.float32, torch.float32), (torch.float16, torch.float32),
                                                   (torch.float32, torch.float16), ("q8_0", torch.float32),
                                                   ("q8_0", torch.float16)])
def test_append_with_rope_equals_rope_then_append(dev, cache_dtype, src_dtype, mode, n_dims):
    B, Hkv, D = 2, 4, 128
    nd = D if n_dims is None else n_dims
    rope = {"n_dims": nd, "mode": mode, "freq_base": 10000.0, "freq_scale": 1.0}
    fused = g.KVCache(B, Hkv, 256, D, cache_dtype, dev)
    plain = g.KVCache(B, Hkv, 256, D, cache_dtype, dev)
    start = 0
    for T, seed in ((37, 1), (1, 2), (90, 3)):
        k = randn((B, Hkv, T, D), seed, src_dtype).to(dev)
        v = randn((B, Hkv, T, D), seed + 10, src_dtype).to(dev)
        fused.append(k, v, rope=rope)
        pos = torch.arange(start, start + T, device=dev)
        plain.append(F.rope(k, pos, n_dims=nd, mode=mode), v)
        start += T
    for a, b in ((fused.keys(), plain.keys()), (fused.values(), plain.values())):
        if cache_dtype == "q8_0":
            assert torch.equal(a.data, b.data)
        else:
            assert torch.equal(a, b)
    # and the rotated keys are the oracle's rope of the keys at their cache positions
    if cache_dtype == torch.float32 and src_dtype == torch.float32:
        k = randn((B, Hkv, 5, D), 99, torch.float32).to(dev)
        fused.append(k, k, rope=rope)
        want = oracle_rope(k, torch.arange(start, start + 5), n_dims=nd, mode=mode)
        assert_close(fused.keys()[:, :, start:start + 5], want, torch.float32, "rotated keys")


def test_append_with_rope_per_sequence_lengths(dev):
    # sequences of different lengths: each key row is rotated at its own cache position
    B, Hkv, D = 3, 2, 64
    cache = g.KVCache(B, Hkv, 64, D, torch.float32, dev)
    k0 = randn((B, Hkv, 10, D), 5).to(dev)
    cache.append(k0, k0)
    cache.clear(1)
    k1 = randn((B, Hkv, 4, D), 6).to(dev)
    cache.append(k1, k1, rope={"mode": 2})
    keys = cache.keys()
    for b, start in ((0, 10), (1, 0), (2, 10)):
        want = oracle_rope(k1[b:b + 1], torch.arange(start, start + 4), mode=2)
        assert_close(keys[b:b + 1, :, start:start + 4], want, torch.float32, f"sequence {b}")


def test_decode_over_a_rotated_cache_equals_attention_of_rotated_q_and_k(dev):
    B, H, Hkv, T, D = 2, 8, 2, 65, 128
    q = randn((B, H, T, D), 7, torch.float16).to(dev)
    k = randn((B, Hkv, T, D), 8, torch.float16).to(dev)
    v = randn((B, Hkv, T, D), 9, torch.float16).to(dev)
    pos = torch.arange(T, device=dev)
    qr, kr = F.rope(q, pos, mode=2), F.rope(k, pos, mode=2)
    cache = g.KVCache(B, Hkv, 128, D, torch.float16, dev)
    cache.append(k[:, :, :-1], v[:, :, :-1], rope={"mode": 2})
    cache.append(k[:, :, -1:], v[:, :, -1:], rope={"mode": 2})
    assert torch.equal(cache.keys()[:, :, :T], kr)
    got = cache.attention(qr[:, :, -1:])
    want = oracle_forward(qr[:, :, -1:], kr, v)
    assert_close(got, want, torch.float16, "decode over the rotated cache")


def test_append_rope_errors(dev):
    cache = g.KVCache(1, 1, 8, 64, torch.float16, dev)
    k = torch.zeros(1, 1, 2, 64, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="mode must be 0 \\(normal\\) or 2 \\(NeoX\\)"):
        cache.append(k, k, rope={"mode": 1})
    with pytest.raises(RuntimeError, match="n_dims must be an even number between 2 and the head dimension 64"):
        cache.append(k, k, rope={"n_dims": 66})
    with pytest.raises(TypeError):
        cache.append(k, k, rope={"theta": 1.0})
    assert cache.lengths == [0]


# ---- attention of rotated queries and keys (gt_flash_attention_rope) ------------------------------

FUSED_CASES = [
    # (dtype, B, H, Hkv, L, S, D, mode, causal)  -- the prefill kernel rotates q as it loads it
    (torch.float16, 2, 8, 2, 300, 300, 128, 2, True),
    (torch.float16, 1, 4, 4, 256, 256, 128, 0, True),
    (torch.bfloat16, 2, 4, 2, 200, 200, 64, 2, True),
    (torch.bfloat16, 1, 4, 1, 130, 130, 64, 0, False),
    (torch.float16, 1, 8, 8, 512, 512, 128, 2, False),
]


@pytest.mark.parametrize("case", FUSED_CASES)
def test_fused_query_rope_equals_rope_then_attention(dev, case):
    dtype, B, H, Hkv, L, S, D, mode, causal = case
    q = randn((B, H, L, D), 51, dtype).to(dev)
    k = randn((B, Hkv, S, D), 52, dtype).to(dev)
    v = randn((B, Hkv, S, D), 53, dtype).to(dev)
    pos = torch.from_numpy(np.random.default_rng(54).permutation(4 * max(L, S))[: max(L, S)]).to(dev)
    got = g.flash_attention_rope(q, k, v, pos, None, 0.0, causal, None, mode)
    qr, kr = F.rope(q, pos, mode=mode), F.rope(k, pos, mode=mode)
    want = g.flash_attention(qr, kr, v, None, 0.0, causal)
    # the same kernel on the same rotated values: bit for bit
    assert torch.equal(got, want)
    ref = oracle_forward(qr, kr, v, is_causal=causal)
    assert_close(got, ref, dtype, "fused rope attention")


def test_fused_query_rope_with_a_key_padding_mask(dev):
    B, H, L, D = 2, 4, 257, 128
    q, k, v = (randn((B, H, L, D), s, torch.float16).to(dev) for s in (61, 62, 63))
    mask = torch.zeros(B, 1, 1, L, device=dev)
    mask[0, ..., 200:] = float("-inf")
    pos = torch.arange(L, device=dev) + 17
    got = g.flash_attention_rope(q, k, v, pos, mask, 0.0, True, None, 2)
    want = g.flash_attention(F.rope(q, pos, mode=2), F.rope(k, pos, mode=2), v, mask, 0.0, True)
    assert torch.equal(got, want)


@pytest.mark.parametrize("variant", ["float32", "partial_dims", "bool_mask", "decode", "host"])
def test_unfused_shapes_rotate_q_first(dev, variant):
    B, H, L, D = 1, 4, 96, 64
    dtype = torch.float32 if variant == "float32" else torch.float16
    q, k, v = (randn((B, H, L, D), s, dtype).to(dev) for s in (71, 72, 73))
    pos = torch.arange(L, device=dev)
    n_dims, mask, causal = None, None, True
    if variant == "partial_dims":
        n_dims = 32
    if variant == "bool_mask":
        mask = torch.rand(1, 1, L, L, generator=torch.Generator().manual_seed(3)).to(dev) > 0.3
        mask[..., 0] = True
        causal = False
    if variant == "decode":
        q = q[:, :, -1:].contiguous()
        causal = False
    if variant == "host":
        q, k, v, pos = q.cpu(), k.cpu(), v.cpu(), pos.cpu()
    nd = D if n_dims is None else n_dims
    got = g.flash_attention_rope(q, k, v, pos, mask, 0.0, causal, n_dims, 0)
    want = g.flash_attention(F.rope(q, pos, n_dims=nd), F.rope(k, pos, n_dims=nd), v, mask, 0.0, causal)
    assert got.device == q.device
    assert torch.equal(got, want)


def test_fused_rope_errors(dev):
    q = torch.zeros(1, 2, 8, 64, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="a position for each of the 8 sequence elements"):
        g.flash_attention_rope(q, q, q, torch.arange(4, device=dev))
    with pytest.raises(RuntimeError, match="mode must be 0 \\(normal\\) or 2 \\(NeoX\\)"):
        g.flash_attention_rope(q, q, q, torch.arange(8, device=dev), mode=1)
    with pytest.raises(RuntimeError, match="n_dims must be an even number"):
        g.flash_attention_rope(q, q, q, torch.arange(8, device=dev), n_dims=65)
