"""KV cache on the GPU (gguf_train_amd.KVCache, gt_kv_cache_*).

The reference's decode cache is llama.cpp's, behind LlamaContext; its own test of it is the
invariant that a sequence fed in two pieces (the tail at pos_offset) gives what the whole
sequence gives (tests/test_llama_bridge.py:105-111).  Here the same invariant, decode
step by step against causal prefill rows, per-sequence lengths, clear, GQA, Q8_0 rows that
are gt_quantize's bytes, and the error behaviour (positions that do not continue the cache,
capacity).  Every attention result is checked against the float64 oracle with the mask that
the cache semantics define: key s of sequence b is present when s < len_b, and query row l
(token len_b - L + l) sees s <= len_b - L + l when causal."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
import oracle

from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


def cache_mask(lengths, L, S, causal):
    m = torch.zeros(len(lengths), 1, L, S, dtype=torch.bool)
    for b, n in enumerate(lengths):
        for l in range(L):
            last = n - L + l if causal else n - 1
            m[b, 0, l, : last + 1] = True
    return m


def dense_kv(cache, dtype):
    """The cached K and V as dense float tensors of the cache's values (Q8_0: dequantized)."""
    k, v = cache.keys(), cache.values()
    if cache.dtype == "q8_0":
        k, v = g.dequantize(k, torch.float32), g.dequantize(v, torch.float32)
    return k, v


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128, 96])  # 96: heads padded for the MFMA kernels (fp16 / bf16)
def test_two_pieces_equal_the_whole_sequence(dev, dtype, D):
    B, H, Hkv, T = 2, 8, 2, 300
    q, k, v = randn((B, H, T, D), 1, dtype), randn((B, Hkv, T, D), 2, dtype), randn((B, Hkv, T, D), 3, dtype)
    want = oracle_forward(q, k, v, is_causal=True)
    cache = g.KVCache(B, Hkv, 512, D, dtype, dev)
    cut = 137
    cache.append(k[:, :, :cut].to(dev), v[:, :, :cut].to(dev))
    head = cache.attention(q[:, :, :cut].to(dev))
    cache.append(k[:, :, cut:].to(dev), v[:, :, cut:].to(dev), pos_offset=cut)
    tail = cache.attention(q[:, :, cut:].to(dev))
    assert cache.lengths == [T, T]
    assert_close(torch.cat([head, tail], dim=2), want, dtype, "two pieces")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_decode_steps_equal_prefill_rows(dev, dtype):
    B, H, Hkv, T, D = 3, 8, 2, 40, 128
    q, k, v = randn((B, H, T, D), 4, dtype), randn((B, Hkv, T, D), 5, dtype), randn((B, Hkv, T, D), 6, dtype)
    want = oracle_forward(q, k, v, is_causal=True)
    cache = g.KVCache(B, Hkv, 64, D, dtype, dev)
    rows = []
    for t in range(T):
        cache.append(k[:, :, t:t + 1].to(dev), v[:, :, t:t + 1].to(dev), pos_offset=t)
        rows.append(cache.attention(q[:, :, t:t + 1].to(dev)))
    assert_close(torch.cat(rows, dim=2), want, dtype, "decode steps")


@pytest.mark.parametrize("D", [64, 80])  # 80: heads padded for the MFMA kernels
def test_per_sequence_lengths_and_clear(dev, D):
    dtype, B, H, Hkv = torch.float16, 3, 4, 4
    cache = g.KVCache(B, Hkv, 256, D, dtype, dev)
    k1, v1 = randn((B, Hkv, 100, D), 7, dtype), randn((B, Hkv, 100, D), 8, dtype)
    cache.append(k1.to(dev), v1.to(dev))
    cache.clear(1)                       # sequence 1 starts over
    k2, v2 = randn((B, Hkv, 30, D), 9, dtype), randn((B, Hkv, 30, D), 10, dtype)
    cache.append(k2.to(dev), v2.to(dev))
    assert cache.lengths == [130, 30, 130]
    K, V = dense_kv(cache, dtype)
    S = 130
    for L, causal in ((1, True), (1, False), (30, True), (17, False)):
        q = randn((B, H, L, D), 11 + L, dtype)
        got = cache.attention(q.to(dev), is_causal=causal)
        want = oracle_forward(q, K[:, :, :S].cpu(), V[:, :, :S].cpu(), mask=cache_mask(cache.lengths, L, S, causal))
        assert_close(got, want, dtype, f"L={L} causal={causal}")
    # sequence 1's rows are what was appended after the clear
    assert torch.equal(K[1, :, :30].cpu(), k2[1])
    cache.clear()
    assert cache.lengths == [0, 0, 0]


@pytest.mark.parametrize("D", [64, 128])
def test_q8_0_cache_rows_and_attention(dev, D):
    B, H, Hkv, T = 2, 8, 2, 300
    k, v = randn((B, Hkv, T, D), 12), randn((B, Hkv, T, D), 13)
    cache = g.KVCache(B, Hkv, 320, D, "q8_0", dev)
    cache.append(k[:, :, :200].to(dev), v[:, :, :200].to(dev))
    cache.append(k[:, :, 200:].half().to(dev), v[:, :, 200:].half().to(dev))  # any float dtype
    kb = cache.keys().data.cpu().numpy().reshape(B, Hkv, 320, D // 32 * 34)
    for b in range(B):
        for h in range(Hkv):
            rows = np.concatenate([k[b, h, :200].numpy(), k[b, h, 200:].half().float().numpy()])
            want = oracle.q8_0_quantize(rows).reshape(T, D // 32 * 34)
            assert np.array_equal(kb[b, h, :T], want), (b, h)
    K, V = dense_kv(cache, torch.float16)
    for L in (1, 5):
        q = randn((B, H, L, D), 14 + L, torch.float16)
        got = cache.attention(q.to(dev))
        want = oracle_forward(q, K[:, :, :T].cpu(), V[:, :, :T].cpu(), mask=cache_mask(cache.lengths, L, T, True))
        assert_close(got, want, torch.float16, f"q8_0 L={L}")


@pytest.mark.parametrize("rope", [None, {"mode": 0}, {"mode": 2}, {"mode": 2, "n_dims": 64}, {"mode": 0, "n_dims": 40}])
@pytest.mark.parametrize("cache_dtype,src_dtype", [
    (torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
    (torch.float16, torch.float32), (torch.bfloat16, torch.float16), (torch.float32, torch.bfloat16),
    ("q8_0", torch.float32), ("q8_0", torch.float16), ("q8_0", torch.bfloat16)])
def test_dense_rows_append_the_same_bytes_as_strided_rows(dev, cache_dtype, src_dtype, rope):
    """Dense, 16-byte aligned source rows (appended 8 elements per thread) and the same values as
    a view with a non-unit stride along D (one element per thread) fill the cache with the same
    bytes, RoPE on append included (n_dims 40 is not a multiple of 16: both take the general
    path there)."""
    B, Hkv, D = 2, 3, 128
    dense = g.KVCache(B, Hkv, 64, D, cache_dtype, dev)
    strided = g.KVCache(B, Hkv, 64, D, cache_dtype, dev)
    for T, seed in ((45, 1), (7, 2)):
        k = randn((B, Hkv, T, D), seed, src_dtype, scale=3.0).to(dev)
        v = randn((B, Hkv, T, D), seed + 10, src_dtype, scale=3.0).to(dev)
        k[0, 0, 0, :32] = 0.0  # an all-zero Q8_0 block
        ks, vs = (x.transpose(2, 3).contiguous().transpose(2, 3) for x in (k, v))
        assert ks.stride(3) == T and torch.equal(ks, k)
        dense.append(k, v, rope=rope)
        strided.append(ks, vs, rope=rope)
    for a, b in ((dense.keys(), strided.keys()), (dense.values(), strided.values())):
        if cache_dtype == "q8_0":
            assert torch.equal(a.data, b.data)
        else:
            assert torch.equal(a.view(torch.int16 if a.element_size() == 2 else torch.int32),
                               b.view(torch.int16 if b.element_size() == 2 else torch.int32))


@pytest.mark.parametrize("dtype", [torch.float16, "q8_0"])
def test_a_new_cache_starts_zero_filled(dev, dtype):
    """A cache's storage is zero-filled when it is created (by a fill kernel, byte by byte past
    the last whole 16-byte chunk: 2 x 7 rows of 68-byte Q8_0 blocks are 952 bytes), also where
    it takes over memory that a freed cache had written."""
    B, Hkv, cap, D = 2, 1, 7, 64
    first = g.KVCache(B, Hkv, cap, D, dtype, dev)
    first.append(randn((B, Hkv, cap, D), 30).to(dev), randn((B, Hkv, cap, D), 31).to(dev))
    torch.cuda.synchronize()
    del first
    cache = g.KVCache(B, Hkv, cap, D, dtype, dev)
    for name, st in (("keys", cache.keys()), ("values", cache.values())):
        data = st.data if dtype == "q8_0" else st
        nbytes = data.numel() * data.element_size()
        assert nbytes == (B * Hkv * cap * (D // 32 * 34) if dtype == "q8_0" else B * Hkv * cap * D * 2)
        assert not data.contiguous().view(torch.uint8).any(), name


def test_host_inputs_and_explicit_scale(dev):
    dtype, B, H, Hkv, D = torch.float16, 1, 2, 1, 128
    cache = g.KVCache(B, Hkv, 16, D, dtype, dev)
    k, v = randn((B, Hkv, 9, D), 20, dtype), randn((B, Hkv, 9, D), 21, dtype)
    cache.append(k, v)  # host tensors
    q = randn((B, H, 2, D), 22, dtype)
    got = cache.attention(q, scale=0.3)
    assert got.device.type == "cpu"
    assert_close(got, oracle_forward(q, k, v, mask=cache_mask([9], 2, 9, True), scale=0.3), dtype, "host")


def test_errors(dev):
    cache = g.KVCache(2, 2, 8, 64, torch.float16, dev)
    k = torch.zeros(2, 2, 5, 64, dtype=torch.float16, device=dev)
    cache.append(k, k)
    with pytest.raises(RuntimeError, match="do not continue"):
        cache.append(k[:, :, :1], k[:, :, :1], pos_offset=3)
    with pytest.raises(RuntimeError, match="capacity = 8"):
        cache.append(k, k)
    assert cache.lengths == [5, 5]  # nothing written by the failed calls
    with pytest.raises(RuntimeError, match="fewer than"):
        cache.attention(torch.zeros(2, 4, 6, 64, dtype=torch.float16, device=dev))
    with pytest.raises(RuntimeError, match="does not match the cache"):
        cache.append(k[:, :1], k[:, :1])
    with pytest.raises(RuntimeError, match="multiple of 32"):
        g.KVCache(1, 1, 8, 48, "q8_0", dev)


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
def test_q8_0_cache_prefill_chunk_on_mfma(dev, qdtype):
    # a prefill chunk over a Q8_0 cache much larger than what it holds: only the rows the
    # sequences hold are dequantized (float16 for float16 queries, attended by the MFMA prefill
    # kernel with the cache's lengths and query positions; float32 for bfloat16 queries)
    from gguf_train_amd import _C

    B, H, Hkv, D, cap = 2, 8, 2, 128, 4096
    k, v = randn((B, Hkv, 430, D), 31), randn((B, Hkv, 430, D), 32)
    cache = g.KVCache(B, Hkv, cap, D, "q8_0", dev)
    cache.append(k[:, :, :300].to(dev), v[:, :, :300].to(dev))
    cache.append(k[:, :, 300:].to(dev), v[:, :, 300:].to(dev))
    T, L = 430, 130
    q = randn((B, H, L, D), 33, qdtype, 0.5)
    got = cache.attention(q.to(dev))
    launch = _C.last_launch()
    # float16 queries: float16 K/V and the fp16 kernel; float32: the float32 MFMA kernel; bfloat16
    # queries over float32 K/V (mixed dtypes, bfloat16 output): the generic kernel in float32
    want_kernel = {torch.float16: "prefill f16 D=128", torch.float32: "prefill f32 D=128"}.get(qdtype, "generic f32")
    assert launch.startswith("dequantize q8_0 cache rows") and want_kernel in launch, launch
    K, V = dense_kv(cache, torch.float32)
    want = oracle_forward(q, K[:, :, :T].cpu(), V[:, :, :T].cpu(), mask=cache_mask(cache.lengths, L, T, True))
    assert_close(got, want, qdtype, "q8_0 cache prefill chunk")
