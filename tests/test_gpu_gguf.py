"""GGUF tensors straight into HBM (gt_gguf_get_tensor_device): the bytes that land on the device
are the file's bytes (every plain type, Q8_0 blocks, a tensor larger than all the pinned staging
chunks together), dequantize=True is the oracle's Q8_0 closed form bit for bit, and K/V read from a file
feed the attention kernels and the KV cache exactly as the same blocks quantized in memory do.
The reference reads a GGUF tensor to the host (csrc/gt_ops_extra.cpp:1846-1918) and moves it
with gt_tensor_to_device; the device reader must give the same tensor."""

import struct
import time

import numpy as np
import pytest
import torch

import gguf_train_amd as g
import oracle
from gguf_train_amd import _bridge
from gguf_train_amd.gguf import load_gguf
from gguf_train_amd.nn import functional as F

import _gguf_file as gf
from _gguf_file import GGUFBuilder
from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


def test_device_reader_gives_the_host_readers_tensors(dev, tmp_path):
    rng = np.random.default_rng(5)
    b = GGUFBuilder().kv("general.name", gf.STRING, "kv")
    b.tensor("f32", [8, 3, 2], gf.T_F32, rng.standard_normal(48).astype(np.float32).tobytes())
    b.tensor("f16", [16, 5], gf.T_F16, rng.standard_normal(80).astype(np.float16).tobytes())
    b.tensor("bf16", [4, 4], gf.T_BF16, oracle.f32_to_bf16_bits(rng.standard_normal(16).astype(np.float32)).tobytes())
    b.tensor("f64", [3], gf.T_F64, rng.standard_normal(3).tobytes())
    b.tensor("i32", [5, 2], gf.T_I32, rng.integers(-9, 9, 10).astype(np.int32).tobytes())
    b.tensor("i64", [2], gf.T_I64, struct.pack("<2q", -2**63, 2**63 - 1))
    b.kv("gguf_train.dtype.flags", gf.STRING, "bool").tensor("flags", [3], gf.T_I8, bytes([1, 0, 1]))
    b.tensor("q8", [64, 2, 3], gf.T_Q8_0, oracle.q8_0_quantize(rng.standard_normal(384).astype(np.float32)).tobytes())
    b.tensor("empty", [0, 4], gf.T_F32, b"")
    p = b.write(tmp_path / "mixed.gguf")
    host, on_dev = load_gguf(p), load_gguf(p, device=dev)
    assert list(host.keys()) == list(on_dev.keys()) and on_dev.metadata == host.metadata
    for name in host.keys():
        h, d = host[name], on_dev[name]
        if isinstance(h, _bridge.QuantizedTensor):
            assert isinstance(d, _bridge.QuantizedTensor) and d.device.type == "cuda" and d.shape == h.shape
            assert torch.equal(d.data.cpu(), h.data)
        else:
            assert d.is_cuda and d.dtype == h.dtype and d.shape == h.shape, name
            assert torch.equal(d.cpu(), h), name


def test_dequantize_on_the_device_is_the_closed_form(dev, tmp_path):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(32 * 257) * rng.choice([1e-3, 1.0, 30.0], 32 * 257)).astype(np.float32)
    x[:32] = 0.0
    blocks = oracle.q8_0_quantize(x)
    p = GGUFBuilder().tensor("w", [32 * 257], gf.T_Q8_0, blocks.tobytes()).write(tmp_path / "w.gguf")
    want = oracle.q8_0_dequantize(blocks)
    d = load_gguf(p, dequantize=True, device=dev)["w"]
    assert d.is_cuda and d.dtype == torch.float32 and d.shape == (32 * 257,)
    assert np.array_equal(d.cpu().numpy(), want)
    h = load_gguf(p, dequantize=True)["w"]  # host result, dequantized by the same kernel
    assert h.device.type == "cpu" and np.array_equal(h.numpy(), want)


def test_a_tensor_larger_than_the_staging_chunks(dev, tmp_path):
    # 200 MiB of Q8_0 blocks: 13 chunks of 16 MiB over the 8 reader threads, the last one partial
    n_blocks = (200 << 20) // 34
    rng = np.random.default_rng(7)
    blocks = rng.integers(0, 256, n_blocks * 34, dtype=np.uint8)
    blocks.reshape(n_blocks, 34)[:, 1] &= 0x3B  # keep the fp16 scales finite
    p = GGUFBuilder().tensor("big", [n_blocks * 32], gf.T_Q8_0, blocks.tobytes()).write(tmp_path / "big.gguf")
    for attempt in range(2):  # the first load also allocates the pinned staging chunks
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        d = load_gguf(p, device=dev)["big"]
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        print(f"[gguf] load {attempt}: {blocks.nbytes / 2**20:.0f} MiB file (page cache) -> HBM in {dt * 1e3:.1f} ms "
              f"({blocks.nbytes / dt / 1e9:.2f} GB/s)")
        assert d.data.numel() == blocks.nbytes
        assert torch.equal(d.data.cpu(), torch.from_numpy(blocks))
    # the host -> device copy rate of pinned memory, for comparison
    pinned = torch.from_numpy(blocks).pin_memory()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    pinned.to(dev, non_blocking=True)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"[gguf] pinned host -> HBM copy of the same bytes: {dt * 1e3:.1f} ms ({blocks.nbytes / dt / 1e9:.2f} GB/s)")


def test_kv_read_from_a_file_feeds_decode_and_the_cache(dev, tmp_path):
    # a Q8_0 K/V pair written as GGUF (B, Hkv, S, D) = ne [D, S, Hkv, B]
    B, H, Hkv, S, D = 2, 8, 2, 160, 128
    k = randn((B, Hkv, S, D), 11, torch.float32)
    v = randn((B, Hkv, S, D), 12, torch.float32)
    kq, vq = oracle.q8_0_quantize(k.numpy()), oracle.q8_0_quantize(v.numpy())
    p = (GGUFBuilder().tensor("cache.k", [D, S, Hkv, B], gf.T_Q8_0, kq.tobytes())
         .tensor("cache.v", [D, S, Hkv, B], gf.T_Q8_0, vq.tobytes()).write(tmp_path / "kv.gguf"))
    f = load_gguf(p, device=dev)
    kd, vd = f["cache.k"], f["cache.v"]
    assert kd.shape == (B, Hkv, S, D)
    q = randn((B, H, 1, D), 13, torch.float16).to(dev)
    out = F.scaled_dot_product_attention(q, kd, vd)
    # the same blocks made in memory give the same result, bit for bit
    mem_k = _bridge.QuantizedTensor(torch.from_numpy(kq).to(dev), (B, Hkv, S, D))
    mem_v = _bridge.QuantizedTensor(torch.from_numpy(vq).to(dev), (B, Hkv, S, D))
    assert torch.equal(out, F.scaled_dot_product_attention(q, mem_k, mem_v))
    kf = torch.from_numpy(oracle.q8_0_dequantize(kq).reshape(B, Hkv, S, D))
    vf = torch.from_numpy(oracle.q8_0_dequantize(vq).reshape(B, Hkv, S, D))
    assert_close(out.cpu(), oracle_forward(q.cpu(), kf, vf), torch.float16)

    # into a Q8_0 cache: the blocks are stored unchanged, in two pieces
    cache = g.KVCache(B, Hkv, 256, D, dtype="q8_0", device=dev)
    half = _bridge.QuantizedTensor(torch.from_numpy(kq.reshape(B, Hkv, S, -1)[:, :, :100].copy()).to(dev).reshape(-1),
                                   (B, Hkv, 100, D))
    halfv = _bridge.QuantizedTensor(torch.from_numpy(vq.reshape(B, Hkv, S, -1)[:, :, :100].copy()).to(dev).reshape(-1),
                                    (B, Hkv, 100, D))
    rest = _bridge.QuantizedTensor(torch.from_numpy(kq.reshape(B, Hkv, S, -1)[:, :, 100:].copy()).reshape(-1),
                                   (B, Hkv, S - 100, D))  # a host tensor
    restv = _bridge.QuantizedTensor(torch.from_numpy(vq.reshape(B, Hkv, S, -1)[:, :, 100:].copy()).reshape(-1),
                                    (B, Hkv, S - 100, D))
    cache.append(half, halfv)
    cache.append(rest, restv, pos_offset=100)
    assert cache.lengths == [S, S]
    stored = cache.keys().data.cpu().numpy().reshape(B, Hkv, 256, -1)[:, :, :S]
    assert np.array_equal(stored, kq.reshape(B, Hkv, S, -1))
    assert torch.equal(cache.attention(q, is_causal=False), out)

    # into a float16 cache: the dequantized values, rounded to float16
    c16 = g.KVCache(B, Hkv, 256, D, dtype=torch.float16, device=dev)
    c16.append(kd, vd)
    assert torch.equal(c16.keys()[:, :, :S].cpu(), kf.half())
    assert torch.equal(c16.values()[:, :, :S].cpu(), vf.half())


def test_q8_0_rows_need_whole_blocks(dev):
    cache = g.KVCache(1, 1, 8, 48, dtype=torch.float16, device=dev)
    rows = g.quantize(torch.zeros(1, 1, 2, 48, device=dev))  # 96 values: 3 blocks across rows
    with pytest.raises(RuntimeError, match="multiple of 32"):
        cache.append(rows, rows)
