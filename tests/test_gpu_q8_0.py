"""GGUF Q8_0 on the GPU: quantized bytes and dequantized values bit-exact against the oracle's
ggml restatement, and attention over a Q8_0 K/V cache against the oracle on the dequantized
values (the reference's only meaning for it: gt_dequantize, then attention)."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
import oracle
from gguf_train_amd.nn import functional as F

from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


def test_quantize_and_dequantize_are_bit_exact(dev):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(32 * 4096) * rng.choice([1e-4, 1.0, 50.0], 32 * 4096)).astype(np.float32)
    x[:32] = 0.0                      # an all-zero block
    x[32:64] = np.arange(32) - 16.5   # ties after scaling
    x[64] = 127.0
    q = g.quantize(torch.from_numpy(x).to(dev).reshape(64, 2048))
    assert q.shape == (64, 2048) and q.data.numel() == x.size // 32 * 34
    want = oracle.q8_0_quantize(x)
    assert np.array_equal(q.data.cpu().numpy(), want)
    for dt in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        y = g.dequantize(q, dt)
        ref = oracle.q8_0_dequantize(want).reshape(64, 2048)
        assert np.array_equal(y.float().cpu().numpy(), torch.from_numpy(ref).to(dt).float().numpy())


def test_quantize_host_and_half_inputs(dev):
    x = randn((4, 96), 3, torch.float16)
    q = g.quantize(x)  # host input: quantized on the device, returned on the host
    assert q.data.device.type == "cpu"
    assert np.array_equal(q.data.numpy(), oracle.q8_0_quantize(x.float().numpy()))


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16, torch.float32])
def test_attention_over_a_q8_0_cache(dev, qdtype):
    B, H, Hkv, S, D = 2, 8, 2, 300, 128
    q = randn((B, H, 1, D), 10, qdtype)
    k, v = randn((B, Hkv, S, D), 11), randn((B, Hkv, S, D), 12)
    kq, vq = g.quantize(k.to(dev)), g.quantize(v.to(dev))
    got = F.scaled_dot_product_attention(q.to(dev), kq, vq)
    assert got.dtype == qdtype
    kd = torch.from_numpy(oracle.q8_0_dequantize(oracle.q8_0_quantize(k.numpy())).reshape(k.shape))
    vd = torch.from_numpy(oracle.q8_0_dequantize(oracle.q8_0_quantize(v.numpy())).reshape(v.shape))
    want = oracle_forward(q, kd, vd)
    assert_close(got, want, torch.float16 if qdtype != torch.float32 else torch.float32, "q8_0 decode")
