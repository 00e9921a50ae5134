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


@pytest.mark.parametrize("nblocks,offset", [(64 * 37 + 13, 0), (64 * 5, 1), (7, 3)])
def test_quantize_tiles_tails_and_misaligned_inputs(dev, nblocks, offset):
    """Whole 64-block tiles (assembled in LDS, 16-byte stores), a ragged last tile and an input
    view that starts off 16-byte alignment (element loads) all give the oracle's bytes."""
    rng = np.random.default_rng(nblocks + offset)
    x = (rng.standard_normal(nblocks * 32 + offset) * rng.choice([1e-3, 1.0, 300.0], nblocks * 32 + offset))
    x = x.astype(np.float32)
    x[offset:offset + 32] = 0.0
    xd = torch.from_numpy(x).to(dev)[offset:].reshape(nblocks, 32)
    assert xd.data_ptr() % 16 == (4 * offset) % 16
    q = g.quantize(xd)
    assert np.array_equal(q.data.cpu().numpy(), oracle.q8_0_quantize(x[offset:]))


def test_dequantize_to_float16_every_scale_and_quant(dev):
    """Every Q8_0 value q * d (all 2^16 scale bit patterns, including subnormal, infinite and NaN
    scales, times all 256 int8 quants) dequantized to float16 on the device equals the
    round-to-nearest-even float16 of the exact float32 product, computed here by numpy; NaN
    products stay NaN (their payload bits are not compared: inf * 0 has no portable payload)."""
    nd = 65536
    d_bits = np.arange(nd, dtype=np.uint32).astype(np.uint16)
    quants = (np.arange(256) - 128).astype(np.int8).reshape(8, 32)  # 8 blocks per scale
    nb = nd * 8
    blocks = np.zeros((nb, 34), np.uint8)
    blocks[:, 0:2] = np.repeat(d_bits, 8).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:] = np.tile(quants, (nd, 1)).view(np.uint8)
    qt = g.QuantizedTensor(torch.from_numpy(blocks.reshape(-1)).to(dev), (nb, 32))
    got = g.dequantize(qt, torch.float16).cpu().numpy().view(np.uint16).reshape(nb, 32)
    with np.errstate(over="ignore", invalid="ignore"):
        y = np.tile(quants, (nd, 1)).astype(np.float32) * np.repeat(d_bits.view(np.float16).astype(np.float32), 8)[:, None]
        want = y.astype(np.float16).view(np.uint16)
    nan = np.isnan(y)
    assert nan.any() and np.isinf(y).any() and (np.abs(y[y != 0]) < 2 ** -14).any()
    assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(got.view(np.float16)[nan]).all()


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


@pytest.mark.parametrize("G,D", [(1, 64), (2, 128), (4, 128), (8, 128), (4, 64), (8, 64)])
@pytest.mark.parametrize("S", [1, 255, 256, 1000, 8192])
def test_q8_0_decode_kernel_shapes(dev, G, D, S):
    B, Hkv = 2, 2
    seed = G * 1000 + D + S
    q = randn((B, Hkv * G, 1, D), seed, torch.float16)
    k, v = randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    kb, vb = oracle.q8_0_quantize(k.numpy()), oracle.q8_0_quantize(v.numpy())
    kq = g.QuantizedTensor(torch.from_numpy(kb).to(dev), tuple(k.shape))
    vq = g.QuantizedTensor(torch.from_numpy(vb).to(dev), tuple(v.shape))
    got = g.flash_attention(q.to(dev), kq, vq)
    kd = torch.from_numpy(oracle.q8_0_dequantize(kb).reshape(k.shape))
    vd = torch.from_numpy(oracle.q8_0_dequantize(vb).reshape(v.shape))
    assert_close(got, oracle_forward(q, kd, vd), torch.float16, f"q8_0 G={G} D={D} S={S}")


@pytest.mark.parametrize("G,D", [(3, 128), (7, 64), (12, 128), (16, 64), (20, 64), (32, 128)])
@pytest.mark.parametrize("S", [300, 8192])
def test_q8_0_decode_any_query_group(dev, G, D, S):
    # query groups that are not 1, 2, 4 or 8 heads (groups of up to 8 over the same keys), with a
    # per-head mask so that each group's query, mask and output rows are checked
    B, Hkv = 2, 2
    seed = G * 100 + D + S
    q = randn((B, Hkv * G, 1, D), seed, torch.float16)
    k, v = randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    kb, vb = oracle.q8_0_quantize(k.numpy()), oracle.q8_0_quantize(v.numpy())
    kq = g.QuantizedTensor(torch.from_numpy(kb).to(dev), tuple(k.shape))
    vq = g.QuantizedTensor(torch.from_numpy(vb).to(dev), tuple(v.shape))
    kd = torch.from_numpy(oracle.q8_0_dequantize(kb).reshape(k.shape))
    vd = torch.from_numpy(oracle.q8_0_dequantize(vb).reshape(v.shape))
    assert_close(g.flash_attention(q.to(dev), kq, vq), oracle_forward(q, kd, vd), torch.float16,
                 f"q8_0 G={G} D={D} S={S}")
    per_head = torch.from_numpy(np.random.default_rng(seed).random((B, Hkv * G, 1, S)) < 0.3)
    per_head[:, ::3, :, S // 2:] = False
    per_head[..., 0] = True
    assert_close(g.flash_attention(q.to(dev), kq, vq, per_head.to(dev)), oracle_forward(q, kd, vd, mask=per_head),
                 torch.float16, f"q8_0 per-head mask G={G} D={D} S={S}")


def test_q8_0_decode_masks_and_causal(dev):
    B, H, Hkv, S, D = 3, 8, 2, 600, 128
    q = randn((B, H, 1, D), 21, torch.float16)
    k, v = randn((B, Hkv, S, D), 22), randn((B, Hkv, S, D), 23)
    kq, vq = g.quantize(k.to(dev)), g.quantize(v.to(dev))
    kd, vd = g.dequantize(kq).cpu(), g.dequantize(vq).cpu()
    lens = [600, 3, 257]
    add = torch.zeros(B, 1, 1, S)
    for b, n in enumerate(lens):
        add[b, ..., n:] = float("-inf")
    got = g.flash_attention(q.to(dev), kq, vq, add.to(dev))
    assert_close(got, oracle_forward(q, kd, vd, mask=add), torch.float16, "q8_0 key padding")
    got = g.flash_attention(q.to(dev), kq, vq, (add == 0).to(dev))
    assert_close(got, oracle_forward(q, kd, vd, mask=add), torch.float16, "q8_0 bool")
    got = g.flash_attention(q.to(dev), kq, vq, None, 0.0, True)
    assert_close(got, oracle_forward(q, kd, vd, is_causal=True), torch.float16, "q8_0 causal")


@pytest.mark.parametrize("S", [2, 64, 300])
def test_q8_0_decode_structured_inputs(dev, S):
    """Isolates the phases of the Q8_0 decode kernel: identical V rows make the output that row
    whatever the weights; all-zero K makes the weights uniform (output = mean of V)."""
    B, H, Hkv, D = 1, 4, 1, 128
    q = randn((B, H, 1, D), 31, torch.float16)
    k = randn((B, Hkv, S, D), 32)
    vrow = randn((D,), 33)
    v_same = vrow.expand(B, Hkv, S, D).contiguous()
    kq = g.quantize(k.to(dev))
    vq_same = g.quantize(v_same.to(dev))
    row = g.dequantize(vq_same).cpu()[0, 0, 0]
    got = g.flash_attention(q.to(dev), kq, vq_same).float().cpu()
    assert (got - row.expand(B, H, 1, D)).abs().max().item() < 2e-3, "identical V rows"
    v = randn((B, Hkv, S, D), 34)
    vq = g.quantize(v.to(dev))
    kz = g.quantize(torch.zeros(B, Hkv, S, D, device=dev))
    got = g.flash_attention(q.to(dev), kz, vq).float().cpu()
    mean = g.dequantize(vq).cpu().mean(dim=2, keepdim=True).expand(B, H, 1, D)
    assert (got - mean).abs().max().item() < 2e-3, "uniform weights"


def test_q8_0_decode_lse_exposes_the_scores(dev):
    B, H, Hkv, S, D = 1, 4, 1, 40, 128
    q = randn((B, H, 1, D), 41, torch.float16)
    k, v = randn((B, Hkv, S, D), 42), randn((B, Hkv, S, D), 43)
    kq, vq = g.quantize(k.to(dev)), g.quantize(v.to(dev))
    kd, vd = g.dequantize(kq).cpu(), g.dequantize(vq).cpu()
    out, lse = g.flash_attention_lse(q.to(dev), kq, vq)
    want_o, want_l = oracle_forward(q, kd, vd, return_lse=True)
    assert np.abs(lse.cpu().numpy() - want_l).max() < 1e-3, (lse.cpu().numpy().ravel(), want_l.ravel())
    assert_close(out, want_o, torch.float16, "q8_0 out")


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("L", [2, 130, 512])
@pytest.mark.parametrize("causal", [False, True])
def test_prefill_chunks_over_q8_0_kv_run_on_mfma(dev, qdtype, L, causal):
    # L > 1 over Q8_0 K/V: for float16 queries the blocks are dequantized once to float16 and
    # the MFMA prefill kernel attends; bfloat16 queries take the exact float32 values (generic
    # kernel).  The reference's meaning: csrc/gt_core.cpp:800-808, then
    # csrc/gt_ops_nn.cpp:2423-2525; checked against the oracle on the exact dequantized values
    from gguf_train_amd import _C

    B, H, Hkv, S, D = 2, 8, 2, 640, 128
    seed = L * 7 + (3 if causal else 0)
    q = randn((B, H, L, D), seed, qdtype, 0.5)
    k, v = randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    kb, vb = oracle.q8_0_quantize(k.numpy()), oracle.q8_0_quantize(v.numpy())
    kq = g.QuantizedTensor(torch.from_numpy(kb).to(dev), tuple(k.shape))
    vq = g.QuantizedTensor(torch.from_numpy(vb).to(dev), tuple(v.shape))
    got = g.flash_attention(q.to(dev), kq, vq, None, 0.0, causal)
    launch = _C.last_launch()
    # float16 queries: float16 K/V and the fp16 kernel; float32: the float32 MFMA kernel; bfloat16
    # queries over float32 K/V (mixed dtypes, bfloat16 output): the generic kernel in float32
    want_kernel = {torch.float16: "prefill f16 D=128", torch.float32: "prefill f32 D=128"}.get(qdtype, "generic f32")
    assert launch.startswith("dequantize q8_0 k/v") and want_kernel in launch, launch
    kd = torch.from_numpy(oracle.q8_0_dequantize(kb).reshape(k.shape))
    vd = torch.from_numpy(oracle.q8_0_dequantize(vb).reshape(v.shape))
    assert_close(got, oracle_forward(q, kd, vd, is_causal=causal), qdtype, f"q8_0 prefill L={L} causal={causal}")
