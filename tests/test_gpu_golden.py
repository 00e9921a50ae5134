"""The GPU path against the committed golden fixtures (tests/golden/): the fp32 parity
workload (B1 H4 L=S=128 D64 causal, scale 1/8), GQA with bool/additive masks and a fully
masked row, fp16 decode and prefill, the float64 backward, and the Q8_0 codec bit for bit."""

from pathlib import Path

import numpy as np
import pytest
import torch

import gguf_train_amd as g

from _util import assert_close

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def cases():
    return np.load(GOLD / "attention_cases.npz")


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_cfg1(cases, dev):
    rng = np.random.default_rng(int(cases["cfg1_seed"]))
    q, k, v = (_t(rng.standard_normal((1, 4, 128, 64)).astype(np.float32), dev) for _ in range(3))
    out = g.flash_attention(q, k, v, scale=0.125, is_causal=True)
    assert out.dtype == torch.float32
    assert_close(out, cases["cfg1_out"], torch.float32, "cfg1")


@pytest.mark.parametrize("name", ["plain", "causal", "bool", "add_causal"])
def test_gqa_masks(cases, dev, name):
    q, k, v = (_t(cases[f"gqa_{x}"], dev) for x in "qkv")
    mask = None
    if name == "bool":
        mask = _t(cases["gqa_bool_mask"], dev)
    elif name == "add_causal":
        mask = _t(cases["gqa_add_mask"], dev)
    out, lse = g.flash_attention_lse(q, k, v, mask=mask, is_causal=name in ("causal", "add_causal"))
    assert_close(out, cases[f"gqa_{name}_out"], torch.float32, "gqa " + name)
    want = cases[f"gqa_{name}_lse"]
    got = lse.double().cpu().numpy()
    fin = np.isfinite(want)
    assert np.array_equal(np.isinf(got), ~fin)
    assert np.max(np.abs(got[fin] - want[fin])) < 1e-4


def test_decode_fp16(cases, dev):
    q, k, v = (_t(cases[f"dec_{x}"], dev) for x in "qkv")
    out, lse = g.flash_attention_lse(q, k, v)
    assert out.dtype == torch.float16
    assert_close(out, cases["dec_out"], torch.float16, "decode")
    assert np.max(np.abs(lse.double().cpu().numpy() - cases["dec_lse"])) < 2e-3


def test_prefill_fp16(cases, dev):
    q, k, v = (_t(cases[f"f16_{x}"], dev) for x in "qkv")
    out = g.flash_attention(q, k, v, is_causal=True)
    assert_close(out, cases["f16_out"], torch.float16, "fp16 prefill")


def test_backward_fp64(cases, dev):
    q, k, v, do = (_t(cases[f"bwd_{x}"], dev) for x in ("q", "k", "v", "dout"))
    dq, dk, dv = g.flash_attention_backward(do, q, k, v, None, None, None, 0.0, True)
    for got, key in ((dq, "bwd_dq"), (dk, "bwd_dk"), (dv, "bwd_dv")):
        np.testing.assert_allclose(got.double().cpu().numpy(), cases[key], rtol=1e-9, atol=1e-10)


def test_q8_0_codec(dev):
    z = np.load(GOLD / "q8_0_blocks.npz")
    qt = g.quantize(_t(z["x"], dev))
    assert np.array_equal(qt.data.cpu().numpy(), z["blocks"])
    y = g.dequantize(qt, torch.float32)
    assert np.array_equal(y.cpu().numpy().reshape(-1), z["dequantized"])
