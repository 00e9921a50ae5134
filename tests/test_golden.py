"""The committed golden fixtures (tests/golden/, written by make_golden.py from the float64
oracle and cross-checked there against PyTorch's CPU SDPA): the oracle must reproduce them
exactly, the fp32 parity workload must regenerate from its seed, and the Q8_0 vectors must
follow ggml's closed form (y = qs * fp16_to_fp32(d), csrc/gt_core.cpp:800-808)."""

from pathlib import Path

import numpy as np
import pytest

import oracle

GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def cases():
    return np.load(GOLD / "attention_cases.npz")


@pytest.fixture(scope="module")
def q8():
    return np.load(GOLD / "q8_0_blocks.npz")


def _cfg1_inputs(seed):
    rng = np.random.default_rng(seed)
    return tuple(rng.standard_normal((1, 4, 128, 64)).astype(np.float32) for _ in range(3))


def test_cfg1_regenerates_and_oracle_matches(cases):
    q, k, v = _cfg1_inputs(int(cases["cfg1_seed"]))
    assert np.array_equal(np.array([x.astype(np.float64).sum() for x in (q, k, v)]), cases["cfg1_checksum"])
    out = oracle.flash_attention(q, k, v, scale=0.125, is_causal=True)
    assert out.dtype == np.float32 and np.array_equal(out, cases["cfg1_out"])


@pytest.mark.parametrize("name,kw", [("plain", {}), ("causal", {"is_causal": True}), ("bool", {"mask": "gqa_bool_mask"}),
                                     ("add_causal", {"mask": "gqa_add_mask", "is_causal": True})])
def test_gqa_mask_cases(cases, name, kw):
    kw = dict(kw)
    if "mask" in kw:
        kw["mask"] = cases[kw["mask"]]
    o, lse = oracle.flash_attention(cases["gqa_q"], cases["gqa_k"], cases["gqa_v"], out_dtype=oracle.F64,
                                    return_lse=True, **kw)
    np.testing.assert_allclose(o, cases[f"gqa_{name}_out"], rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(lse, cases[f"gqa_{name}_lse"], rtol=1e-13, atol=1e-14)


def test_fully_masked_row_is_zero(cases):
    # batch 1, query row 3 has no visible key in the bool mask: the reference writes 0
    assert np.all(cases["gqa_bool_out"][1, :, 3, :] == 0)
    assert np.all(np.isinf(cases["gqa_bool_lse"][1, :, 3]))


def test_decode_and_fp16_cases(cases):
    o, lse = oracle.flash_attention(cases["dec_q"], cases["dec_k"], cases["dec_v"], out_dtype=oracle.F64, return_lse=True)
    np.testing.assert_allclose(o, cases["dec_out"], rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(lse, cases["dec_lse"], rtol=1e-13, atol=1e-14)
    o = oracle.flash_attention(cases["f16_q"], cases["f16_k"], cases["f16_v"], is_causal=True, out_dtype=oracle.F64)
    np.testing.assert_allclose(o, cases["f16_out"], rtol=1e-13, atol=1e-14)


def test_backward_case(cases):
    dq, dk, dv = oracle.flash_attention_backward(cases["bwd_dout"], cases["bwd_q"], cases["bwd_k"], cases["bwd_v"],
                                                 is_causal=True)
    for got, key in ((dq, "bwd_dq"), (dk, "bwd_dk"), (dv, "bwd_dv")):
        np.testing.assert_allclose(got, cases[key], rtol=1e-12, atol=1e-13)


def test_q8_0_vectors(q8):
    x, blocks, deq = q8["x"], q8["blocks"], q8["dequantized"]
    assert np.array_equal(oracle.q8_0_quantize(x), blocks)
    assert np.array_equal(oracle.q8_0_dequantize(blocks), deq)
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    qs = b[:, 2:].copy().view(np.int8).astype(np.float32)
    assert np.array_equal((qs * d).reshape(-1), deq)  # one float32 multiply per value
    # the reference's own check on arange(64)/64 (tests/test_numpy_interop.py:443-454)
    assert np.max(np.abs(deq[:64] - x[:64])) < 0.01
    # ties round half away from zero: 0.5 -> 1, -0.5 -> -1, 126.5 -> 127
    ties = qs[4].astype(np.int64)
    assert list(ties[:9]) == [127, 1, -1, 2, -2, 3, -3, 127, -127]
