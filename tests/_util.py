"""Helpers shared by the GPU parity tests: seeded inputs, oracle calls on the same rounded
values, and the tolerances the attention path is held to (fp32: max-abs 1e-4 against the
float64 oracle; fp16/bf16: |got - ref| <= 2e-3 * max(1, |ref|) per element, the reference's
relative idiom from tests/test_views_and_fast_paths.py:73-82)."""

import numpy as np
import torch

import oracle

TOL = {torch.float32: 1e-4, torch.float64: 1e-10, torch.float16: 2e-3, torch.bfloat16: 2e-3}


def randn(shape, seed, dtype=torch.float32, scale=1.0):
    g = np.random.default_rng(seed)
    x = torch.from_numpy((g.standard_normal(shape) * scale).astype(np.float32))
    return x.to(dtype)


def to_oracle(t):
    """A torch tensor (any device) as an oracle input carrying exactly the same values."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return oracle.BF16(t.view(torch.int16).numpy().view(np.uint16))
    if t.dtype == torch.float16:
        return t.numpy()
    return t.numpy()


def oracle_forward(q, k, v, mask=None, scale=-1.0, is_causal=False, return_lse=False):
    return oracle.flash_attention(to_oracle(q), to_oracle(k), to_oracle(v),
                                  mask=None if mask is None else to_oracle(mask), scale=scale,
                                  is_causal=is_causal, out_dtype=oracle.F64, return_lse=return_lse)


def assert_close(got, want, dtype, what=""):
    got = got.detach().double().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if dtype in (torch.float16, torch.bfloat16):
        err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    else:
        err = np.abs(got - want)
    worst = float(np.nanmax(err)) if err.size else 0.0
    assert not np.isnan(got).any() or np.isnan(want).any(), f"{what}: NaN in result"
    assert worst <= TOL[dtype], f"{what}: max error {worst:.3e} > {TOL[dtype]}"
    return worst
