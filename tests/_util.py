"""Helpers shared by the GPU parity tests: seeded inputs, oracle calls on the same rounded
values, and the tolerances the attention path is held to:
  fp32 results: max-abs error <= 1e-4 against the float64 oracle;
  fp16/bf16 results: |got - ref| <= 2e-3 * max(1, |ref|) per element (the reference's relative
  idiom, tests/test_views_and_fast_paths.py:73-82) plus the rounding of the result's own
  format, half an ulp: 2^-11 |ref| for float16, 2^-8 |ref| for bfloat16 (the reference's
  output is rounded the same way, csrc/gt_internal.h:263-266).
`ref` is the float64 oracle on the same (already rounded) inputs."""

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


def assert_close(got, want, dtype, what="", out_dtype=None):
    """`dtype` selects the tolerance; the output-rounding allowance is that of `out_dtype`
    (default: `dtype`; pass torch.float32 for float32 results held to the fp16/bf16 bar)."""
    got = got.detach().double().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert not np.isnan(got).any() or np.isnan(want).any(), f"{what}: NaN in result"
    diff = np.abs(got - want)
    if dtype in (torch.float16, torch.bfloat16):
        od = dtype if out_dtype is None else out_dtype
        half_ulp = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}.get(od, 0.0)
        bound = TOL[dtype] * np.maximum(1.0, np.abs(want)) + half_ulp * np.abs(want)
    else:
        bound = np.full(diff.shape, TOL[dtype])
    ratio = diff / bound
    worst = float(np.nanmax(ratio)) if ratio.size else 0.0
    assert worst <= 1.0, f"{what}: error {worst:.3f}x the bound (max abs diff {float(np.nanmax(diff)):.3e})"
    return worst
