"""Pins the oracle's RoPE (oracle_rope, a restatement of gt_rope / gt_rope_backward,
csrc/gt_ops_nn.cpp:2298-2421 -> ggml_rope_ext) before the parity tests trust it.

Each check uses something other than the oracle's own formula:
  * the reference's own known-answer test (tests/test_losses_and_rope.py:254-291): the textbook
    closed form  angle = pos * freq_scale * freq_base^(-2i/n_dims)  evaluated in float64, on the
    same head and positions, to the reference's 4 decimal places;
  * the same closed form at large positions, within the error bound of the float32 angle chain
    ggml uses (theta_{i+1} = fl(theta_i * theta_scale));
  * invariants a wrong index, sign or pairing breaks: position 0 is the identity, the backward
    inverts the forward and is its adjoint, norms are kept, NeoX equals NORMAL under the pair
    permutation, elements from n_dims on are copied, float16/bfloat16 results are the float32
    result rounded once (numpy / torch conversions).
"""

import math

import numpy as np
import pytest
import torch

import oracle


def closed_form(x, positions, n_dims=None, neox=False, freq_base=10000.0, freq_scale=1.0):
    """Textbook RoPE of x (..., S, D) in float64."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    nd = D if n_dims is None else n_dims
    out = x.copy()
    for s, p in enumerate(positions[: x.shape[-2]]):
        for i in range(nd // 2):
            th = p * freq_scale * freq_base ** (-2.0 * i / nd)
            a, b = (i, i + nd // 2) if neox else (2 * i, 2 * i + 1)
            xa, xb = x[..., s, a], x[..., s, b]
            out[..., s, a] = xa * math.cos(th) - xb * math.sin(th)
            out[..., s, b] = xa * math.sin(th) + xb * math.cos(th)
    return out


def head(seq=3, dim=6):
    # the reference test's head (tests/test_losses_and_rope.py:269-270)
    return [[0.5 + 0.25 * s - 0.125 * d + 0.03 * s * d for d in range(dim)] for s in range(seq)]


@pytest.mark.parametrize("kwargs", [{}, {"n_dims": 4}, {"neox": True}, {"n_dims": 2, "neox": True},
                                    {"freq_base": 100.0}, {"freq_scale": 0.5}])
def test_reference_known_answers(kwargs):
    x = np.array([head(), head()], dtype=np.float32)  # (heads, seq, dim)
    pos = [0, 1, 7]
    call = dict(kwargs)
    mode = 2 if call.pop("neox", False) else 0
    got = oracle.rope(x, pos, mode=mode, **call)
    want = closed_form(x, pos, **kwargs)
    assert got.shape == (2, 3, 6) and got.dtype == np.float32
    np.testing.assert_allclose(got, want, atol=5e-5, rtol=0)  # assertAlmostEqual(places=4)
    got4 = oracle.rope(x.reshape(1, 2, 3, 6), pos, mode=mode, **call)
    np.testing.assert_array_equal(got4.reshape(2, 3, 6), got)


@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("n_dims", [128, 64])
def test_large_positions_within_the_float32_angle_chain_bound(mode, n_dims):
    rng = np.random.default_rng(3)
    D, S = 128, 64
    pos = np.concatenate([np.arange(8), rng.integers(0, 200_000, S - 8)]).astype(np.int64)
    x = rng.standard_normal((1, 2, S, D)).astype(np.float32)
    got = oracle.rope(x, pos, n_dims=n_dims, mode=mode)
    want = closed_form(x, pos, n_dims=n_dims, neox=mode == 2)
    # angle_i = p * ts^i by i float32 products, ts = powf(base, -2/n) off by <= 1 ulp plus the
    # rounding of -2/n (times ln(base)): relative angle error <= (i + 1) * u * (2 + ln(1e4) * 2/n) + u
    u = 2.0 ** -24
    half = n_dims // 2
    i = np.arange(half)
    ts = 10000.0 ** (-2.0 / n_dims)
    ang = pos[:, None].astype(np.float64) * ts ** i[None, :]
    err_ang = ang * ((i + 1) * u * (2 + math.log(1e4) * 2 / n_dims) + u)[None, :]
    # per output: |x_pair| * angle error + cos/sin errors + the final rounding
    xa = np.abs(x[0, 0])
    pair_mag = np.zeros((S, half))
    for k in range(half):
        a, b = (k, k + half) if mode == 2 else (2 * k, 2 * k + 1)
        pair_mag[:, k] = np.hypot(xa[:, a], xa[:, b])
    bound = 2 * (pair_mag * err_ang + pair_mag * 4 * u + 1e-7)
    diff = np.abs(got[0, 0].astype(np.float64) - want[0, 0])
    for k in range(half):
        a, b = (k, k + half) if mode == 2 else (2 * k, 2 * k + 1)
        assert (diff[:, a] <= bound[:, k]).all() and (diff[:, b] <= bound[:, k]).all(), k
    # the tail is copied
    np.testing.assert_array_equal(got[..., n_dims:], x[..., n_dims:])


def test_position_zero_is_the_identity():
    x = np.random.default_rng(0).standard_normal((2, 3, 5, 16)).astype(np.float32)
    for mode in (0, 2):
        np.testing.assert_array_equal(oracle.rope(x, np.zeros(5, np.int32), mode=mode), x)


@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("n_dims", [8, 4])
def test_backward_is_the_inverse_and_the_adjoint(mode, n_dims):
    # the reference's own check (tests/test_losses_and_rope.py:305-318), plus the inverse
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 5, 8)).astype(np.float32)
    y = rng.standard_normal((2, 3, 5, 8)).astype(np.float32)
    pos = [4, 0, 9, 2, 2]
    fx = oracle.rope(x, pos, n_dims=n_dims, mode=mode).astype(np.float64)
    by = oracle.rope(y, pos, n_dims=n_dims, mode=mode, backward=True).astype(np.float64)
    assert abs((fx * y).sum() - (x * by).sum()) < 1e-4
    assert abs((fx * fx).sum() - (x.astype(np.float64) ** 2).sum()) < 1e-3
    back = oracle.rope(fx.astype(np.float32), pos, n_dims=n_dims, mode=mode, backward=True)
    np.testing.assert_allclose(back, x, atol=2e-6, rtol=0)


def test_neox_is_normal_under_the_pair_permutation():
    rng = np.random.default_rng(2)
    D, nd = 12, 8
    x = rng.standard_normal((1, 2, 4, D)).astype(np.float32)
    pos = [3, 11, 250, 4096]
    # NeoX pair i = (i, i + nd/2); NORMAL pair i = (2i, 2i + 1): move NeoX's pairs into NORMAL's slots
    perm = np.arange(D)
    perm[0:nd:2] = np.arange(nd // 2)
    perm[1:nd:2] = np.arange(nd // 2) + nd // 2
    normal_of_perm = oracle.rope(np.ascontiguousarray(x[..., perm]), pos, n_dims=nd, mode=0)
    neox = oracle.rope(x, pos, n_dims=nd, mode=2)
    np.testing.assert_array_equal(neox[..., perm], normal_of_perm)


def test_half_and_bfloat16_results_are_the_float32_result_rounded_once():
    rng = np.random.default_rng(4)
    x32 = rng.standard_normal((1, 2, 6, 16)).astype(np.float32)
    pos = [0, 1, 2, 100, 1000, 30000]
    x16 = x32.astype(np.float16)
    got16 = oracle.rope(x16, pos)
    want16 = oracle.rope(x16.astype(np.float32), pos).astype(np.float16)
    np.testing.assert_array_equal(got16, want16)
    xb = torch.from_numpy(x32).bfloat16()
    gotb = oracle.rope(oracle.BF16(xb.view(torch.int16).numpy().view(np.uint16)), pos)
    wantb = torch.from_numpy(oracle.rope(xb.float().numpy(), pos)).bfloat16().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(gotb.bits, wantb)
    # float64 input is computed in float32 (the reference converts it) and returned as float64
    x64 = x32.astype(np.float64) + 1e-12
    np.testing.assert_array_equal(oracle.rope(x64, pos), oracle.rope(x64.astype(np.float32), pos).astype(np.float64))


def test_hand_computed_rotation():
    # a unit vector at index 0 (NORMAL) goes to (cos p, sin p); at index 1 to (-sin p, cos p)
    for p in (1, 7, 123):
        e0 = np.zeros((1, 1, 1, 2), np.float32)
        e0[..., 0] = 1
        e1 = np.zeros((1, 1, 1, 2), np.float32)
        e1[..., 1] = 1
        r0 = oracle.rope(e0, [p])[0, 0, 0]
        r1 = oracle.rope(e1, [p])[0, 0, 0]
        np.testing.assert_allclose(r0, [math.cos(p), math.sin(p)], atol=1e-6)
        np.testing.assert_allclose(r1, [-math.sin(p), math.cos(p)], atol=1e-6)
