"""The software-pipelined fp16 head-size-128 prefill kernel (attn_prefill_asm.hip, body from
prefill_asm_gen.py) against the float64 oracle: causal tiles of every size class (one query
tile pair whose blocks all straddle the diagonal, the generic loop with and without full
iterations, pairs of unequal tiles), non-causal shapes with ragged query counts, GQA, strided
query views, explicit scales, the log-sum-exp, and score distributions that make the
reference point move in later key blocks (the kernel's slow path); also the same calls on the
HIP prefill kernel for comparison.  The kernel cannot be selected at present (asm_enabled() is
false); these tests stay, skipped, for when its first GPU run's cause is known."""

import os

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C, _ops

from _util import assert_close, oracle_forward, randn

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="the pipelined prefill kernel is switched off: its first GPU run (causal L=S=128) "
                            "did not finish and the cause is not known; it must not run on the GPU until it is"),
]


def _run(q, k, v, causal, scale=0.0):
    out, lse = _ops.flash_attention_lse(q, k, v, None, scale, causal)
    return out, lse, _C.last_launch()


CAUSAL = [  # (B, H, Hkv, L)
    (1, 2, 2, 128),    # one query tile: every block on the diagonal
    (2, 4, 2, 256),    # two tiles: the generic path, no loop iteration
    (1, 2, 1, 384),    # three tiles, the middle one alone in its workgroup
    (1, 3, 3, 640),    # loop with one full iteration
    (1, 1, 1, 1024),   # several iterations
    (1, 2, 2, 1152),   # odd tile count
]


@pytest.mark.parametrize("B,H,Hkv,L", CAUSAL)
def test_causal_against_the_oracle(dev, B, H, Hkv, L):
    seed = L + 7 * H
    q = randn((B, H, L, 128), seed, torch.float16, 0.5)
    k = randn((B, Hkv, L, 128), seed + 1, torch.float16, 0.5)
    v = randn((B, Hkv, L, 128), seed + 2, torch.float16)
    out, lse, launch = _run(q.to(dev), k.to(dev), v.to(dev), True)
    print(f"[pipelined] causal B{B} H{H}/{Hkv} L{L}: {launch}", flush=True)
    assert launch.startswith("prefill pipelined f16 D=128")
    want, want_lse = oracle_forward(q, k, v, is_causal=True, return_lse=True)
    assert_close(out, want, torch.float16, f"causal L={L}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, rtol=1e-4, atol=1e-4)


NONCAUSAL = [  # (B, H, Hkv, L, S)
    (1, 2, 2, 2, 256),
    (2, 2, 1, 100, 384),
    (1, 4, 2, 129, 256),
    (1, 2, 2, 256, 512),
    (1, 1, 1, 300, 1024),
]


@pytest.mark.parametrize("B,H,Hkv,L,S", NONCAUSAL)
def test_full_attention_against_the_oracle(dev, B, H, Hkv, L, S):
    seed = L * 3 + S
    q = randn((B, H, L, 128), seed, torch.float16)
    k = randn((B, Hkv, S, 128), seed + 1, torch.float16)
    v = randn((B, Hkv, S, 128), seed + 2, torch.float16)
    out, lse, launch = _run(q.to(dev), k.to(dev), v.to(dev), False)
    print(f"[pipelined] full B{B} H{H}/{Hkv} L{L} S{S}: {launch}", flush=True)
    assert launch.startswith("prefill pipelined f16 D=128")
    want, want_lse = oracle_forward(q, k, v, return_lse=True)
    assert_close(out, want, torch.float16, f"L={L} S={S}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("causal", [True, False])
def test_reference_point_moves_in_later_blocks(dev, causal):
    # keys whose scores grow along the sequence (a ramp on K) and large scores: most later
    # blocks push the row max more than 2^8 above the reference point, so the slow path runs
    # on many blocks and rescales O and the row sums
    B, H, L = 1, 2, 512
    q = randn((B, H, L, 128), 31, torch.float16, 2.0)
    ramp = torch.linspace(0.2, 3.0, L).reshape(1, 1, L, 1)
    k = (randn((B, H, L, 128), 32, torch.float32, 2.0) * ramp).to(torch.float16)
    v = randn((B, H, L, 128), 33, torch.float16)
    out, lse, launch = _run(q.to(dev), k.to(dev), v.to(dev), causal)
    assert launch.startswith("prefill pipelined")
    want, want_lse = oracle_forward(q, k, v, is_causal=causal, return_lse=True)
    assert_close(out, want, torch.float16, f"ramp causal={causal}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, rtol=1e-4, atol=1e-3)


def test_strided_queries_and_explicit_scale(dev):
    # q as a (B, L, H, D) buffer viewed (B, H, L, D); scale 0.05
    B, H, L = 2, 4, 256
    qb = randn((B, L, H, 128), 41, torch.float16)
    q = qb.transpose(1, 2)
    k = randn((B, H, L, 128), 42, torch.float16)
    v = randn((B, H, L, 128), 43, torch.float16)
    out, _, launch = _run(q.to(dev), k.to(dev), v.to(dev), True, 0.05)
    assert launch.startswith("prefill pipelined")
    assert_close(out, oracle_forward(q.contiguous(), k, v, scale=0.05, is_causal=True), torch.float16, "strided q")


def test_same_result_as_the_hip_kernel(dev, monkeypatch):
    B, H, L = 2, 8, 768
    q, k, v = (randn((B, H, L, 128), 50 + i, torch.float16, 0.5).to(dev) for i in range(3))
    for causal in (True, False):
        a, _, la = _run(q, k, v, causal)
        monkeypatch.setenv("GT_ATTN_PREFILL_ASM", "0")
        b, _, lb = _run(q, k, v, causal)
        monkeypatch.delenv("GT_ATTN_PREFILL_ASM")
        assert la.startswith("prefill pipelined") and lb.startswith("prefill f16")
        diff = (a.float() - b.float()).abs().max().item()
        assert diff < 2e-3, (causal, diff)


def test_repeated_calls_are_deterministic(dev):
    B, H, L = 4, 32, 2048
    q, k, v = (randn((B, H, L, 128), 60 + i, torch.float16, 0.5).to(dev) for i in range(3))
    first = g.flash_attention(q, k, v, None, 0.0, True)
    for _ in range(3):
        assert torch.equal(g.flash_attention(q, k, v, None, 0.0, True), first)
