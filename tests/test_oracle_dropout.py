"""The oracle's dropout pieces, pinned on the CPU:

* Philox4x32-10 against tests/golden/philox4x32_10.json: rocRAND's engine (an independent
  implementation) on 48 inputs, among them the three known-answer inputs of the Random123
  distribution, whose published words are also written out below;
* the decision layout (which word decides which element) against single-block Philox calls,
  and its statistics: the kept fraction, p = 0 and p = 1, independence of offsets and seeds;
* the dropout composition of scaled_dot_product_attention (gguf_train/nn/functional.py:750-767)
  against torch.autograd through the same composition in float64 with the same keep mask:
  forward and gradients, causal, bool and additive masks, GQA by repeat_interleave, p = 1."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "philox4x32_10.json"

# Random123 kat_vectors, philox4x32 10 rounds: (counter, key) -> words
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


def test_philox_known_answers():
    for ctr, key, words in KAT:
        got = oracle.philox4x32_10(np.array([ctr], np.uint32), np.array(key, np.uint32))
        assert tuple(int(x) for x in got[0]) == words


def test_philox_matches_rocrand():
    vec = json.loads(GOLDEN.read_text())["vectors"]
    ctr = np.array([v["counter"] for v in vec], np.uint32)
    key = np.array([v["key"] for v in vec], np.uint32)
    want = np.array([v["words"] for v in vec], np.uint32)
    assert np.array_equal(oracle.philox4x32_10(ctr, key), want)
    # the golden file holds the known answers too
    for (c, k, w), v in zip(KAT, vec[:3]):
        assert tuple(v["counter"]) == c and tuple(v["key"]) == k and tuple(v["words"]) == w


def test_a_planted_round_change_fails_the_known_answers():
    # one round fewer (a plausible slip) must not reproduce the published words
    def nine_rounds(ctr, key):
        c = [np.uint64(x) for x in ctr]
        k0, k1 = np.uint64(key[0]), np.uint64(key[1])
        m = np.uint64(0xFFFFFFFF)
        for _ in range(9):
            p0, p1 = np.uint64(0xD2511F53) * c[0], np.uint64(0xCD9E8D57) * c[2]
            c = [(p1 >> np.uint64(32)) ^ c[1] ^ k0, p1 & m, (p0 >> np.uint64(32)) ^ c[3] ^ k1, p0 & m]
            k0, k1 = (k0 + np.uint64(0x9E3779B9)) & m, (k1 + np.uint64(0xBB67AE85)) & m
        return tuple(int(x) for x in c)

    assert all(nine_rounds(c, k) != w for c, k, w in KAT)


@pytest.mark.parametrize("S", [1, 3, 4, 7, 64, 101])
def test_decision_layout(S):
    B, H, L, p, seed, offset = 2, 3, 5, 0.375, 0xDEADBEEF12345678, 9
    keep = oracle.dropout_keep(B, H, L, S, p, seed, offset)
    thresh = oracle.dropout_threshold(p)
    nb = (S + 3) // 4
    rng = np.random.default_rng(S)
    for _ in range(40):
        b, h, l, s = (int(rng.integers(n)) for n in (B, H, L, S))
        n = ((b * H + h) * L + l) * nb + s // 4
        w = oracle.philox4x32_10(np.array([[n & 0xFFFFFFFF, n >> 32, offset, 0]], np.uint32),
                                 np.array([seed & 0xFFFFFFFF, seed >> 32], np.uint32))[0, s % 4]
        assert bool(keep[b, h, l, s]) == (int(w) < thresh)


def test_decision_statistics():
    keep = oracle.dropout_keep(4, 8, 64, 1000, 0.3, 99)
    n = keep.size
    frac = keep.mean()
    assert abs(frac - 0.7) < 4 * np.sqrt(0.7 * 0.3 / n)
    assert oracle.dropout_keep(2, 2, 3, 5, 0.0, 1).all()
    assert not oracle.dropout_keep(2, 2, 3, 5, 1.0, 1).any()
    a = oracle.dropout_keep(2, 2, 64, 64, 0.5, 7, 0)
    assert np.array_equal(a, oracle.dropout_keep(2, 2, 64, 64, 0.5, 7, 0))
    for other in (oracle.dropout_keep(2, 2, 64, 64, 0.5, 7, 1), oracle.dropout_keep(2, 2, 64, 64, 0.5, 8, 0)):
        agree = (a == other).mean()
        assert 0.45 < agree < 0.55  # independent draws agree half the time
    assert oracle.dropout_threshold(0.25) == 3 * 2 ** 30 and oracle.dropout_threshold(1.0) == 0


def _torch_composition(q, k, v, keep, p, mask, scale, causal):
    """gguf_train/nn/functional.py:750-767 in torch float64 (the ops the reference composes)."""
    B, H, L, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    ku = k if H == Hkv else k.repeat_interleave(H // Hkv, dim=1)
    vu = v if H == Hkv else v.repeat_interleave(H // Hkv, dim=1)
    scores = q.matmul(ku.transpose(-2, -1)) * scale
    if causal:
        scores = scores + torch.ones(L, S, dtype=torch.float64).triu(diagonal=1) * (-1e9)
    if mask is not None:
        scores = scores.masked_fill(~mask, -1e9) if mask.dtype == torch.bool else scores + mask
    probs = torch.softmax(scores, dim=-1)
    probs = probs * (keep.to(torch.float64) / (1.0 - p)) if p < 1.0 else torch.zeros_like(probs)
    return probs.matmul(vu)


CASES = [
    # B, H, Hkv, L, S, D, causal, mask kind, p
    (1, 2, 2, 7, 9, 8, False, None, 0.2),
    (2, 4, 2, 6, 11, 5, True, None, 0.5),
    (1, 3, 1, 5, 5, 4, True, "bool", 0.1),
    (2, 2, 2, 4, 13, 6, False, "add", 0.7),
    (1, 2, 2, 3, 6, 4, False, "add4", 0.3),
    (1, 2, 1, 4, 4, 3, True, None, 1.0),
]


@pytest.mark.parametrize("B,H,Hkv,L,S,D,causal,mkind,p", CASES)
def test_composition_matches_autograd(B, H, Hkv, L, S, D, causal, mkind, p):
    g = torch.Generator().manual_seed(B * 100 + L * 10 + S)
    q = torch.randn(B, H, L, D, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(B, Hkv, S, D, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(B, Hkv, S, D + 1, generator=g, dtype=torch.float64, requires_grad=True)
    dout = torch.randn(B, H, L, D + 1, generator=g, dtype=torch.float64)
    mask = None
    if mkind == "bool":
        mask = torch.rand(L, S, generator=g) > 0.3
        mask[:, 0] = True  # every row sees a key
    elif mkind == "add":
        mask = torch.randn(B, H, L, S, generator=g, dtype=torch.float64)
    elif mkind == "add4":
        mask = torch.zeros(B, 1, 1, S, dtype=torch.float64)
        mask[..., -2:] = float("-inf")
    keep = torch.from_numpy(oracle.dropout_keep(B, H, L, S, p, seed=5 + S, offset=L))
    scale = float(np.float32(1.0 / np.sqrt(D)))  # the oracle (as the library) takes a float32 scale
    want = _torch_composition(q, k, v, keep, p, mask, scale, causal)
    want.backward(dout)
    out, (dq, dk, dv) = oracle.attention_dropout(q.detach().numpy(), k.detach().numpy(), v.detach().numpy(),
                                                 keep.numpy(), p, mask=None if mask is None else mask.numpy(),
                                                 scale=scale, is_causal=causal, dout=dout.numpy())
    # (p = 1: the reference's dropout returns a fresh zeros tensor, so autograd gives no gradient)
    grads = [np.zeros(t.shape) if t.grad is None else t.grad.numpy() for t in (q, k, v)]
    np.testing.assert_allclose(out, want.detach().numpy(), rtol=1e-12, atol=1e-12)
    for got, ref in zip((dq, dk, dv), grads):
        np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)
    if p == 1.0:
        assert not out.any() and not dq.any() and not dk.any() and not dv.any()
