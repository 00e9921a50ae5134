"""Single-query (decode) attention over float32 K/V (decode_f32_kernel: head sizes 64 and 128,
scores on v_mfma_f32_16x16x4_f32, P.V in float32 on the VALU, query heads in groups of up to 8)
against the float64 oracle at the float32 bar (max-abs 1e-4): GQA / MQA group sizes including
partial groups, KV lengths around the 64-key steps and the splits, one key, key-padding, bool and
per-head masks, causal (top-left: key 0 only), the log-sum-exp, the split merge in the kernel
and by a second launch (same bits), and the launch log naming the kernel and its head groups."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C

from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


def _check(dev, q, k, v, mask=None, causal=False, what=""):
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), None if mask is None else mask.to(dev), 0.0,
                                     causal)
    launch = _C.last_launch()
    D, G = q.shape[3], q.shape[1] // k.shape[1]
    tile = 1 if G == 1 else 2 if G == 2 else 4 if G <= 4 else 8
    assert launch.startswith(f"decode f32 D={D} heads_per_group={tile} "), (what, launch)
    want_o, want_l = oracle_forward(q, k, v, mask=mask, is_causal=causal, return_lse=True)
    assert_close(out, want_o, torch.float32, what)
    got_l = lse.cpu().double().numpy()
    fin = np.isfinite(want_l)
    assert np.array_equal(np.isinf(got_l), ~fin), what
    assert np.abs(got_l[fin] - want_l[fin]).max(initial=0.0) < 1e-4, what
    return launch


@pytest.mark.parametrize("G,D,S", [
    (1, 64, 1), (1, 128, 63), (2, 128, 64), (2, 64, 65), (4, 128, 1000), (4, 64, 4097), (8, 128, 4096),
    (8, 64, 300), (3, 128, 700), (5, 64, 129), (12, 128, 2000), (32, 128, 1500), (32, 64, 33)])
def test_float32_decode_matches_oracle(dev, G, D, S):
    B, Hkv = 3, 2
    seed = 13 * G + D + S
    q = randn((B, Hkv * G, 1, D), seed)
    k, v = randn((B, Hkv, S, D), seed + 1), randn((B, Hkv, S, D), seed + 2)
    _check(dev, q, k, v, what=f"decode f32 G={G} D={D} S={S}")


@pytest.mark.parametrize("D", [64, 128])
def test_float32_decode_masks_and_causal(dev, D):
    B, H, Hkv, S = 4, 8, 2, 700
    q = randn((B, H, 1, D), 1)
    k, v = randn((B, Hkv, S, D), 2), randn((B, Hkv, S, D), 3)
    lens = [700, 1, 333, 512]
    add = torch.zeros(B, 1, 1, S)
    allowed = torch.zeros(B, 1, 1, S, dtype=torch.bool)
    for b, n in enumerate(lens):
        add[b, ..., n:] = float("-inf")
        allowed[b, ..., :n] = True
    _check(dev, q, k, v, mask=add, what=f"key padding D={D}")
    _check(dev, q, k, v, mask=allowed, what=f"bool key padding D={D}")
    per_head = torch.from_numpy(np.random.default_rng(D).random((B, H, 1, S)) < 0.3)
    per_head[:, ::3, :, S // 2:] = False
    per_head[..., 0] = True
    _check(dev, q, k, v, mask=per_head, what=f"per-head bool D={D}")
    addh = torch.from_numpy((np.random.default_rng(D + 1).standard_normal((B, H, 1, S)) * 2).astype(np.float32))
    _check(dev, q, k, v, mask=addh, what=f"per-head additive D={D}")
    _check(dev, q, k, v, causal=True, what=f"causal D={D}")  # top-left: key 0 only


def test_float32_decode_split_merges_give_the_same_bits(dev):
    # more than 16 streams: the later ones merge their splits with a second launch over pooled
    # memory instead of in the kernel; the sums run in the same order either way
    B, H, Hkv, S, D = 4, 32, 8, 4096, 128
    q = randn((B, H, 1, D), 61).to(dev)
    k, v = randn((B, Hkv, S, D), 62).to(dev), randn((B, Hkv, S, D), 63).to(dev)
    want = g.flash_attention(q, k, v)
    launch = _C.last_launch()
    assert launch.startswith("decode f32 D=128 heads_per_group=4") and " splits=1 " not in launch, launch
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in range(20)]
    outs = []
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            outs.append(g.flash_attention(q, k, v))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, want), f"stream {i}"
    assert_close(want, oracle_forward(q.cpu(), k.cpu(), v.cpu()), torch.float32, "benchmark-size f32 decode")
