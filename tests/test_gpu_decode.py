"""Single-query (decode) attention, the split-K kernel: GQA / MQA group sizes, head sizes, KV lengths
that are not multiples of the chunk, key-padding masks, causal (top-left: key 0 only), and the
invariant that decoding row t equals row t of a causal prefill (tests/test_llama_bridge.py:105-111)."""

import numpy as np
import pytest
import torch

import gguf_train_amd as g

from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G,D", [(1, 64), (2, 128), (4, 128), (8, 128), (4, 256), (8, 64)])
@pytest.mark.parametrize("S", [1, 255, 256, 1000, 4096])
def test_decode_matches_oracle(dev, dtype, G, D, S):
    B, Hkv = 3, 2
    seed = G * 100 + D + S
    q = randn((B, Hkv * G, 1, D), seed, dtype)
    k, v = randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev))
    assert_close(got, oracle_forward(q, k, v), dtype, f"decode G={G} D={D} S={S}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G,D", [(3, 128), (5, 64), (7, 128), (12, 128), (16, 64), (20, 128), (32, 128), (32, 64), (48, 64)])
@pytest.mark.parametrize("S", [300, 4096])
def test_decode_any_query_group(dev, dtype, G, D, S):
    # GQA / MQA groups that are not 1, 2, 4 or 8 heads: the kv head's query heads run in groups
    # of up to 16 over the same keys (16: P.V on MFMA), the last group partial; a per-head mask
    # checks that every group reads its own heads' query and mask rows and writes its own rows
    B, Hkv = 2, 2
    seed = G * 10 + D + S
    q = randn((B, Hkv * G, 1, D), seed, dtype)
    k, v = randn((B, Hkv, S, D), seed + 1, dtype), randn((B, Hkv, S, D), seed + 2, dtype)
    assert_close(g.flash_attention(q.to(dev), k.to(dev), v.to(dev)), oracle_forward(q, k, v), dtype,
                 f"decode G={G} D={D} S={S}")
    per_head = torch.from_numpy(np.random.default_rng(seed).random((B, Hkv * G, 1, S)) < 0.3)
    per_head[:, ::3, :, S // 2:] = False
    per_head[..., 0] = True
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev), per_head.to(dev))
    want_o, want_l = oracle_forward(q, k, v, mask=per_head, return_lse=True)
    assert_close(out, want_o, dtype, f"per-head mask G={G} D={D} S={S}")
    assert np.abs(lse.cpu().numpy() - want_l).max() < 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_with_key_padding_and_bool_masks(dev, dtype):
    B, H, Hkv, S, D = 4, 8, 2, 700, 128
    q = randn((B, H, 1, D), 1, dtype)
    k, v = randn((B, Hkv, S, D), 2, dtype), randn((B, Hkv, S, D), 3, dtype)
    lens = [700, 1, 333, 512]
    add = torch.zeros(B, 1, 1, S)
    allowed = torch.zeros(B, 1, 1, S, dtype=torch.bool)
    for b, n in enumerate(lens):
        add[b, ..., n:] = float("-inf")
        allowed[b, ..., :n] = True
    want = oracle_forward(q, k, v, mask=add)
    assert_close(g.flash_attention(q.to(dev), k.to(dev), v.to(dev), add.to(dev)), want, dtype, "additive")
    assert_close(g.flash_attention(q.to(dev), k.to(dev), v.to(dev), allowed.to(dev)), want, dtype, "bool")
    per_head = torch.rand(B, H, 1, S) < 0.5
    per_head[..., 0] = True
    assert_close(g.flash_attention(q.to(dev), k.to(dev), v.to(dev), per_head.to(dev)),
                 oracle_forward(q, k, v, mask=per_head), dtype, "per-head bool")
    nothing = torch.zeros(B, 1, 1, S, dtype=torch.bool)
    out = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), nothing.to(dev))
    assert torch.equal(out.cpu(), torch.zeros(B, H, 1, D, dtype=dtype))


def test_decode_causal_sees_key_zero_only(dev):
    q = randn((2, 4, 1, 128), 5, torch.float16)
    k, v = randn((2, 2, 300, 128), 6, torch.float16), randn((2, 2, 300, 128), 7, torch.float16)
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None, 0.0, True).cpu()
    want = v[:, :, :1].repeat_interleave(2, dim=1)
    assert torch.equal(got, want)


def test_decode_row_equals_prefill_row(dev):
    B, H, Hkv, T, D = 2, 8, 2, 513, 128
    q = randn((B, H, T, D), 8, torch.float16).to(dev)
    k, v = randn((B, Hkv, T, D), 9, torch.float16).to(dev), randn((B, Hkv, T, D), 10, torch.float16).to(dev)
    full = g.flash_attention(q, k, v, None, 0.0, True)
    for t in (0, 100, 512):
        row = g.flash_attention(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1])
        diff = (row.float() - full[:, :, t:t + 1].float()).abs().max().item()
        assert diff <= 2e-3, (t, diff)


def test_decode_lse(dev):
    q = randn((2, 4, 1, 64), 11, torch.bfloat16)
    k, v = randn((2, 1, 900, 64), 12, torch.bfloat16), randn((2, 1, 900, 64), 13, torch.bfloat16)
    out, lse = g.flash_attention_lse(q.to(dev), k.to(dev), v.to(dev))
    want_o, want_l = oracle_forward(q, k, v, return_lse=True)
    assert_close(out, want_o, torch.bfloat16, "out")
    assert np.abs(lse.cpu().numpy() - want_l).max() < 1e-4


@pytest.mark.parametrize("G", [8, 16, 20])
@pytest.mark.parametrize("S", [64, 300, 4096])
@pytest.mark.parametrize("masked", [False, True])
def test_bf16_decode_with_peaked_logits(dev, G, S, masked):
    # query heads in groups of 8 and 16 do P.V on MFMA; with bfloat16 the probabilities must keep
    # more than bf16's 8 bits there (a few large weights dominate when the logits are peaked:
    # q scaled by 4 gives logits of standard deviation 4)
    B, Hkv, D = 2, 2, 128
    seed = 7 * G + S + (1 if masked else 0)
    q = randn((B, Hkv * G, 1, D), seed, torch.bfloat16, scale=4.0)
    k, v = randn((B, Hkv, S, D), seed + 1, torch.bfloat16), randn((B, Hkv, S, D), seed + 2, torch.bfloat16)
    mask = None
    if masked:
        allowed = torch.from_numpy(np.random.default_rng(seed).random((B, Hkv * G, 1, S)) < 0.5)
        allowed[..., 0] = True
        mask = allowed
    got = g.flash_attention(q.to(dev), k.to(dev), v.to(dev), None if mask is None else mask.to(dev))
    worst = assert_close(got, oracle_forward(q, k, v, mask=mask), torch.bfloat16, f"peaked G={G} S={S} masked={masked}")
    print(f"[decode-peaked] G={G} S={S} masked={masked}: {worst:.3f}", flush=True)


@pytest.mark.parametrize("q8", [False, True])
def test_decode_on_many_streams_gives_the_same_bits(dev, q8):
    # The in-kernel split merge needs a per-stream uncached workspace; at most 16 streams per
    # device get one (uncached memory is never freed), calls on further streams merge their
    # splits with a second launch over pooled memory.  Either way the output is the same bits.
    B, H, Hkv, S, D = 4, 32, 8, 4096, 128
    q = randn((B, H, 1, D), 61, torch.float16).to(dev)
    k, v = randn((B, Hkv, S, D), 62, torch.float32).to(dev), randn((B, Hkv, S, D), 63, torch.float32).to(dev)
    if q8:
        k, v = g.quantize(k), g.quantize(v)
    else:
        k, v = k.half(), v.half()
    want = g.flash_attention(q, k, v)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev) for _ in range(24)]
    outs = []
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            outs.append(g.flash_attention(q, k, v))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, want), f"stream {i}"
