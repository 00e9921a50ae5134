"""The benchmark's own launches against the oracle.

Every configuration bench.py times runs here at its real batch and head counts on the inputs
the benchmark draws (bench.forward_inputs / bench.train_inputs: the same generators, seeds and
distributions), so the grid-dependent paths that only the full shapes reach are compared with
the float64 restatement of gt_flash_attention (csrc/gt_ops_nn.cpp:2423-2525) and of the
backward composition (gguf_train/_functions.py:1933-1965):
  decode fp16 B32 Hq32 Hkv8 S4096 D128     whole output, 2 splits merged in the kernel
  decode Q8_0 B16 Hq32 Hkv8 S8192 D128     whole output on the dequantized values, 4 splits
  prefill fp16 B4 H32 L=S=2048 D128 causal eight (batch, head) units, one in each of the eight
                                           head ranges the kernel deals to one XCD (16 heads
                                           each), the first and the last unit among them
  training bf16 B8 H16 L=S=1024 D64        the float32 output and dQ/dK/dV of six heads from
                                           six sequences, the shortest and the longest key
                                           lengths among them (every head's dK/dV workgroups
                                           run in both of the launch's two rounds: key tiles
                                           0-3, then 4-7)
  fp32 B1 H4 L=S=128 D64 causal            whole output
The launch each call made is read back from gt_last_launch and checked against the split
counts the benchmark's JSON line reports for the same shapes."""

import re

import numpy as np
import pytest
import torch

import bench
import gguf_train_amd as g
import oracle
from gguf_train_amd import _C

from _util import assert_close, oracle_forward, to_oracle

pytestmark = pytest.mark.gpu


def _cfg(name):
    cfg = dict(bench.CONFIGS[name])
    cfg["dtype"] = getattr(torch, cfg["dtype"])
    return cfg


def _splits(launch):
    m = re.search(r"splits=(\d+)", launch)
    assert m, launch
    return int(m.group(1))


def test_decode_workload_whole(dev):
    cfg = _cfg("decode")
    q, k, v = bench.forward_inputs(cfg, dev)[0]
    out = g.flash_attention(q, k, v)
    launch = _C.last_launch()
    print(f"[bench-launch] decode: {launch}", flush=True)
    assert launch.startswith("decode f16 D=128 heads_per_group=4") and "merge=in-kernel" in launch
    assert _splits(launch) == 2 and "units=256" in launch
    assert_close(out, oracle_forward(q, k, v), torch.float16, "decode B32 H32/8 S4096 D128")


def test_q8_0_decode_workload_whole(dev):
    cfg = _cfg("decode_q8_0")
    q, k, v, k32, v32 = bench.forward_inputs(cfg, dev, keep_draws=True)[0]
    out = g.flash_attention(q, k, v)
    launch = _C.last_launch()
    print(f"[bench-launch] decode_q8_0: {launch}", flush=True)
    assert launch.startswith("decode q8_0 D=128 heads_per_group=4") and "merge=in-kernel" in launch
    assert _splits(launch) == 4 and "units=128" in launch
    # the cache bytes are ggml's quantization of the float32 draws, bit for bit
    kb, vb = k.data.cpu().numpy().reshape(-1), v.data.cpu().numpy().reshape(-1)
    assert np.array_equal(kb, oracle.q8_0_quantize(k32.cpu().numpy()))
    assert np.array_equal(vb, oracle.q8_0_quantize(v32.cpu().numpy()))
    shape = (16, 8, 8192, 128)
    kd, vd = oracle.q8_0_dequantize(kb).reshape(shape), oracle.q8_0_dequantize(vb).reshape(shape)
    assert np.array_equal(g.dequantize(k, torch.float32).cpu().numpy(), kd)
    want = oracle.flash_attention(to_oracle(q), kd, vd, out_dtype=oracle.F64)
    assert_close(out, want, torch.float16, "q8_0 decode B16 H32/8 S8192 D128")


def test_prefill_workload_units_in_every_xcd_range(dev):
    cfg = _cfg("prefill")
    q, k, v = bench.forward_inputs(cfg, dev)[0]
    out = g.flash_attention(q, k, v, None, 0.0, True)
    launch = _C.last_launch()
    print(f"[bench-launch] prefill: {launch}", flush=True)
    assert launch == "prefill f16 D=128 B=4 H=32 L=2048 S=2048"
    # (batch*H + head) units: XCD x runs units [16x, 16x + 16) when B*H = 128 splits evenly
    units = [0, 21, 42, 63, 68, 89, 110, 127]
    assert sorted({u // 16 for u in units}) == list(range(8))
    pick = lambda t: torch.stack([t[u // 32, u % 32] for u in units]).unsqueeze(0)
    want = oracle_forward(pick(q), pick(k), pick(v), is_causal=True)
    assert_close(pick(out), want, torch.float16, f"prefill units {units}")


def test_training_workload_heads(dev):
    cfg = _cfg("train")
    q, k, v, dout, mask, lens = bench.train_inputs(cfg, dev)
    out, lse, out32 = g.flash_attention_train(q, k, v, mask, 0.0, True)
    fwd_launch = _C.last_launch()
    dq, dk, dv = g.flash_attention_backward(dout, q, k, v, mask, out32, lse, 0.0, True)
    bwd_launch = _C.last_launch()
    print(f"[bench-launch] train: {fwd_launch} | {bwd_launch}", flush=True)
    assert fwd_launch == "prefill bf16 D=64 B=8 H=16 L=1024 S=1024"
    assert bwd_launch == "backward mfma bf16 D=64"
    order = np.argsort(lens)
    # six sequences (the shortest and the longest key lengths included), one head each
    seqs = [int(order[0]), int(order[-1]), int(order[1]), int(order[-2]), int(order[3]), int(order[4])]
    heads = [(b, (5 * i + 3 * b) % 16) for i, b in enumerate(seqs)]
    pick = lambda t: torch.stack([t[b, h] for b, h in heads]).unsqueeze(0)
    m = torch.stack([mask[b, 0] for b, _ in heads]).unsqueeze(0)  # (1, 6, 1, S): each head's padding
    args = [to_oracle(t) for t in (pick(q), pick(k), pick(v))]
    want32 = oracle.flash_attention(*args, mask=to_oracle(m), is_causal=True, out_dtype=oracle.F64)
    assert_close(pick(out32), want32, torch.bfloat16, f"out32 heads {heads}", out_dtype=torch.float32)
    wq, wk, wv = oracle.flash_attention_backward(to_oracle(pick(dout)), *args, mask=to_oracle(m), is_causal=True)
    for name, got, want in (("dq", pick(dq), wq), ("dk", pick(dk), wk), ("dv", pick(dv), wv)):
        worst = assert_close(got, want, torch.bfloat16, f"{name} heads {heads}", out_dtype=torch.float32)
        print(f"[bench-train] {name}: {worst:.3f} of the bound", flush=True)
    for (b, h), n in zip(heads, (lens[b] for b, _ in heads)):
        assert not dk[b, h, n:].any() and not dv[b, h, n:].any()


def test_fp32_workload_whole(dev):
    cfg = _cfg("fp32")
    q, k, v = bench.forward_inputs(cfg, dev)[0]
    out = g.flash_attention(q, k, v, None, 0.0, True)
    # the float32 MFMA kernel for small grids (4 wavefronts splitting each 32-row group's keys)
    assert _C.last_launch() == "prefill f32 D=64 B=1 H=4 L=128 S=128 split"
    assert_close(out, oracle_forward(q, k, v, is_causal=True), torch.float32, "fp32 B1 H4 L128 D64")
