"""Writes the golden fixtures of the attention path (tests/golden/*.npz) from the float64
oracle (oracle/, a restatement of csrc/gt_ops_nn.cpp:2423-2525, gguf_train/_functions.py:
1933-1965 and csrc/gt_core.cpp:800-832).  The reference's own tests hold no numeric vectors
for attention or Q8_0, so these are the build's: the fp32 parity workload (B1 H4 L=S=128 D64,
causal, scale 1/8) in full, tiny GQA / mask / decode / fp16 / backward cases, and Q8_0 block
vectors.  Before writing, every attention case is cross-checked against PyTorch's CPU SDPA in
float64 (rows with at least one visible key), an implementation independent of the oracle.

Run: python tests/golden/make_golden.py   (writes attention_cases.npz and q8_0_blocks.npz)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402

CFG1_SEED = 20240601


def cfg1_inputs():
    """Inputs of the fp32 parity workload, regenerated from the seed (numpy PCG64)."""
    rng = np.random.default_rng(CFG1_SEED)
    return tuple(rng.standard_normal((1, 4, 128, 64)).astype(np.float32) for _ in range(3))


def torch_reference(q, k, v, mask=None, scale=None, is_causal=False):
    """PyTorch CPU SDPA in float64 with GQA expanded and the reference's mask conventions
    (bool True = attend, additive float); rows with no visible key are left as NaN."""
    import torch

    qt, kt, vt = (torch.from_numpy(oracle.to_f64(x)) for x in (q, k, v))
    G = qt.shape[1] // kt.shape[1]
    kt, vt = kt.repeat_interleave(G, 1), vt.repeat_interleave(G, 1)
    L, S = qt.shape[2], kt.shape[2]
    bias = torch.zeros(L, S, dtype=torch.float64)
    if is_causal:
        bias = bias.masked_fill(torch.ones(L, S, dtype=torch.bool).triu(1), float("-inf"))
    if mask is not None:
        m = torch.from_numpy(np.asarray(mask))
        bias = bias + (torch.zeros_like(m, dtype=torch.float64).masked_fill(~m, float("-inf")) if m.dtype == torch.bool
                       else m.double())
    # the ABI's scale is a float: the default 1/sqrt(D) is evaluated in float32
    sc_val = float(np.float32(scale)) if scale is not None else float(np.float32(1.0) / np.sqrt(np.float32(qt.shape[-1])))
    sc = (qt @ kt.transpose(-1, -2)) * sc_val + bias
    return torch.softmax(sc, -1).matmul(vt).numpy()


def check_against_torch(name, out, q, k, v, mask=None, scale=None, is_causal=False):
    ref = torch_reference(q, k, v, mask, scale, is_causal)
    ok = ~np.isnan(ref)
    err = float(np.max(np.abs(np.asarray(out, np.float64)[ok] - ref[ok]))) if ok.any() else 0.0
    assert err < 1e-9, f"{name}: oracle and PyTorch float64 SDPA differ by {err}"
    # rows with nothing to attend to: the reference returns 0 (csrc/gt_ops_nn.cpp:2499-2511)
    assert np.all(np.asarray(out)[~ok] == 0), f"{name}: empty rows must be 0"


def main():
    cases = {}
    # 1. the fp32 parity workload: seed + output (float32, as the reference writes it)
    q, k, v = cfg1_inputs()
    out = oracle.flash_attention(q, k, v, scale=0.125, is_causal=True)
    out64 = oracle.flash_attention(q, k, v, scale=0.125, is_causal=True, out_dtype=oracle.F64)
    check_against_torch("cfg1", out64, q, k, v, scale=0.125, is_causal=True)
    cases.update(cfg1_seed=np.int64(CFG1_SEED), cfg1_checksum=np.array([x.astype(np.float64).sum() for x in (q, k, v)]),
                 cfg1_out=out)

    rng = np.random.default_rng(7)
    # 2. GQA with masks, fp32 inputs stored in full
    q = rng.standard_normal((2, 4, 5, 8)).astype(np.float32)
    k = rng.standard_normal((2, 2, 7, 8)).astype(np.float32)
    v = rng.standard_normal((2, 2, 7, 8)).astype(np.float32)
    bmask = rng.random((2, 1, 5, 7)) < 0.7
    bmask[1, 0, 3, :] = False  # a row with nothing to attend to
    amask = np.where(rng.random((1, 4, 5, 7)) < 0.2, -np.inf, rng.standard_normal((1, 4, 5, 7))).astype(np.float32)
    cases.update(gqa_q=q, gqa_k=k, gqa_v=v, gqa_bool_mask=bmask, gqa_add_mask=amask)
    variants = {"plain": dict(), "causal": dict(is_causal=True), "bool": dict(mask=bmask),
                "add_causal": dict(mask=amask, is_causal=True)}
    for name, kw in variants.items():
        o, lse = oracle.flash_attention(q, k, v, out_dtype=oracle.F64, return_lse=True, **kw)
        check_against_torch("gqa_" + name, o, q, k, v, **kw)
        cases[f"gqa_{name}_out"] = o
        cases[f"gqa_{name}_lse"] = lse

    # 3. GQA decode, fp16 inputs (one query row, odd KV length)
    q = rng.standard_normal((2, 8, 1, 16)).astype(np.float16)
    k = rng.standard_normal((2, 2, 37, 16)).astype(np.float16)
    v = rng.standard_normal((2, 2, 37, 16)).astype(np.float16)
    o, lse = oracle.flash_attention(q, k, v, out_dtype=oracle.F64, return_lse=True)
    check_against_torch("decode", o, q, k, v)
    cases.update(dec_q=q, dec_k=k, dec_v=v, dec_out=o, dec_lse=lse)

    # 4. fp16 causal prefill across tile edges (L = S = 70, D = 64)
    q, k, v = (rng.standard_normal((1, 2, 70, 64)).astype(np.float16) for _ in range(3))
    o = oracle.flash_attention(q, k, v, is_causal=True, out_dtype=oracle.F64)
    check_against_torch("fp16_prefill", o, q, k, v, is_causal=True)
    cases.update(f16_q=q, f16_k=k, f16_v=v, f16_out=o)

    # 5. backward, float64, the reference's gradcheck shape (tests/test_autograd.py:137-140)
    q, k, v, g = (rng.standard_normal((1, 2, 4, 8)) for _ in range(4))
    dq, dk, dv = oracle.flash_attention_backward(g, q, k, v, is_causal=True)
    cases.update(bwd_q=q, bwd_k=k, bwd_v=v, bwd_dout=g, bwd_dq=dq, bwd_dk=dk, bwd_dv=dv)
    np.savez_compressed(HERE / "attention_cases.npz", **cases)

    # Q8_0 blocks: the reference's own input arange(64)/64 (tests/test_numpy_interop.py:443-454),
    # a zero block, a block with a single large value, ties at half steps, and random blocks
    x = [np.arange(64, dtype=np.float32) / 64, np.zeros(32, np.float32)]
    big = np.zeros(32, np.float32)
    big[5] = -3.0e4
    big[6] = 1.0
    x.append(big)
    # amax 127 -> d = 1 exactly, so x * (1/d) = x: ties k + 0.5 round half away from zero
    ties = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 3.5, -3.5, 64.5, -64.5]
                    + [float(j) + 0.5 for j in range(19)], np.float32)
    x.append(ties)
    x.append(rng.standard_normal(32 * 8).astype(np.float32))
    x = np.concatenate(x)
    blocks = oracle.q8_0_quantize(x)
    deq = oracle.q8_0_dequantize(blocks)
    np.savez_compressed(HERE / "q8_0_blocks.npz", x=x, blocks=blocks, dequantized=deq)
    print("wrote", HERE / "attention_cases.npz", "and", HERE / "q8_0_blocks.npz")


if __name__ == "__main__":
    main()
