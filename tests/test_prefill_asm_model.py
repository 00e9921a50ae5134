"""The generated body of the software-pipelined prefill kernel (csrc/prefill_asm_gen.py) run
for one workgroup in a functional model of the instructions it uses (_gcn_model.py): every path
must finish (no deadlock at a barrier, no read of a register or LDS byte with a load still in
flight, memory accesses in bounds) and give the attention of the reference operator
(csrc/gt_ops_nn.cpp:2423-2525, here in float64 numpy) within the fp16 bar.  Cases: causal query
tiles whose blocks all straddle the diagonal (one tile), pairs of tiles through the generic
loop, non-causal ragged query counts, and scores that move the reference point in most blocks
(the slow path)."""

import importlib.util
from pathlib import Path

import numpy as np
import pytest

import _gcn_model as gm

ROOT = Path(__file__).resolve().parents[1]


def _gen():
    spec = importlib.util.spec_from_file_location("_prefill_asm_gen", ROOT / "gguf_train_amd" / "csrc" / "prefill_asm_gen.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _reference(q, k, v, causal, scale):
    L, S = q.shape[0], k.shape[0]
    s = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    if causal:
        s = np.where(np.arange(S)[None, :] <= np.arange(L)[:, None], s, -np.inf)
    m = s.max(1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(1, keepdims=True)
    return (p @ v.astype(np.float64)) / l, m[:, 0] + np.log(l[:, 0])


def _run(L, S, causal, pair, seed=0, amp=0.5, ramp=None):
    gen = _gen()
    rng = np.random.default_rng(seed)
    D = 128
    q = (rng.standard_normal((L, D)) * amp).astype(np.float16)
    k = rng.standard_normal((S, D)) * amp
    if ramp is not None:
        k = k * np.linspace(ramp[0], ramp[1], S)[:, None]
    k = k.astype(np.float16)
    v = rng.standard_normal((S, D)).astype(np.float16)
    scale = 1.0 / np.sqrt(D)
    mem = gm.Memory()
    addr = {n: mem.alloc(n, a) for n, a in (("q", q), ("k", k), ("v", v), ("o", np.zeros((L, D), np.float16)),
                                            ("lse", np.zeros(L, np.float32)))}
    nq = (L + 127) // 128
    qa, qb = nq - 1 - pair, pair
    c = np.float32(scale) * np.float32(1.4426950408889634)
    ops = {"%[q]": addr["q"], "%[k]": addr["k"], "%[v]": addr["v"], "%[o]": addr["o"], "%[lse]": addr["lse"],
           "%[qsl]": 256, "%[kvrow]": 256, "%[L]": L, "%[ntk]": S // 64, "%[c]": int(np.float32(c).view(np.uint32)),
           "%[qa]": qa, "%[qb]": qb, "%[np]": 1 if qa == qb else 2, "%[lds]": 0}
    ins, labels = gm.parse([l.replace("%=", "0") for l in gen.body(causal)])
    emu = gm.Emu(ins, labels, mem, 2, 65536, ops)
    for w in emu.waves:
        w.v[0] = np.arange(64) + 64 * w.wid
    emu.run()
    o = mem.get("o").view(np.float16).reshape(L, D).astype(np.float64)
    lse = mem.get("lse").view(np.float32)
    want, want_lse = _reference(q, k, v, causal, scale)
    rows = sorted({r for t in {qa, qb} for r in range(t * 128, min(L, t * 128 + 128))})
    err = np.abs(o[rows] - want[rows]) / np.maximum(1.0, np.abs(want[rows]))
    return err.max(), np.abs(lse[rows] - want_lse[rows]).max()


@pytest.mark.parametrize("L,S,causal,pair,kw", [
    (128, 128, True, 0, {}),                             # one tile: the per-wavefront diagonal path
    (512, 512, True, 1, {}),                             # tiles 2 and 1: generic path
    (300, 512, False, 1, {}),                            # ragged query rows, full attention
    (512, 512, True, 0, dict(seed=3, amp=2.0, ramp=(0.2, 3.0))),  # the reference point moves often
])
def test_generated_body_in_the_instruction_model(L, S, causal, pair, kw):
    err, lerr = _run(L, S, causal, pair, **kw)
    assert err < 2e-3 + 2 ** -11, err
    assert lerr < 1e-3, lerr
