#!/usr/bin/env python
"""Attention-path benchmark on one MI355X.

A step is one call of the native entry point gt_flash_attention (through the C ABI, on
handles made once over device-resident inputs) over one batch of synthetic data:

  prefill      causal SDPA fp16, B=4 H=32 L=S=2048 D=128, q/k/v ~ 0.5*N(0,1)   (headline)
  decode       GQA decode fp16, B=32 Hq=32 Hkv=8, one query row, KV length 4096, D=128
  decode_q8_0  GQA decode over a GGUF Q8_0 K/V cache, B=16 Hq=32 Hkv=8, KV length 8192, D=128
  train        bf16 forward + backward, B=8 H=16 L=S=1024 D=64, causal + key padding (-inf)
  train_dropout  the same with dropout p = 0.1 on the probabilities (a fresh seed per step; not in
               the default list)
  fp32         fp32 causal forward, B=1 H=4 L=S=128 D=64 (the parity configuration)
  copy         (not in the default list) a plain 1 GiB device copy, the calibration workload
               for the HBM byte counters (FETCH_SIZE / WRITE_SIZE) of the traffic figures

The JSON line's `value` is the headline (prefill) TFLOP/s; the other configurations are
reported under "configs".  Work is counted algorithmically: attention FLOPs = 4*D per
unmasked (query, key) pair and head, backward = 2.5x forward; decode bytes = K + V (read once
per kv head) + Q + O, Q8_0 = 34 bytes per 32 values.

Timing: each configuration runs its step untimed for --settle-ms (the GPU clocks leave their
idle state), then --warmup steps, then exactly --steps steps between HIP events on the stream
the library enqueues on (PyTorch's current stream).

cpu_baseline: the CPU restatement of the reference path (the oracle: the float64
gt_flash_attention loop with OpenMP over (batch, head) like csrc/gt_ops_nn.cpp:2468, closed-form
Q8_0 dequantization, the backward composition in float32 GEMMs) on a bounded sample of every
configuration, with all of this host's threads and with 8, 1 warm-up and the median of 3.
"""

from __future__ import annotations

import argparse
import csv
import ctypes
import json
import math
import os
import re
import subprocess
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP16_TFLOPS = 2516.6  # dense MFMA fp16/bf16, MI355X
PEAK_HBM_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--configs", default="prefill,decode,decode_q8_0,train,fp32")
    p.add_argument("--settle-ms", type=float, default=30.0,
                   help="before its warm-up steps, each configuration runs its own step untimed for this long "
                        "(synchronising every 10 steps), so that the GPU clocks have left their idle state")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--measure-traffic", action="store_true",
                   help="run rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes over the benchmark's kernels (child "
                        "processes), calibrate them against a plain copy and write the summary under profiles/")
    p.add_argument("--measure-mfma", action="store_true",
                   help="run one rocprofv3 --pmc pass of MFMA / VALU / LDS counters over the prefill and training "
                        "configs (child processes) and write the summary under profiles/")
    p.add_argument("--measure-trace", action="store_true",
                   help="run rocprofv3 --kernel-trace --stats over the default benchmark (a child process) and write "
                        "the per-kernel summary with the per-launch rates under profiles/")
    return p.parse_args()


def causal_pairs(L, valid=None):
    """Unmasked (query, key) pairs of a causal L x L block with keys limited to `valid`."""
    v = L if valid is None else valid
    return v * (v + 1) // 2 + (L - v) * v


class Runner:
    """Calls gt_flash_attention (or the backward) on fixed borrowed handles."""

    def __init__(self):
        import torch

        from gguf_train_amd import _C, _bridge

        self.torch, self.C, self.bridge = torch, _C, _bridge
        self.dev = torch.device("cuda:0")
        _bridge.bind_stream(self.dev)

    def handles(self, *ts):
        return [self.bridge.borrow(t) if t is not None else None for t in ts]

    settle_ms = 0.0

    def time_steps(self, step, steps, warmup):
        """Mean over exactly `steps` steps bracketed by synchronisations (events on the current
        stream, which the native calls are bound to), then the median of a second pass timed
        step by step.  Before the `warmup` steps the step runs untimed for `settle_ms` of wall
        time: an idle MI355X drops its clocks within a fraction of a second and needs ~10 ms of
        load to raise them again (measured: 197 us per prefill step after 5 warm-up steps,
        161 us after 50, the same kernel)."""
        torch = self.torch
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < self.settle_ms:
            for _ in range(10):
                step(0)
            torch.cuda.synchronize()
        for _ in range(warmup):
            step(0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for i in range(steps):
            step(i)
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i, (a, b) in enumerate(ev):
            a.record()
            step(i)
            b.record()
        torch.cuda.synchronize()
        per = sorted(a.elapsed_time(b) for a, b in ev)
        return e0.elapsed_time(e1) / steps, wall * 1e3 / steps, per[len(per) // 2]


def forward_inputs(cfg, dev, nbuf=1, keep_draws=False):
    """The synthetic (q, k, v) sets of a forward configuration on device `dev`: N(0,1) (times
    cfg["amp"]) from torch's generator seeded 1234, in the order q, k, v of set 0, then set 1 ...;
    Q8_0 K/V are the library's quantization of the float32 draws (with keep_draws, each set also
    carries those float32 K and V: (q, k, v, k32, v32)).  cfg["dtype"] is a torch dtype."""
    import torch

    B, H, Hkv, L, S, D = cfg["B"], cfg["H"], cfg["Hkv"], cfg["L"], cfg["S"], cfg["D"]
    dt = cfg["dtype"]
    g = torch.Generator(device=dev).manual_seed(1234)
    sets = []
    for _ in range(nbuf):
        q = (torch.randn(B, H, L, D, device=dev, generator=g) * cfg.get("amp", 1.0)).to(dt)
        k = (torch.randn(B, Hkv, S, D, device=dev, generator=g) * cfg.get("amp", 1.0))
        v = (torch.randn(B, Hkv, S, D, device=dev, generator=g) * cfg.get("amp", 1.0))
        k32, v32 = k, v
        if cfg.get("q8_0"):
            from gguf_train_amd import quantize

            k, v = quantize(k), quantize(v)
        else:
            k, v = k.to(dt), v.to(dt)
        sets.append((q, k, v, k32, v32) if keep_draws else (q, k, v))
    return sets


def train_inputs(cfg, dev):
    """(q, k, v, dout, mask, valid_lengths) of the training configuration on device `dev`: q, k,
    v, dout ~ N(0,1) from torch's generator seeded 99 (in that order), rounded to cfg["dtype"];
    key lengths uniform in [512, 1024] from numpy's default_rng(5); mask (B, 1, 1, L) float32,
    0 for valid keys and -inf past each sequence's length."""
    import numpy as np
    import torch

    B, H, L, D = cfg["B"], cfg["H"], cfg["L"], cfg["D"]
    g = torch.Generator(device=dev).manual_seed(99)
    q, k, v, dout = (torch.randn(B, H, L, D, device=dev, generator=g).to(cfg["dtype"]) for _ in range(4))
    lens = np.random.default_rng(5).integers(512, 1025, size=B)
    mask = torch.zeros(B, 1, 1, L, device=dev)
    for b, n in enumerate(lens):
        mask[b, ..., int(n):] = float("-inf")
    return q, k, v, dout, mask, [int(x) for x in lens]


def bench_forward(r: Runner, name, cfg, steps, warmup):
    torch = r.torch
    lib = r.C.lib
    B, H, Hkv, L, S, D = cfg["B"], cfg["H"], cfg["Hkv"], cfg["L"], cfg["S"], cfg["D"]
    dt = cfg["dtype"]
    nbuf = cfg.get("rotate", 1)
    sets = forward_inputs(cfg, r.dev, nbuf)
    hs = [r.handles(*s) for s in sets]
    causal = 1 if cfg.get("causal") else 0

    def step(i):
        hq, hk, hv = hs[i % nbuf]
        p = lib.gt_flash_attention(hq.ptr, hk.ptr, hv.ptr, None, ctypes.c_float(0.0), causal)
        if not p:
            raise RuntimeError(r.C.last_error())
        lib.gt_tensor_free(p)

    ms, wall_ms, med_ms = r.time_steps(step, steps, warmup)
    out = {"ms_per_step": ms, "wall_ms_per_step": wall_ms, "median_ms": med_ms, "launch": r.C.last_launch()}
    es = 2 if dt != torch.float32 else 4
    if "decode" in name:
        if cfg.get("q8_0"):
            kv = 2 * B * Hkv * S * D // 32 * 34
        else:
            kv = 2 * B * Hkv * S * D * es
        nbytes = kv + 2 * B * H * D * es
        out.update(bytes_per_step=nbytes, value=nbytes / (ms * 1e-3) / 1e9, unit="GB/s",
                   frac_of_peak=nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, rotated_buffers=nbuf)
    else:
        pairs = causal_pairs(L) if causal else L * S
        flops = 4 * D * pairs * B * H
        out.update(flop_per_step=flops, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s",
                   frac_of_peak=flops / (ms * 1e-3) / 1e12 / (PEAK_FP16_TFLOPS if dt != torch.float32 else 157.3))
    return out


def bench_train(r: Runner, cfg, steps, warmup):
    lib = r.C.lib
    B, H, L, D = cfg["B"], cfg["H"], cfg["L"], cfg["D"]
    q, k, v, dout, mask, lens = train_inputs(cfg, r.dev)
    hq, hk, hv, hm, hg = r.handles(q, k, v, mask, dout)
    p_drop = float(cfg.get("dropout", 0.0))

    def step(i):
        po, pl, p32 = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        if p_drop:
            rc = lib.gt_flash_attention_dropout(hq.ptr, hk.ptr, hv.ptr, hm.ptr, ctypes.c_float(0.0), 1, p_drop, i + 1, 0,
                                                ctypes.byref(po), ctypes.byref(pl), ctypes.byref(p32))
        else:
            rc = lib.gt_flash_attention_train(hq.ptr, hk.ptr, hv.ptr, hm.ptr, ctypes.c_float(0.0), 1,
                                              ctypes.byref(po), ctypes.byref(pl), ctypes.byref(p32))
        if rc:
            raise RuntimeError(r.C.last_error())
        dq, dk, dv = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        if p_drop:
            rc = lib.gt_flash_attention_dropout_backward(hg.ptr, hq.ptr, hk.ptr, hv.ptr, hm.ptr, p32, pl,
                                                         ctypes.c_float(0.0), 1, p_drop, i + 1, 0, ctypes.byref(dq),
                                                         ctypes.byref(dk), ctypes.byref(dv))
        else:
            rc = lib.gt_flash_attention_backward(hg.ptr, hq.ptr, hk.ptr, hv.ptr, hm.ptr, p32, pl, ctypes.c_float(0.0),
                                                 1, ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv))
        if rc:
            raise RuntimeError(r.C.last_error())
        for p in (po, pl, p32, dq, dk, dv):
            lib.gt_tensor_free(p)

    ms, wall_ms, med_ms = r.time_steps(step, steps, warmup)
    fwd = sum(4 * D * causal_pairs(L, int(n)) * H for n in lens)
    flops = int(fwd * 3.5)
    return {"ms_per_step": ms, "wall_ms_per_step": wall_ms, "median_ms": med_ms, "flop_per_step": flops,
            "forward_flop": fwd, "launch": r.C.last_launch(),
            "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s",
            "frac_of_peak": flops / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, "valid_lengths": lens}


def bench_copy(r: Runner, steps, warmup):
    """torch's device-to-device copy of 1 GiB: reads and writes exactly 2^30 bytes each."""
    torch = r.torch
    n = 1 << 29
    x = torch.ones(n, dtype=torch.float16, device=r.dev)
    y = torch.empty_like(x)

    def step(i):
        y.copy_(x)

    ms, wall_ms, med_ms = r.time_steps(step, steps, warmup)
    nbytes = 2 * x.numel() * x.element_size()
    return {"ms_per_step": ms, "wall_ms_per_step": wall_ms, "median_ms": med_ms, "bytes_per_step": nbytes, "read_bytes": nbytes // 2,
            "write_bytes": nbytes // 2, "value": nbytes / (ms * 1e-3) / 1e9, "unit": "GB/s",
            "frac_of_peak": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS}


def _cpu_threads():
    """(threads the host gives this process, nproc as the OS reports it)."""
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = nproc
    env = os.environ.get("OMP_NUM_THREADS", "")
    return (int(env) if env.isdigit() and int(env) > 0 else avail), nproc


def _median_run(fn, reps=3):
    """One warm-up call, then the median wall time of `reps` calls (seconds)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline():
    """The CPU restatement of the reference path (the oracle: the float64 gt_flash_attention loop
    of csrc/gt_ops_nn.cpp:2423-2525 with OpenMP over (batch, head), the closed-form Q8_0
    dequantization, the backward composition of gguf_train/_functions.py:1933-1965 in float32
    GEMMs) on a bounded sample of each workload, timed with T threads (OMP_NUM_THREADS, else
    every CPU this process may use) and with 8 (the reference's default ggml thread cap,
    csrc/gt_core.cpp:65-67): 1 warm-up and the median of 3 runs each.  Samples keep the
    workload's shapes and per-element cost; each says what it covers."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    import oracle

    T, nproc = _cpu_threads()
    rng = np.random.default_rng(7)
    f16 = lambda shape, sc=1.0: (rng.standard_normal(shape) * sc).astype(np.float16)
    bf16 = lambda shape: oracle.BF16(oracle.f32_to_bf16_bits(rng.standard_normal(shape).astype(np.float32)))
    nh = max(T, 8)  # (batch, head) units of the samples: every thread has one at T threads
    cases = {}

    # fp32 forward, B1 H4 L=S=128 D64 causal: the whole configuration
    q, k, v = (rng.standard_normal((1, 4, 128, 64)).astype(np.float32) for _ in range(3))
    cases["fp32"] = dict(fn=lambda t: oracle.flash_attention(q, k, v, is_causal=True, nthreads=t),
                         work=4 * 64 * causal_pairs(128) * 4, unit="TFLOP/s", sample="the whole configuration")
    # causal fp16 prefill, L=S=2048 D128: nh of the 128 (sequence, head) units, whole
    pq, pk, pv = (f16((1, nh, 2048, 128), 0.5) for _ in range(3))
    cases["prefill"] = dict(fn=lambda t: oracle.flash_attention(pq, pk, pv, is_causal=True, nthreads=t),
                            work=4 * 128 * causal_pairs(2048) * nh, unit="TFLOP/s",
                            sample=f"{nh} of the 128 (sequence, head) units: L=S=2048, D=128, causal, fp16")
    # GQA decode fp16: 4 of the 32 sequences, every head, KV length 4096
    dq_, dk_, dv_ = f16((4, 32, 1, 128)), f16((4, 8, 4096, 128)), f16((4, 8, 4096, 128))
    cases["decode"] = dict(fn=lambda t: oracle.flash_attention(dq_, dk_, dv_, nthreads=t),
                           work=2 * 4 * 8 * 4096 * 128 * 2 + 2 * 4 * 32 * 128 * 2, unit="GB/s",
                           sample="4 of the 32 sequences (Hq=32, Hkv=8, KV length 4096, D=128, fp16)")
    # Q8_0 decode: 2 of the 16 sequences; closed-form dequantization, then the loop
    qq = f16((2, 32, 1, 128))
    kb = oracle.q8_0_quantize(rng.standard_normal((2, 8, 8192, 128)).astype(np.float32))
    vb = oracle.q8_0_quantize(rng.standard_normal((2, 8, 8192, 128)).astype(np.float32))

    def q8_step(t):
        kd = oracle.q8_0_dequantize(kb).reshape(2, 8, 8192, 128)
        vd = oracle.q8_0_dequantize(vb).reshape(2, 8, 8192, 128)
        return oracle.flash_attention(qq, kd, vd, nthreads=t)

    cases["decode_q8_0"] = dict(fn=q8_step, work=2 * (2 * 8 * 8192 * 128 // 32 * 34) + 2 * 2 * 32 * 128 * 2,
                                unit="GB/s", sample="2 of the 16 sequences (Hq=32, Hkv=8, KV length 8192, D=128), "
                                                    "dequantized in closed form then attended")
    # training step bf16 D64: nh heads of one sequence, query rows and keys 0..511 (all valid at the
    # workload's key lengths >= 512), forward loop + float32-GEMM backward composition
    Lt = 512
    tq, tk, tv, tg = (bf16((1, nh, Lt, 64)) for _ in range(4))

    def train_step(t):
        oracle.flash_attention(tq, tk, tv, is_causal=True, nthreads=t)
        with threadpool_limits(limits=t):
            oracle.backward_composition_f32(tg, tq, tk, tv, is_causal=True)

    cases["train"] = dict(fn=train_step, work=int(3.5 * 4 * 64 * causal_pairs(Lt) * nh), unit="TFLOP/s",
                          sample=f"{nh} heads of one sequence, query rows and keys 0..{Lt - 1} (L=S=1024, D=64, "
                                 "causal, bf16); backward in float32 GEMMs (numpy BLAS), not ggml's")
    out = {}
    total = 0.0
    for name, c in cases.items():
        row = {"unit": c["unit"], "sample": c["sample"]}
        for label, t in (("threads_all", T), ("threads_8", 8)):
            sec = _median_run(lambda: c["fn"](t))
            total += sec
            scale = 1e12 if c["unit"] == "TFLOP/s" else 1e9
            row[label] = {"threads": t, "seconds": sec, "value": c["work"] / sec / scale}
        out[name] = row
    head = out["prefill"]
    return {"value": head["threads_all"]["value"], "unit": "TFLOP/s", "cores": T, "kind": "port",
            "sample": head["sample"] + f"; {T} threads (nproc {nproc}), median of 3 after 1 warm-up",
            "nproc": nproc, "configs": out, "timed_seconds": total}


# Dominant kernel of each configuration (substring of its symbol) for the HBM byte counters.
TRAFFIC_KERNELS = {
    "prefill": "prefill_fwd_kernelIDF16_Li128ELb1ELi0E",
    "decode": "decode_stream_kernelIDF16_Li128ELi4ELi0E",
    "decode_q8_0": "decode_q8_lds_kernel<128, 4, 0>",
}
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_prefill_decode.md"


def _pmc_pass(counters, config, steps=3, warmup=1):
    """Average per-dispatch value of each counter for every kernel of `python bench.py --configs
    <config>`, from one rocprofv3 --pmc pass: {counter: {kernel: average}}."""
    with tempfile.TemporaryDirectory() as d:
        cmd = ["rocprofv3", "--pmc", *counters, "-d", d, "-o", "run", "--output-format", "csv", "--",
               sys.executable, str(ROOT / "bench.py"), "--configs", config, "--no-cpu", "--settle-ms", "0",
               "--steps", str(steps),
               "--warmup", str(warmup)]
        n = len(counters)
        print("[pmc] " + " ".join(cmd[:2 + n] + ["-d", "<tmp>"] + cmd[4 + n:]), file=sys.stderr, flush=True)
        subprocess.run(cmd, check=True, timeout=120, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
        files = list(Path(d).rglob("*counter_collection.csv"))
        if not files:
            raise RuntimeError(f"rocprofv3 wrote no counter file for {counters} / {config}")
        vals = {}
        with open(files[0]) as f:
            for row in csv.DictReader(f):
                vals.setdefault(row["Counter_Name"], {}).setdefault(row["Kernel_Name"], []).append(
                    float(row["Counter_Value"]))
    return {c: {k: sum(v) / len(v) for k, v in per.items()} for c, per in vals.items()}


def _pmc_average(counter, config):
    """Average per-dispatch value of `counter` (KiB for FETCH_SIZE / WRITE_SIZE) for every kernel
    of `python bench.py --configs <config>`, from one rocprofv3 --pmc pass."""
    return _pmc_pass([counter], config).get(counter, {})


# MFMA / VALU / LDS counters of the compute-bound kernels (one pass: 7 SQ counters and GRBM's
# clock; MfmaUtil = MFMA-busy SIMD cycles / (GPU-active cycles x SIMDs), MfmaFlops* = MOPS x 512)
MFMA_COUNTERS = ["MfmaUtil", "MfmaFlopsF16", "MfmaFlopsBF16", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_INSTS_LDS",
                 "SQ_BUSY_CYCLES"]
MFMA_KERNELS = {"prefill": ["prefill_fwd_kernel"], "train": ["prefill_fwd_kernel", "bwd_dkdv_kernel", "bwd_dq_kernel"]}
MFMA_FILE = ROOT / "profiles" / "mfma_counters_prefill_train.md"


def measure_mfma():
    """MFMA utilisation and instruction mix of the prefill and training kernels."""
    lines = ["# MFMA utilisation and instruction mix of the prefill and training kernels", "",
             f"Measured on library `{library_hash()[:16]}` (source fingerprint gt_source_hash).", "",
             "Command: `python bench.py --measure-mfma` (per config: `rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) +
             " -d <tmp> -o run --output-format csv -- python bench.py --configs <config> --no-cpu --steps 3 "
             "--warmup 1`). Values are per dispatch, averaged over the run's dispatches of each kernel.", "",
             "- `MfmaUtil`: MFMA-busy SIMD cycles / (GPU-active cycles x SIMDs), in percent.",
             "- MFMA GFLOP executed per dispatch: `MfmaFlopsF16 + MfmaFlopsBF16` (MOPS x 512): every MFMA the kernel "
             "issues, including the masked work of diagonal tiles and the bf16 hi/lo split, so it exceeds the "
             "algorithmic count.",
             "- VALU and LDS instructions per MFMA: `SQ_INSTS_VALU / SQ_INSTS_MFMA`, `SQ_INSTS_LDS / SQ_INSTS_MFMA` "
             "(`SQ_INSTS_VALU` counts the MFMAs too).", "",
             "| config | kernel | MfmaUtil % | MFMA GFLOP executed | MFMA instructions | VALU per MFMA | LDS per MFMA |",
             "|---|---|---|---|---|---|---|"]
    for config, pats in MFMA_KERNELS.items():
        r = _pmc_pass(MFMA_COUNTERS, config)
        seen = set()
        for kernel in sorted(r.get("SQ_INSTS_MFMA", {})):
            if not any(p in kernel for p in pats) or kernel in seen:
                continue
            seen.add(kernel)
            def g(c, default=float("nan")):
                return r.get(c, {}).get(kernel, default)

            mfma = g("SQ_INSTS_MFMA")
            flops = g("MfmaFlopsF16", 0.0) + g("MfmaFlopsBF16", 0.0)
            name = kernel.split("(")[0]
            lines.append(f"| {config} | `{name}` | {g('MfmaUtil'):.1f} | {flops / 1e9:.1f} | {mfma:.4g} | "
                         f"{g('SQ_INSTS_VALU') / mfma:.2f} | {g('SQ_INSTS_LDS') / mfma:.2f} |")
    MFMA_FILE.parent.mkdir(exist_ok=True)
    MFMA_FILE.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def measure_traffic():
    """HBM bytes per launch of the dominant kernels: FETCH_SIZE and WRITE_SIZE (KiB per dispatch),
    each scaled by what the same counter reads for a plain device copy of known size."""
    copy_bytes = 1 << 30  # bench_copy: reads and writes 1 GiB
    cal = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        avg = _pmc_average(counter, "copy")
        kib = max(v for k, v in avg.items() if "copy" in k.lower())
        cal[counter] = {"KiB": kib, "factor": copy_bytes / 1024 / kib}
    rows = {}
    for config, pat in TRAFFIC_KERNELS.items():
        r = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            avg = _pmc_average(counter, config)
            hits = [v for k, v in avg.items() if pat in k]
            if not hits:
                raise RuntimeError(f"no dispatch of {pat} in {config}")
            r[counter] = hits[0]
        r["bytes"] = (r["FETCH_SIZE"] * cal["FETCH_SIZE"]["factor"] + r["WRITE_SIZE"] * cal["WRITE_SIZE"]["factor"]) * 1024
        rows[config] = r
    lines = ["# HBM traffic per launch of the benchmark's dominant kernels", "",
             f"Measured on library `{library_hash()[:16]}` (the source fingerprint gt_source_hash of the "
             "libgt_attn.so that ran; bench.py uses these figures only while the loaded library matches).", "",
             "Command: `python bench.py --measure-traffic` (each pass: `rocprofv3 --pmc <COUNTER> -d <tmp> -o run "
             "--output-format csv -- python bench.py --configs <config> --no-cpu --steps 3 --warmup 1`).", "",
             "Calibration (plain 1 GiB device copy, `--configs copy`):", ""]
    for c, v in cal.items():
        lines.append(f"- {c}: {v['KiB']:.0f} KiB per copy of 1048576 KiB -> factor {v['factor']:.4f}")
    lines += ["", "| config | kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic bytes per launch |", "|---|---|---|---|---|"]
    for config, r in rows.items():
        lines.append(f"| {config} | `{TRAFFIC_KERNELS[config]}` | {r['FETCH_SIZE']:.0f} | {r['WRITE_SIZE']:.0f} | "
                     f"traffic_bytes[{config}] = {r['bytes']:.0f} |")
    TRAFFIC_FILE.parent.mkdir(exist_ok=True)
    TRAFFIC_FILE.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def library_hash() -> str:
    """Source fingerprint of libgt_attn.so (the package's loader refuses a library whose compiled-in
    fingerprint differs from its sources, so the sources' fingerprint is the loaded library's)."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("_gt_srchash", ROOT / "gguf_train_amd" / "_srchash.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.source_hash() or ""


TRACE_FILE = ROOT / "profiles" / "kernel_trace_bench_prefill_decode_q8_train_fp32.md"
# kernel-name substrings of each configuration's kernels (the training step is three launches)
TRACE_KERNELS = {
    "prefill": ["prefill_fwd_kernelIDF16_Li128ELb1ELi0E"],
    "decode": ["decode_stream_kernelIDF16_Li128ELi4ELi0E"],
    "decode_q8_0": ["decode_q8_lds_kernel<128, 4, 0>"],
    "train": ["prefill_fwd_kernelIDF16bLi64ELb1ELi4E", "bwd_dq_kernelIDF16bLi64ELb1ELi4E",
              "bwd_dkdv_kernelIDF16bLi64ELb1ELi4E"],
    "fp32": ["generic_fwd"],
}


def measure_trace():
    """Kernel durations of the default benchmark from rocprofv3 --kernel-trace --stats, and each
    configuration's work divided by its kernels' average duration per launch."""
    with tempfile.TemporaryDirectory() as d:
        cmd = ["rocprofv3", "--kernel-trace", "--stats", "-d", d, "-o", "run", "--output-format", "csv", "--",
               sys.executable, str(ROOT / "bench.py"), "--no-cpu", "--steps", "200", "--warmup", "50"]
        print("[trace] " + " ".join(cmd[:3] + ["-d", "<tmp>"] + cmd[5:]), file=sys.stderr, flush=True)
        proc = subprocess.run(cmd, timeout=300, stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True)
        files = list(Path(d).rglob("*kernel_stats.csv"))
        if not files:
            raise RuntimeError(f"rocprofv3 wrote no kernel statistics (exit {proc.returncode})")
        rows = list(csv.DictReader(open(files[0])))
        line = json.loads(proc.stdout.strip().splitlines()[-1])
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    lines = ["# Kernel trace of the default benchmark", "",
             "Workloads: prefill fp16 B4 H32 L2048 D128 causal; decode fp16 B32 H32/8 S4096 D128; decode Q8_0 B16 "
             "H32/8 S8192 D128; train bf16 B8 H16 L1024 D64 causal + key padding; fp32 B1 H4 L128 D64 causal.", "",
             f"Library `{library_hash()[:16]}` (source fingerprint gt_source_hash).", "",
             "Command: `python bench.py --measure-trace`, which runs `rocprofv3 --kernel-trace --stats -d <tmp> -o run "
             "--output-format csv -- python bench.py --no-cpu --steps 200 --warmup 50` and summarises "
             "`run_kernel_stats.csv` (durations in microseconds; the PyTorch kernels are the benchmark's input "
             "generation).", "",
             "| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|"]
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    avg = {}
    for r in rows:
        name = r["Name"]
        a_us = float(r["AverageNs"]) / 1e3
        avg[name] = a_us
        short = name if len(name) <= 110 else name[:107] + "..."
        lines.append(f"| `{short}` | {r['Calls']} | {a_us:.1f} | {float(r['MinNs']) / 1e3:.1f} | "
                     f"{float(r['MaxNs']) / 1e3:.1f} | {100 * float(r['TotalDurationNs']) / total:.1f} |")
    lines += ["", "Per launch (work as counted by the benchmark, divided by the summed average duration of the "
              "configuration's kernels):", ""]
    for cfg, pats in TRACE_KERNELS.items():
        res = line["configs"].get(cfg)
        if not res:
            continue
        us = sum(v for k, v in avg.items() for p in pats if p in k)
        if us <= 0:
            continue
        if res["unit"] == "GB/s":
            work = res["bytes_per_step"]
            rate = work / (us * 1e-6) / 1e9
            lines.append(f"- {cfg}: {work / 1e6:.1f} MB / {us:.1f} us = {rate:.0f} GB/s "
                         f"({100 * rate / PEAK_HBM_GBS:.1f}% of 8 TB/s); bench.py's HIP-event time "
                         f"{res['ms_per_step'] * 1e3:.1f} us per step")
        else:
            work = res["flop_per_step"]
            rate = work / (us * 1e-6) / 1e12
            peak = 157.3 if cfg == "fp32" else PEAK_FP16_TFLOPS
            lines.append(f"- {cfg}: {work / 1e9:.2f} GFLOP / {us:.1f} us = {rate:.1f} TFLOP/s "
                         f"({100 * rate / peak:.1f}% of {peak}); bench.py's HIP-event time "
                         f"{res['ms_per_step'] * 1e3:.1f} us per step")
    TRACE_FILE.parent.mkdir(exist_ok=True)
    TRACE_FILE.write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def committed_traffic(config, build):
    """HBM bytes per launch of the config's dominant kernel as last measured by --measure-traffic,
    or None when that measurement was made on a library built from other sources."""
    try:
        text = TRAFFIC_FILE.read_text()
    except OSError:
        return None
    lib = re.search(r"library `([0-9a-f]+)`", text)
    if not lib or not build.startswith(lib.group(1)):
        return None
    m = re.search(r"traffic_bytes\[" + re.escape(config) + r"\] = (\d+)", text)
    return int(m.group(1)) if m else None


CONFIGS = {
    "prefill": dict(B=4, H=32, Hkv=32, L=2048, S=2048, D=128, dtype="float16", causal=True, amp=0.5),
    "decode": dict(B=32, H=32, Hkv=8, L=1, S=4096, D=128, dtype="float16", rotate=3),
    "decode_q8_0": dict(B=16, H=32, Hkv=8, L=1, S=8192, D=128, dtype="float16", q8_0=True, rotate=3),
    "train": dict(B=8, H=16, L=1024, D=64, dtype="bfloat16"),
    "train_dropout": dict(B=8, H=16, L=1024, D=64, dtype="bfloat16", dropout=0.1),
    "fp32": dict(B=1, H=4, Hkv=4, L=128, S=128, D=64, dtype="float32", causal=True),
    "copy": dict(dtype="float16"),
}


def main():
    args = parse_args()
    if args.measure_traffic:
        measure_traffic()
        return 0
    if args.measure_mfma:
        measure_mfma()
        return 0
    if args.measure_trace:
        measure_trace()
        return 0
    if args.gpus != 1:
        print(f"bench.py: the benchmark measures one GPU; --gpus {args.gpus} is not supported "
              "(the attention path has no multi-GPU exchange)", file=sys.stderr)
        return 2
    import torch

    r = Runner()
    results = {}
    r.settle_ms = args.settle_ms
    names = [c for c in args.configs.split(",") if c]
    for name in names:
        cfg = dict(CONFIGS[name])
        cfg["dtype"] = getattr(torch, cfg["dtype"])
        if name in ("train", "train_dropout"):
            results[name] = bench_train(r, cfg, args.steps, args.warmup)
        elif name == "copy":
            results[name] = bench_copy(r, args.steps, args.warmup)
        else:
            results[name] = bench_forward(r, name, cfg, args.steps, args.warmup)
        print(f"[bench] {name}: {json.dumps(results[name])}", file=sys.stderr, flush=True)

    head = results.get("prefill") or next(iter(results.values()))
    build = library_hash()
    for name in TRAFFIC_KERNELS:
        if name in results:
            results[name]["traffic_bytes"] = committed_traffic(name, build)
    if head["unit"] == "TFLOP/s":
        roofline = {"bound": "mfma", "achieved": head["value"], "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                    "frac": head["value"] / PEAK_FP16_TFLOPS, "traffic": committed_traffic("prefill", build)}
    else:
        roofline = {"bound": "hbm", "achieved": head["value"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": head["value"] / PEAK_HBM_GBS, "traffic": None}
    line = {
        "metric": "SDPA prefill TFLOP/s + decode KV GB/s on 1 MI355X (% roofline) vs ggml CPU",
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "causal prefill SDPA fp16, B=4 H=32 L=S=2048 D=128",
                   "batch": 4, "heads": 32, "seq_len": 2048, "head_dim": 128, "causal": True},
        "roofline": roofline,
        "configs": results,
        "settle_ms": args.settle_ms,
        "library": build[:16],
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
