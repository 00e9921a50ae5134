"""gt_flash_attention_noalloc, called through the C ABI, against gt_flash_attention on the same
inputs: two calls in a row (the second one smaller, so it runs over what the first left in the
scratch array), for each kernel the entry point can reach - the split-K decode kernels (fp16,
bf16 groups of 16 heads, head size 256, Q8_0 K/V), the MFMA prefill and the generic kernel -
at the attention bar (fp32: 1e-4 max-abs; fp16/bf16: 2e-3 * max(1, |ref|) plus half an ulp of
the output), and bit for bit where both entry points run the same kernels with the same splits.
Every noalloc call runs with the library's allocation failure switch on (GT_ATTN_FAIL_ALLOC=1:
every device storage allocation fails), so a call that allocated would fail.
Also: the refusals (host tensors, mixed dtypes, q8_0 prefill, a wrong output, partials larger
than the scratch array, a call that would overlap one still running on another stream) leave an
error and touch nothing."""

import contextlib
import ctypes
import os

import pytest
import torch

import gguf_train_amd as g
from gguf_train_amd import _C, _bridge

from _util import assert_close, oracle_forward, randn

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def allocation_fails():
    """While active, every device storage allocation of the library fails (GT_ATTN_FAIL_ALLOC)."""
    old = os.environ.get("GT_ATTN_FAIL_ALLOC")
    os.environ["GT_ATTN_FAIL_ALLOC"] = "1"
    try:
        yield
    finally:
        if old is None:
            del os.environ["GT_ATTN_FAIL_ALLOC"]
        else:
            os.environ["GT_ATTN_FAIL_ALLOC"] = old


def noalloc(q, k, v, mask=None, scale=0.0, causal=False, out=None):
    """gt_flash_attention_noalloc on borrowed handles made beforehand, with allocation failing."""
    _bridge.bind_stream(q.device)
    hs = [_bridge.borrow(t) for t in (q, k, v)]
    hm = _bridge.borrow(mask) if mask is not None else None
    ho = _bridge.borrow(out)
    with allocation_fails():
        rc = _C.lib.gt_flash_attention_noalloc(hs[0].ptr, hs[1].ptr, hs[2].ptr, hm.ptr if hm else None,
                                               ctypes.c_float(scale), 1 if causal else 0, ho.ptr)
    return rc


def test_the_allocation_switch_makes_allocating_calls_fail(dev):
    # the switch the noalloc calls run under: gt_flash_attention, which allocates its output,
    # fails while it is on and works again once it is off
    q, k, v = (randn((1, 2, 1, 128), i, torch.float16).to(dev) for i in range(3))
    with allocation_fails():
        with pytest.raises(Exception):
            g.flash_attention(q, k, v)
    assert g.flash_attention(q, k, v).shape == (1, 2, 1, 128)


def _inputs(dev, dtype, B, H, Hkv, L, S, D, seed, q8=False):
    q = randn((B, H, L, D), seed, torch.float16 if q8 else dtype).to(dev)
    k = randn((B, Hkv, S, D), seed + 1, torch.float32 if q8 else dtype).to(dev)
    v = randn((B, Hkv, S, D), seed + 2, torch.float32 if q8 else dtype).to(dev)
    if q8:
        k, v = g.quantize(k), g.quantize(v)
    return q, k, v


def _check(dev, dtype, shape, causal=False, q8=False, mask_kind=None, exact=True):
    B, H, Hkv, L, S, D = shape
    q, k, v = _inputs(dev, dtype, B, H, Hkv, L, S, D, seed=B * 31 + L + S + D, q8=q8)
    mask = None
    if mask_kind == "bool":
        mask = (torch.rand(B, 1, L, S, device=dev) < 0.7)
        mask[..., 0] = True
    elif mask_kind == "float":
        mask = torch.randn(B, 1, 1, S, device=dev) * 0.5
        mask[..., S // 2:] = float("-inf")
    out = torch.full((B, H, L, D), float("nan"), dtype=q.dtype, device=dev)
    rc = noalloc(q, k, v, mask, 0.0, causal, out)
    assert rc == 0, _C.last_error()
    want = g.flash_attention(q, k, v, mask, 0.0, causal)
    torch.cuda.synchronize()
    od = torch.float32 if q.dtype == torch.float32 else q.dtype
    assert_close(out, want.double().cpu().numpy(), od, f"noalloc vs gt_flash_attention {shape}")
    if exact:
        assert torch.equal(out, want), f"{shape}: not bit-identical"
    return out


CASES = [
    # (dtype, first shape, second (smaller) shape, options)
    (torch.float16, (8, 32, 8, 1, 4096, 128), (2, 8, 2, 1, 1000, 128), {}),                 # GQA decode, split merge
    (torch.bfloat16, (4, 64, 4, 1, 3000, 128), (2, 32, 2, 1, 700, 128), {}),                # 16-head groups
    (torch.float16, (2, 8, 2, 1, 5000, 256), (1, 4, 1, 1, 300, 256), {}),                   # head size 256
    (torch.float16, (4, 32, 8, 1, 8192, 128), (2, 16, 4, 1, 2048, 128), {"q8": True}),      # Q8_0 K/V
    (torch.float16, (2, 8, 2, 1, 2500, 64), (1, 4, 2, 1, 900, 64), {"mask_kind": "bool"}),
    (torch.bfloat16, (2, 8, 2, 1, 2500, 128), (1, 4, 1, 1, 700, 128), {"mask_kind": "float"}),
    (torch.float16, (2, 8, 2, 512, 512, 128), (1, 4, 1, 130, 300, 128), {"causal": True}),  # MFMA prefill
    (torch.float32, (1, 4, 4, 128, 128, 64), (1, 2, 1, 17, 40, 64), {"causal": True}),      # generic kernel
]


@pytest.mark.parametrize("dtype,first,second,opts", CASES)
def test_noalloc_matches_gt_flash_attention_twice(dev, dtype, first, second, opts):
    _check(dev, dtype, first, **opts)
    _check(dev, dtype, second, **opts)


def test_noalloc_decode_against_the_oracle(dev):
    q, k, v = (randn(s, i, torch.float16) for i, s in enumerate([(3, 8, 1, 128), (3, 2, 3000, 128), (3, 2, 3000, 128)]))
    out = torch.empty(3, 8, 1, 128, dtype=torch.float16, device=dev)
    assert noalloc(q.to(dev), k.to(dev), v.to(dev), out=out) == 0, _C.last_error()
    assert_close(out, oracle_forward(q, k, v), torch.float16, "noalloc decode")


def test_noalloc_refusals(dev):
    q, k, v = _inputs(dev, torch.float16, 1, 4, 2, 1, 256, 128, seed=3)
    out = torch.zeros(1, 4, 1, 128, dtype=torch.float16, device=dev)
    cases = [
        ((q.cpu(), k, v, None, out), "must all be on HIP device"),
        ((q, k.to(torch.bfloat16), v, None, out), "must have one dtype"),
        ((q, k, v, torch.zeros(1, 1, 1, 256, dtype=torch.float16, device=dev), out), "the mask must be bool or float32"),
        ((q, k, v, None, torch.zeros(1, 4, 1, 64, dtype=torch.float16, device=dev)), "out must be a dense"),
        ((q, k, v, None, torch.zeros(1, 4, 1, 128, dtype=torch.float32, device=dev)), "out must be a dense"),
    ]
    kq, vq = g.quantize(k.float()), g.quantize(v.float())
    q2 = randn((1, 4, 2, 128), 4, torch.float16).to(dev)
    cases.append(((q2, kq, vq, None, torch.zeros(1, 4, 2, 128, dtype=torch.float16, device=dev)), "q8_0 k/v need"))
    for (qq, kk, vv, m, o), msg in cases:
        before = o.clone()
        assert noalloc(qq, kk, vv, m, 0.0, False, o) != 0
        assert msg in _C.last_error(), (msg, _C.last_error())
        torch.cuda.synchronize()
        assert torch.equal(o, before)


def test_noalloc_refuses_partials_larger_than_the_scratch_array(dev):
    # head size 256 runs one split per 256 keys: 16 rows x 1020 splits x 258 floats > 16 MiB.
    # Never read: the call is refused before any launch, so the inputs stay uninitialised.
    B, H, S, D = 1, 16, 1020 * 256, 256
    q = torch.empty(B, H, 1, D, dtype=torch.float16, device=dev)
    k = torch.empty(B, H, S, D, dtype=torch.float16, device=dev)
    v = torch.empty(B, H, S, D, dtype=torch.float16, device=dev)
    out = torch.zeros(B, H, 1, D, dtype=torch.float16, device=dev)
    assert noalloc(q, k, v, None, 0.0, False, out) != 0
    assert "more than the 16777216-byte scratch array" in _C.last_error()
    torch.cuda.synchronize()
    assert not out.any()
    del k, v
    # the entry point still works after the refusal
    _check(dev, torch.float16, (2, 8, 2, 1, 1000, 128))


def test_noalloc_refuses_an_overlapping_call_on_another_stream(dev):
    # stream s1 is busy (matrix products queued ahead of a split decode that writes the scratch
    # array); the same decode on stream s2 would race on the array: it is refused while s1's
    # call is pending and runs once s1 has finished
    shape = (8, 32, 8, 1, 4096, 128)  # 2 splits: partials in the scratch array
    B, H, Hkv, L, S, D = shape
    q, k, v = _inputs(dev, torch.float16, B, H, Hkv, L, S, D, seed=77)
    out1 = torch.zeros(B, H, L, D, dtype=torch.float16, device=dev)
    out2 = torch.zeros_like(out1)
    a = torch.randn(8192, 8192, device=dev)
    c = torch.empty_like(a)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        for _ in range(20):
            torch.mm(a, a, out=c)
        assert noalloc(q, k, v, out=out1) == 0, _C.last_error()
    with torch.cuda.stream(s2):
        assert noalloc(q, k, v, out=out2) != 0
        assert "may still be running" in _C.last_error(), _C.last_error()
    torch.cuda.synchronize()
    assert not out2.any()
    with torch.cuda.stream(s2):
        assert noalloc(q, k, v, out=out2) == 0, _C.last_error()
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    assert torch.equal(out1, g.flash_attention(q, k, v))
