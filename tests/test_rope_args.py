"""RoPE argument checks and empty inputs, without a GPU: gt_rope / gt_rope_backward refuse every
argument the reference refuses, with the reference's messages, before any device work
(ported from tests/test_losses_and_rope.py:332-391)."""

import pytest
import torch

from gguf_train_amd import _C, _bridge
from gguf_train_amd.nn import functional as F


def test_positions_too_short_or_not_1d():
    x = torch.ones(1, 3, 4)
    with pytest.raises(RuntimeError, match="a position for each of the 3 sequence elements, got shape \\[2\\]"):
        F.rope(x, torch.arange(2))
    for bad in (torch.arange(6).reshape(2, 3), torch.tensor(0)):
        with pytest.raises(RuntimeError, match="pos must be a 1-D tensor"):
            F.rope(x, bad)
    g, short = _bridge.borrow(torch.ones(1, 3, 4)), _bridge.borrow(torch.arange(2))
    assert not _C.lib.gt_rope_backward(g.ptr, short.ptr, 4, 0, 0, 10000.0, 1.0)
    assert "a position for each of the 3 sequence elements" in _C.last_error()


@pytest.mark.parametrize("n_dims", [3, 8, 0, -2])
def test_bad_n_dims(n_dims):
    with pytest.raises(RuntimeError, match="n_dims must be an even number between 2 and the head dimension 4"):
        F.rope(torch.ones(1, 1, 2, 4), torch.arange(2), n_dims=n_dims)


def test_default_n_dims_is_the_head_dimension():
    with pytest.raises(RuntimeError, match="head dimension 5, got 5"):
        F.rope(torch.ones(1, 1, 2, 5), torch.arange(2))


@pytest.mark.parametrize("mode", [1, 4, 8, 24, 40, -1])
def test_bad_mode(mode):
    with pytest.raises(RuntimeError, match="mode must be 0 \\(normal\\) or 2 \\(NeoX\\)"):
        F.rope(torch.ones(1, 1, 2, 4), torch.arange(2), mode=mode)


@pytest.mark.parametrize("base", [0.0, -1.0, float("nan"), float("inf")])
def test_bad_freq_base(base):
    with pytest.raises(RuntimeError, match="freq_base must be positive"):
        F.rope(torch.ones(1, 1, 2, 4), torch.arange(2), freq_base=base)


def test_bad_shapes_and_dtypes():
    with pytest.raises(RuntimeError, match="expected x of shape"):
        F.rope(torch.ones(2, 4), torch.arange(2))
    with pytest.raises(RuntimeError, match="floating point"):
        F.rope(torch.ones(1, 1, 2, 4, dtype=torch.int64), torch.arange(2))
    g, pos = _bridge.borrow(torch.ones(1, 1, 2, 4)), _bridge.borrow(torch.arange(2))
    for n_dims, mode in ((3, 0), (0, 0), (8, 0), (4, 8)):
        assert not _C.lib.gt_rope_backward(g.ptr, pos.ptr, n_dims, mode, 0, 10000.0, 1.0), (n_dims, mode)


def test_empty_input():
    out = F.rope(torch.ones(1, 2, 0, 4, dtype=torch.float64), torch.arange(0))
    assert tuple(out.shape) == (1, 2, 0, 4) and out.dtype == torch.float64
    assert tuple(F.rope(torch.ones(0, 2, 3, 4), torch.arange(3)).shape) == (0, 2, 3, 4)
