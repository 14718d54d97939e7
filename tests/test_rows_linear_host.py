"""Host-side logic of the decode row kernels (no GPU): the aligned-weight cache
that lets kla_rows_linear_fwd load four k at a time for weights whose rows do
not start 16-byte aligned."""

import gc

import torch

from kla.ops.hip import model_ops


def test_aligned_copy_is_cached_refreshed_and_released():
    w = torch.randn(8, 7)                       # row stride 7: rows not aligned
    a = model_ops._rows_aligned(w)
    assert a.stride(0) % 4 == 0 and a.data_ptr() % 16 == 0 and torch.equal(a, w)
    assert model_ops._rows_aligned(w) is a      # cached
    w.add_(1.0)                                 # in-place update bumps the version
    b = model_ops._rows_aligned(w)
    assert b is not a and torch.equal(b, w)
    key = id(w)
    del w, a, b
    gc.collect()
    assert key not in model_ops._ALIGNED_ROWS   # dropped with the weight


def test_aligned_weight_is_used_as_is():
    w = torch.randn(8, 12)
    assert model_ops._rows_aligned(w) is w
    assert id(w) not in model_ops._ALIGNED_ROWS
