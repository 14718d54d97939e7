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


def test_qk_project_validates_before_any_hip_call():
    """kla_rows_linear_qk_fwd rejects a state width that is not a power of two in
    [1, 16] and a missing q output; an empty problem returns OK without a launch."""
    from kla.ops.hip import _lib

    lib = _lib.lib()
    for S in (0, 3, 12, 32):
        rc = lib.kla_rows_linear_qk_fwd(None, 64, None, 64, None, None, None, 8, 64, S, 1, 0, 0.0, None)
        assert rc == _lib.KLA_ERR_INVALID_ARG and "power of two" in _lib.last_error()
    rc = lib.kla_rows_linear_qk_fwd(None, 64, None, 64, None, None, None, 8, 64, 4, 1, 0, 0.0, None)
    assert rc == _lib.KLA_ERR_INVALID_ARG and "q_out" in _lib.last_error()
    assert lib.kla_rows_linear_qk_fwd(None, 64, None, 64, None, None, None, 0, 64, 4, 1, 0, 0.0, None) == _lib.KLA_OK
