"""Splitting a projection's last dimension, with a HIP backward.

KLALayer splits its two projections along the last dimension (``in_proj`` into
z and the gate, ``sensor_proj`` into v, log sigma^2, k and q; reference
``src/kla/layers/kla_layer.py:206``, ``:313-316``). The pieces are views; in the
backward autograd concatenates their gradients, a full-width copy that torch's
cat kernel runs at well under the HBM rate. :func:`split_last` returns the same
views, and its backward concatenates with ``kla_cat_cols`` (one 16-byte access
per thread, nontemporal stores; a missing gradient becomes zeros).
"""

from __future__ import annotations

import ctypes

import torch

from kla.ops.hip import _lib


def _code(t: torch.Tensor) -> int:
    return _lib.KLA_DTYPE_BF16 if t.dtype == torch.bfloat16 else _lib.KLA_DTYPE_F32


def cat_cols_hip(pieces: list, widths: list[int], like: torch.Tensor) -> torch.Tensor:
    """Concatenate [..., w_i] tensors (None: zeros) along the last dimension into a
    new dense tensor shaped like ``like`` (fp32 or bf16)."""
    lead = like.shape[:-1]
    rows = like.numel() // like.shape[-1] if like.shape[-1] else 0
    out = torch.empty(like.shape, dtype=like.dtype, device=like.device)
    n = len(pieces)
    ptrs = (ctypes.c_void_p * n)()
    lds = (ctypes.c_int64 * n)()
    ws = (ctypes.c_int64 * n)()
    keep = []
    for i, (g, w) in enumerate(zip(pieces, widths)):
        ws[i] = w
        if g is None or w == 0:
            ptrs[i], lds[i] = None, w
            continue
        g2 = g.reshape(rows, w) if g.shape[:-1] == lead else None
        if g2 is None or g2.stride(-1) != 1 or g2.dtype != like.dtype:
            g2 = g.to(like.dtype).reshape(rows, w).contiguous()
        keep.append(g2)
        ptrs[i], lds[i] = g2.data_ptr(), g2.stride(0) if rows > 1 else w
    vp = ctypes.c_void_p
    _lib.check("kla_cat_cols", _lib.lib().kla_cat_cols(
        _code(like), n, ctypes.cast(ptrs, vp), ctypes.cast(lds, vp), ctypes.cast(ws, vp), out.data_ptr(), rows,
        _lib.stream(like.device)))
    return out


class _SplitLast(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, sizes):
        ctx.sizes = list(sizes)
        ctx.like = (x.shape, x.dtype, x.device)
        return tuple(torch.split(x, ctx.sizes, dim=-1))

    @staticmethod
    def backward(ctx, *grads):
        out = cat_cols_hip(list(grads), ctx.sizes, _Like(*ctx.like))
        return out, None


class _Like:
    """Shape, dtype and device of a tensor, for cat_cols_hip's output."""

    def __init__(self, shape, dtype, device):
        self.shape, self.dtype, self.device = shape, dtype, device

    def numel(self):
        n = 1
        for d in self.shape:
            n *= d
        return n


def split_last(x: torch.Tensor, sizes: list[int]) -> tuple[torch.Tensor, ...]:
    """``torch.split(x, sizes, dim=-1)`` for an fp32 / bf16 CUDA tensor whose
    backward concatenates on the MI355X (at most four pieces)."""
    if len(sizes) > 4 or x.dtype not in (torch.float32, torch.bfloat16) or not x.is_cuda:
        return torch.split(x, sizes, dim=-1)
    return _SplitLast.apply(x, sizes)
