"""Inference kernels for the sequence model around the KLA layers on MI355X.

One-token decode is bound by the number of kernel launches. RMSNorm
(reference ``src/kla/layers/common.py:45-55``) is six torch kernels and the
SwiGLU activation (``:120-123``) two; :func:`rms_norm_hip` and
:func:`swiglu_hip` are one HIP kernel each (``kla_rms_norm_fwd``,
``kla_swiglu_fwd``) with torch's values. They carry no gradient: the modules
use them only when no gradient is required, and keep the torch code otherwise.
"""

from __future__ import annotations

import torch

from kla.ops.hip import _lib


def _code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.KLA_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _lib.KLA_DTYPE_BF16
    raise TypeError(f"expected float32 or bfloat16, got {t.dtype}")


def rms_norm_hip(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """((x * rsqrt(mean(x^2, -1) + eps)) * weight) in x's dtype, over the last dimension."""
    xc = x.contiguous()
    w = weight.float().contiguous()
    y = torch.empty_like(xc)
    dim = xc.shape[-1]
    rows = xc.numel() // dim if dim else 0
    _lib.check("kla_rms_norm_fwd", _lib.lib().kla_rms_norm_fwd(
        _code(xc), xc.data_ptr(), w.data_ptr(), float(eps), y.data_ptr(), rows, dim,
        torch.cuda.current_stream(x.device).cuda_stream))
    return y


def swiglu_hip(h: torch.Tensor) -> torch.Tensor:
    """silu(h[..., :H]) * h[..., H:] for h [..., 2H] with a contiguous last dimension."""
    if h.stride(-1) != 1:
        h = h.contiguous()
    hidden = h.shape[-1] // 2
    lead = h.shape[:-1]
    h2 = h.reshape(-1, h.shape[-1]) if h.dim() != 2 else h
    out = torch.empty(*lead, hidden, dtype=h.dtype, device=h.device)
    _lib.check("kla_swiglu_fwd", _lib.lib().kla_swiglu_fwd(
        _code(h), h2.data_ptr(), h2.stride(0), out.data_ptr(), h2.shape[0], hidden,
        torch.cuda.current_stream(h.device).cuda_stream))
    return out
