"""The k and q sensors of a KLA layer on MI355X, differentiable.

:func:`qk_sensors_hip` turns the k and q columns of the sensor projection into
the scan's fp32 sensors: the l2 normalisation over the S states and the clip of
``KLALayer._project_sensors_raw`` followed by ``.float()`` (reference
``src/kla/layers/kla_layer.py:194-231``), as one HIP kernel each way for both
tensors (``kla_qk_sensors_fwd`` / ``kla_qk_sensors_bwd``), where torch runs
about eight small kernels forward and twenty backward. Values round to the
input dtype after every operation as torch's do (bf16 under autocast), and the
backward follows torch's autograd chain of the same operations.
"""

from __future__ import annotations

import torch

from kla.ops.hip import _lib
from kla.ops.hip.fused import _sensor_rows
from kla.ops.hip.scans import _require_device


def _code(t: torch.Tensor) -> int:
    return _lib.KLA_DTYPE_BF16 if t.dtype == torch.bfloat16 else _lib.KLA_DTYPE_F32


@_lib.hip_op("kla_hip::qk_sensors")
def _qk_op(k: torch.Tensor, q: torch.Tensor, norm: bool, has_clip: bool,
           clip: float) -> tuple[torch.Tensor, torch.Tensor]:
    _require_device(k, q)
    B, L, S = k.shape
    yk = torch.empty(B, L, S, dtype=torch.float32, device=k.device)
    yq = torch.empty_like(yk)
    _lib.check("kla_qk_sensors_fwd", _lib.lib().kla_qk_sensors_fwd(
        _code(k), k.data_ptr(), _sensor_rows(k), q.data_ptr(), _sensor_rows(q), yk.data_ptr(), yq.data_ptr(),
        B * L, S, int(norm), int(has_clip), float(clip), _lib.stream(k.device)))
    return yk, yq


@_qk_op.register_fake
def _(k, q, norm, has_clip, clip):
    return k.new_empty(k.shape, dtype=torch.float32), q.new_empty(q.shape, dtype=torch.float32)


@_lib.hip_op("kla_hip::qk_sensors_backward")
def _qk_bwd_op(k: torch.Tensor, q: torch.Tensor, dyk: torch.Tensor, dyq: torch.Tensor, norm: bool, has_clip: bool,
               clip: float) -> tuple[torch.Tensor, torch.Tensor]:
    _require_device(k, q, dyk, dyq)
    B, L, S = k.shape
    dk = torch.empty(B, L, S, dtype=k.dtype, device=k.device)
    dq = torch.empty_like(dk)
    _lib.check("kla_qk_sensors_bwd", _lib.lib().kla_qk_sensors_bwd(
        _code(k), k.data_ptr(), _sensor_rows(k), q.data_ptr(), _sensor_rows(q), dyk.data_ptr(), dyq.data_ptr(),
        dk.data_ptr(), dq.data_ptr(), B * L, S, int(norm), int(has_clip), float(clip),
        _lib.stream(k.device)))
    return dk, dq


@_qk_bwd_op.register_fake
def _(k, q, dyk, dyq, norm, has_clip, clip):
    return torch.empty_like(k), torch.empty_like(q)


def _setup(ctx, inputs, output):
    k, q, norm, has_clip, clip = inputs
    ctx.cfg = (norm, has_clip, clip)
    ctx.save_for_backward(k, q)


def _backward(ctx, dyk, dyq):
    k, q = ctx.saved_tensors
    dyk = torch.zeros(k.shape, dtype=torch.float32, device=k.device) if dyk is None else dyk.float().contiguous()
    dyq = torch.zeros(q.shape, dtype=torch.float32, device=q.device) if dyq is None else dyq.float().contiguous()
    dk, dq = _lib.call(_qk_bwd_op, k, q, dyk, dyq, *ctx.cfg)
    return dk, dq, None, None, None


_qk_op.register_autograd(_backward, setup_context=_setup)


def qk_sensors_hip(k: torch.Tensor, q: torch.Tensor, *, norm: bool, clip: float | None) -> tuple[torch.Tensor,
                                                                                                 torch.Tensor]:
    """(k, q) [B, L, S] of one dtype (fp32 or bf16; column views of the projection
    are read in place) -> fp32 (clamp(l2_norm(k)), clamp(l2_norm(q))) as torch
    computes them in that dtype, then ``.float()``; S <= 64."""
    if k.dtype != q.dtype or k.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"qk_sensors_hip: k and q must share a float32 or bfloat16 dtype, got {k.dtype}, {q.dtype}")
    if k.shape != q.shape or k.dim() != 3 or k.shape[-1] > 64:
        raise ValueError(f"qk_sensors_hip: expected two [B, L, S <= 64] tensors, got {tuple(k.shape)}, {tuple(q.shape)}")
    if _sensor_rows(k) is None:
        k = k.contiguous()
    if _sensor_rows(q) is None:
        q = q.contiguous()
    return _lib.call(_qk_op, k, q, bool(norm), clip is not None, float(clip) if clip is not None else 0.0)
