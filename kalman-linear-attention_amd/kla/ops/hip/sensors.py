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


# Token counts below which the k, q columns of the sensor projection run as
# kla_rows_linear_qk_fwd: at 2048 tokens (k = 1024, S = 16) its product, norm and
# clip take ~9 us against ~19 us for hipBLASLt's 32-row product alone (plus the
# qk sensor kernel); at 32768 tokens hipBLASLt's product is the faster (23
# against 68 us).
QK_PROJECT_MAX_TOKENS = 8192


def qk_project_hip(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, S: int, *, norm: bool,
                   clip: float | None) -> tuple[torch.Tensor, torch.Tensor]:
    """(k, q) [rows, S] fp32 from fp32 x [rows, K] (last dim contiguous) and the
    sensor projection's last 2 S rows ``weight`` [2 S, K], ``bias`` [2 S]: the k
    and q columns of ``sensor_proj(x)``, each l2-normalised over S when ``norm``
    and clamped to +-clip when given (reference
    ``src/kla/layers/kla_layer.py:205-222``), in one HIP kernel. Inference only
    (no autograd); S a power of two <= 16."""
    if x.dtype != torch.float32 or weight.dtype != torch.float32 or x.dim() != 2 or x.stride(-1) != 1:
        raise TypeError("qk_project_hip: x must be fp32 [rows, K] with a contiguous last dimension, weight fp32")
    if S < 1 or S > 16 or S & (S - 1) or weight.shape[0] != 2 * S or weight.shape[1] != x.shape[1]:
        raise ValueError(f"qk_project_hip: S must be a power of two <= 16 and weight [2 S, K]; got S = {S}, "
                         f"weight {tuple(weight.shape)}, x {tuple(x.shape)}")
    _require_device(x, weight, bias)
    if weight.stride(-1) != 1:
        weight = weight.contiguous()
    if bias is not None:
        bias = bias.float().contiguous()
    rows = x.shape[0]
    k = torch.empty(rows, S, dtype=torch.float32, device=x.device)
    q = torch.empty(rows, S, dtype=torch.float32, device=x.device)
    _lib.check("kla_rows_linear_qk_fwd", _lib.lib().kla_rows_linear_qk_fwd(
        x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), _lib.ptr(bias), k.data_ptr(), q.data_ptr(),
        rows, x.shape[1], S, int(bool(norm)), int(clip is not None), float(clip) if clip is not None else 0.0,
        _lib.stream(x.device)))
    return k, q

