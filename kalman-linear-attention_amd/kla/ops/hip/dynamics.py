"""A KLA layer's static dynamics on MI355X, differentiable.

:func:`discretize_hip` returns ``(a_bar, p_bar)`` [M, S] from the layer's
``delta``, ``lambda_log`` and ``process_noise`` parameters: the lines of
``KLALayer._continuous_params`` / ``_discretize`` / ``_compute_aq`` (reference
``src/kla/layers/kla_layer.py:164-190``) as one HIP kernel each way
(``kla_discretize_fwd`` / ``kla_discretize_bwd``), where torch runs about
fifteen small elementwise kernels forward and twenty-five backward. The
backward is the chain rule through the same operations (clamp gradients pass
at equality, softplus's is 1 above its threshold 20, expm1's is exp).
"""

from __future__ import annotations

import torch

from kla.ops.hip import _lib
from kla.ops.hip.scans import _require_device


def _stream(t: torch.Tensor) -> int:
    return _lib.stream(t.device)


@_lib.hip_op("kla_hip::discretize")
def _disc_op(delta: torch.Tensor, lambda_log: torch.Tensor, pnoise: torch.Tensor, ou: bool, zero_pn: bool,
             has_clip: bool, clip: float) -> tuple[torch.Tensor, torch.Tensor]:
    _require_device(delta, lambda_log, pnoise)
    a_bar, p_bar = torch.empty_like(delta), torch.empty_like(delta)
    _lib.check("kla_discretize_fwd", _lib.lib().kla_discretize_fwd(
        delta.data_ptr(), lambda_log.data_ptr(), pnoise.data_ptr(), delta.numel(), int(ou), int(zero_pn),
        int(has_clip), float(clip), a_bar.data_ptr(), p_bar.data_ptr(), _stream(delta)))
    return a_bar, p_bar


@_disc_op.register_fake
def _(delta, lambda_log, pnoise, ou, zero_pn, has_clip, clip):
    return torch.empty_like(delta), torch.empty_like(delta)


@_lib.hip_op("kla_hip::discretize_backward")
def _disc_bwd_op(delta: torch.Tensor, lambda_log: torch.Tensor, pnoise: torch.Tensor, g_a: torch.Tensor,
                 g_p: torch.Tensor, ou: bool, zero_pn: bool, has_clip: bool,
                 clip: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    _require_device(delta, lambda_log, pnoise, g_a, g_p)
    d_delta, d_ll, d_pn = torch.empty_like(delta), torch.empty_like(delta), torch.empty_like(delta)
    _lib.check("kla_discretize_bwd", _lib.lib().kla_discretize_bwd(
        delta.data_ptr(), lambda_log.data_ptr(), pnoise.data_ptr(), delta.numel(), int(ou), int(zero_pn),
        int(has_clip), float(clip), g_a.data_ptr(), g_p.data_ptr(), d_delta.data_ptr(), d_ll.data_ptr(),
        d_pn.data_ptr(), _stream(delta)))
    return d_delta, d_ll, d_pn


@_disc_bwd_op.register_fake
def _(delta, lambda_log, pnoise, g_a, g_p, ou, zero_pn, has_clip, clip):
    return torch.empty_like(delta), torch.empty_like(delta), torch.empty_like(delta)


def _setup(ctx, inputs, output):
    delta, lambda_log, pnoise, ou, zero_pn, has_clip, clip = inputs
    ctx.cfg = (ou, zero_pn, has_clip, clip)
    ctx.save_for_backward(delta, lambda_log, pnoise)


def _backward(ctx, g_a, g_p):
    delta, lambda_log, pnoise = ctx.saved_tensors
    g_a = torch.zeros_like(delta) if g_a is None else g_a.float().contiguous()
    g_p = torch.zeros_like(delta) if g_p is None else g_p.float().contiguous()
    d_delta, d_ll, d_pn = _lib.call(_disc_bwd_op, delta, lambda_log, pnoise, g_a, g_p, *ctx.cfg)
    return d_delta, d_ll, d_pn, None, None, None, None


_disc_op.register_autograd(_backward, setup_context=_setup)


def discretize_hip(delta: torch.Tensor, lambda_log: torch.Tensor, process_noise: torch.Tensor, *,
                   discretization: str = "ou", zero_process_noise: bool = False,
                   clip_value: float | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(a_bar, p_bar) [M, S] fp32 from fp32 parameters [M, S] on a ROCm GPU."""
    for name, t in (("delta", delta), ("lambda_log", lambda_log), ("process_noise", process_noise)):
        if t.dtype != torch.float32:
            raise TypeError(f"discretize_hip: {name} must be float32, got {t.dtype}")
        if t.shape != delta.shape:
            raise ValueError(f"discretize_hip: {name} has shape {tuple(t.shape)}, expected {tuple(delta.shape)}")
    if discretization not in ("ou", "zoh"):
        raise ValueError(f"discretize_hip: unknown discretization {discretization!r}")
    return _lib.call(_disc_op, delta.contiguous(), lambda_log.contiguous(), process_noise.contiguous(),
                     discretization == "ou", bool(zero_process_noise), clip_value is not None,
                     float(clip_value) if clip_value is not None else 0.0)
