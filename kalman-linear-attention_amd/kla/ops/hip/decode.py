"""One-token layer kernels for inference decode on MI355X.

:func:`decode_step_hip` is a KLALayer's whole one-token SSM step as one HIP
kernel (``kla_decode_step_fwd``). It covers:

* the discretisation of the static parameters (reference
  ``src/kla/layers/kla_layer.py:164-190``);
* the sensor read-out of the projection (``:194-231``);
* the filter step (``kla_step``, ``src/kla/ops/kla_ops.py:293-331``);
* the lambda skip and the gating of ``forward`` (``:295-349``).

:func:`conv_step_hip` is the one-token depthwise causal conv with its window
update (``src/kla/layers/common.py:70-96``).

Both are forward-only and fp32. By default both return new tensors for the new
state, as the torch path does; with ``in_place=True`` they write it over the
state they were given and return those tensors (a replayed decode graph keeps
its state in fixed buffers that way, with no copies). The layer routes a
one-token step here only when no gradient is required; every other call keeps
the torch code.
"""

from __future__ import annotations

import ctypes
import math

import torch

from kla.ops.hip import _lib

ACTIVATIONS = {"silu": 1, "gelu": 2, "relu": 3}


def _row_stride(t: torch.Tensor) -> int:
    """Row stride of a [B, ...] view whose last dimension is contiguous."""
    if t.dim() < 2 or t.stride(-1) != 1:
        raise ValueError("expected rows with a contiguous last dimension")
    return t.stride(0)


def decode_step_hip(v, log_var, k, q, delta, lambda_log, process_noise, lam, eta, *, residual=None,
                    lambda_skip=None, gate=None, gate_activation="silu", discretization="ou",
                    zero_process_noise=False, qk_norm=True, clip_value=None, obs_var_min=1e-4, obs_var_max=None,
                    decode_from_prior=False, in_place=False):
    """One SSM step of a KLALayer for one token.

    Inputs:

    * v, log_var [B, M] and k, q [B, S] are fp32 row views, e.g. slices of the
      sensor projection.
    * residual and gate are [B, M] row views, or None. lambda_skip is a 0-d or
      [M] fp32 tensor, or None.
    * delta, lambda_log, process_noise are [M, S].
    * lam, eta are [B, M, S].

    Returns (y [B, M], y_var [B, M], lam' [B, M, S], eta' [B, M, S]). y and
    y_var already include the lambda skip and the gate.
    """
    B, M = v.shape
    S = k.shape[1]
    dev = v.device
    from kla.ops.hip.fused import MAX_STATE

    if S > MAX_STATE:
        raise NotImplementedError(f"the hip decode step supports d_state <= {MAX_STATE}")
    if (residual is None) != (lambda_skip is None):
        raise ValueError("residual and lambda_skip come together")
    y, y_var = torch.empty(B, M, device=dev), torch.empty(B, M, device=dev)
    if in_place:
        if not (lam.is_contiguous() and eta.is_contiguous()):
            raise ValueError("in-place decode needs contiguous state tensors")
        lam_out, eta_out = lam, eta
    else:
        lam_out, eta_out = torch.empty_like(lam), torch.empty_like(eta)
    if B * M * S == 0:
        return y, y_var, lam_out, eta_out
    cfg = _lib.DecodeConfig(
        discretization=0 if discretization == "ou" else 1,
        zero_process_noise=int(bool(zero_process_noise)),
        qk_norm=int(bool(qk_norm)),
        has_clip=int(clip_value is not None),
        clip_value=float(clip_value) if clip_value is not None else 0.0,
        obs_var_min=float(obs_var_min),
        obs_var_max=float(obs_var_max) if obs_var_max is not None else math.inf,
        decode_from_prior=int(bool(decode_from_prior)),
        gate_activation=ACTIVATIONS[gate_activation] if gate is not None else 0,
        skip_vector=int(lambda_skip is not None and lambda_skip.dim() == 1),
    )
    pt = _lib.ptr
    ld_kq = _row_stride(k)
    if _row_stride(q) != ld_kq:
        raise ValueError("k and q must share one row stride")
    _lib.check("kla_decode_step_fwd", _lib.lib().kla_decode_step_fwd(
        pt(v), _row_stride(v), pt(log_var), _row_stride(log_var), pt(k), pt(q), ld_kq,
        pt(residual), _row_stride(residual) if residual is not None else 0, pt(lambda_skip),
        pt(gate), _row_stride(gate) if gate is not None else 0,
        pt(delta), pt(lambda_log), pt(process_noise), pt(lam), pt(eta), pt(lam_out), pt(eta_out), pt(y), pt(y_var),
        ctypes.byref(cfg), B, M, S, _lib.stream(dev)))
    return y, y_var, lam_out, eta_out


def conv_step_hip(x, state, weight, bias, activation="silu", in_place=False):
    """One conv token: x [B, D] row view, state [B, D, K-1], weight [D, K], bias [D] or None.
    Returns (y [B, D], new_state [B, D, K-1]); with in_place, new_state is ``state``
    itself, overwritten."""
    B, D = x.shape
    K = weight.shape[-1]
    y = torch.empty(B, D, device=x.device)
    state_out = state if in_place else torch.empty_like(state)
    if B * D == 0:
        return y, state_out
    pt = _lib.ptr
    _lib.check("kla_conv_step_fwd", _lib.lib().kla_conv_step_fwd(
        pt(x), _row_stride(x), pt(state), pt(state_out), pt(weight), pt(bias), ACTIVATIONS.get(activation, 0),
        pt(y), B, D, K, _lib.stream(x.device)))
    return y, state_out
