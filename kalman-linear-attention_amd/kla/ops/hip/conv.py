"""The KLA layer's short depthwise causal conv on MI355X, differentiable.

:func:`causal_conv_hip` replaces the sequence path of ``CausalConv1d.forward``
(reference ``src/kla/layers/common.py:58-96``). The reference transposes x,
concatenates the state in front of it, and runs a library conv followed by the
activation. Here one HIP kernel streams over [B, L, D] with the K taps in
registers, and the hand-written exact adjoint gives dx, d state, d weight and
d bias (``kla_causal_conv_fwd`` / ``kla_causal_conv_bwd``).

x may be a strided view whose channel dimension is contiguous, e.g. one half of
the layer's input projection. fp32 and bf16 are supported; bf16 follows torch
autocast's rounding.
"""

from __future__ import annotations

from typing import Optional

import torch

from kla.ops.hip import _lib
from kla.ops.hip.scans import _require_device

ACTIVATIONS = {"none": 0, "silu": 1, "gelu": 2, "relu": 3}
MAX_KERNEL = 8


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _lib.KLA_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _lib.KLA_DTYPE_BF16
    raise TypeError(f"causal conv supports float32 and bfloat16, got {t.dtype}")


def _strides(x: torch.Tensor) -> tuple[int, int]:
    if x.stride(-1) != 1:
        raise ValueError("x must have a contiguous channel dimension")
    return x.stride(1), x.stride(0)


@_lib.hip_op("kla_hip::causal_conv")
def _conv_op(x: torch.Tensor, state: Optional[torch.Tensor], weight: torch.Tensor, bias: Optional[torch.Tensor],
             activation: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(y [B, L, D], new_state [B, D, K-1]); weight [D, K] fp32."""
    dev = _require_device(x, weight)
    B, L, D = x.shape
    K = weight.shape[1]
    y = torch.empty(B, L, D, dtype=x.dtype, device=dev)
    new_state = torch.empty(B, D, K - 1, dtype=x.dtype, device=dev)
    if B * D == 0:
        return y, new_state
    ld_t, ld_b = _strides(x) if L > 0 else (D, D)
    pt = _lib.ptr
    _lib.check("kla_causal_conv_fwd", _lib.lib().kla_causal_conv_fwd(
        _dtype_code(x), pt(x), ld_t, ld_b, pt(state), pt(weight), pt(bias), activation, pt(y), pt(new_state),
        B, L, D, K, _lib.stream(dev)))
    return y, new_state


@_conv_op.register_fake
def _(x, state, weight, bias, activation):
    B, L, D = x.shape
    return x.new_empty(B, L, D), x.new_empty(B, D, weight.shape[1] - 1)


@_lib.hip_op("kla_hip::causal_conv_backward")
def _conv_bwd_op(dy: torch.Tensor, dstate_out: Optional[torch.Tensor], x: torch.Tensor, state: Optional[torch.Tensor],
                 weight: torch.Tensor, bias: Optional[torch.Tensor], activation: int,
                 need_dstate: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dx, d state (empty unless need_dstate), d weight [D, K] fp32, d bias [D] fp32 (empty without bias))."""
    dev = _require_device(dy, x, weight)
    B, L, D = x.shape
    K = weight.shape[1]
    dx = torch.empty(B, L, D, dtype=x.dtype, device=dev)
    dstate = torch.empty(B, D, K - 1, dtype=x.dtype, device=dev) if need_dstate else x.new_empty(0)
    dweight = torch.empty(D, K, dtype=torch.float32, device=dev)
    dbias = torch.empty(D, dtype=torch.float32, device=dev) if bias is not None else weight.new_empty(0)
    if B * D == 0:
        dweight.zero_()
        dbias.zero_()
        return dx, dstate, dweight, dbias
    ld_t, ld_b = _strides(x) if L > 0 else (D, D)
    need = int(_lib.lib().kla_causal_conv_workspace_bytes(B, L, D, K))
    ws, stream = _lib.scratch(need, dev)
    pt = _lib.ptr
    _lib.check("kla_causal_conv_bwd", _lib.lib().kla_causal_conv_bwd(
        _dtype_code(x), pt(dy), pt(x), ld_t, ld_b, pt(state), pt(weight), pt(bias), activation,
        pt(dstate_out), pt(dx), pt(dstate) if need_dstate else None, pt(dweight),
        pt(dbias) if bias is not None else None, B, L, D, K, ws.data_ptr(), ws.numel(), stream))
    return dx, dstate, dweight, dbias


@_conv_bwd_op.register_fake
def _(dy, dstate_out, x, state, weight, bias, activation, need_dstate):
    B, L, D = x.shape
    K = weight.shape[1]
    return (x.new_empty(B, L, D), x.new_empty(B, D, K - 1) if need_dstate else x.new_empty(0),
            weight.new_empty(D, K, dtype=torch.float32), weight.new_empty(D if bias is not None else 0))


def _setup(ctx, inputs, output):
    x, state, weight, bias, activation = inputs
    ctx.activation = activation
    ctx.has_state = state is not None
    ctx.has_bias = bias is not None
    ctx.save_for_backward(x, state, weight, bias)


def _backward(ctx, dy, dstate_out):
    x, state, weight, bias = ctx.saved_tensors
    need_dstate = ctx.has_state and ctx.needs_input_grad[1]
    dx, dstate, dweight, dbias = _lib.call(_conv_bwd_op,
        dy.contiguous(), dstate_out.contiguous() if dstate_out is not None else None, x,
        state if ctx.has_state else None, weight, bias if ctx.has_bias else None, ctx.activation, need_dstate)
    return (dx, dstate if need_dstate else None, dweight.to(weight.dtype),
            dbias.to(bias.dtype) if ctx.has_bias else None, None)


_conv_op.register_autograd(_backward, setup_context=_setup)


def causal_conv_hip(x: torch.Tensor, state: Optional[torch.Tensor], weight: torch.Tensor,
                    bias: Optional[torch.Tensor], activation: str = "silu"):
    """y, new_state of the causal depthwise conv. x [B, L, D] (fp32 or bf16, channels
    contiguous), state [B, D, K-1] or None (zeros), weight [D, K], bias [D] or None.
    y is dense [B, L, D] in x's dtype; new_state [B, D, K-1] likewise."""
    K = weight.shape[-1]
    if K > MAX_KERNEL:
        raise NotImplementedError(f"the hip causal conv supports kernel_size <= {MAX_KERNEL}")
    if state is not None:
        state = state.to(x.dtype).contiguous()
    w = weight.float()
    b = bias.float() if bias is not None else None
    return _lib.call(_conv_op, x, state, w, b, ACTIVATIONS[activation])
