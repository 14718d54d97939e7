"""The KLALayer output tail after the scan on MI355X, differentiable.

:func:`gate_skip_hip` computes ``(y + lambda_skip * residual) * act(gate)``,
the lines of ``KLALayer.forward`` between the scan and the output projection
(reference ``src/kla/layers/kla_layer.py:333-337``), as one HIP kernel each way
(``kla_gate_skip_fwd`` / ``kla_gate_skip_bwd``) instead of torch's chain of
elementwise passes and their autograd backward. Values and gradients follow
torch's type promotion and autograd roundings for bf16 residual and gate
tensors (see ``csrc/gate_skip.hpp``); d lambda is summed in a fixed order.
"""

from __future__ import annotations

from typing import Optional

import torch

from kla.ops.hip import _lib
from kla.ops.hip.fused import _sensor_rows
from kla.ops.hip.scans import _require_device

ACTIVATIONS = {"none": 0, "silu": 1, "gelu": 2, "relu": 3}


def _io(residual: Optional[torch.Tensor], gate: Optional[torch.Tensor]) -> int:
    t = residual if residual is not None else gate
    return _lib.KLA_DTYPE_BF16 if t is not None and t.dtype == torch.bfloat16 else _lib.KLA_DTYPE_F32


def _ld(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else _sensor_rows(t)


def _code(dtype: torch.dtype) -> int:
    return _lib.KLA_DTYPE_BF16 if dtype == torch.bfloat16 else _lib.KLA_DTYPE_F32


@_lib.hip_op("kla_hip::gate_skip")
def _tail_op(y: torch.Tensor, residual: Optional[torch.Tensor], gate: Optional[torch.Tensor],
             lambda_skip: Optional[torch.Tensor], activation: int, out_bf16: bool) -> torch.Tensor:
    """out [B, L, M] = (y + lambda_skip * residual) * act(gate), fp32 or (out_bf16) bf16."""
    dev = _require_device(y, residual, gate, lambda_skip)
    B, L, M = y.shape
    out = torch.empty(B, L, M, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=dev)
    pt = _lib.ptr
    _lib.check("kla_gate_skip_fwd", _lib.lib().kla_gate_skip_fwd(
        _io(residual, gate), _code(out.dtype), pt(y), pt(residual), _ld(residual), pt(gate), _ld(gate),
        pt(lambda_skip), int(lambda_skip is not None and lambda_skip.dim() == 1), activation, pt(out), B * L, M,
        _lib.stream(dev)))
    return out


@_tail_op.register_fake
def _(y, residual, gate, lambda_skip, activation, out_bf16):
    return torch.empty_like(y, dtype=torch.bfloat16 if out_bf16 else torch.float32)


@_lib.hip_op("kla_hip::gate_skip_backward")
def _tail_bwd_op(dout: torch.Tensor, y: torch.Tensor, residual: Optional[torch.Tensor], gate: Optional[torch.Tensor],
                 lambda_skip: Optional[torch.Tensor], activation: int, need_res: bool, need_gate: bool
                 ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dy, d residual, d gate, d lambda_skip); the last three are empty when not asked for or absent."""
    dev = _require_device(dout, y, residual, gate, lambda_skip)
    B, L, M = y.shape
    io_dtype = residual.dtype if residual is not None else (gate.dtype if gate is not None else torch.float32)
    dy = torch.empty(B, L, M, dtype=torch.float32, device=dev)
    dres = torch.empty(B, L, M, dtype=io_dtype, device=dev) if need_res and residual is not None else y.new_empty(0)
    dgate = torch.empty(B, L, M, dtype=io_dtype, device=dev) if need_gate and gate is not None else y.new_empty(0)
    dlam = torch.empty(lambda_skip.shape, dtype=torch.float32, device=dev) if residual is not None \
        else y.new_empty(0)
    rows = B * L
    need = int(_lib.lib().kla_gate_skip_workspace_bytes(rows, M))
    ws, stream = _lib.scratch(need, dev)
    pt = _lib.ptr
    _lib.check("kla_gate_skip_bwd", _lib.lib().kla_gate_skip_bwd(
        _io(residual, gate), _code(dout.dtype), pt(dout), pt(y), pt(residual), _ld(residual), pt(gate), _ld(gate),
        pt(lambda_skip), int(lambda_skip is not None and lambda_skip.dim() == 1), activation, pt(dy),
        pt(dres) if dres.numel() else None, pt(dgate) if dgate.numel() else None,
        pt(dlam) if residual is not None else None, rows, M, pt(ws), ws.numel(), stream))
    return dy, dres, dgate, dlam


@_tail_bwd_op.register_fake
def _(dout, y, residual, gate, lambda_skip, activation, need_res, need_gate):
    io_dtype = residual.dtype if residual is not None else (gate.dtype if gate is not None else torch.float32)
    return (torch.empty_like(y), y.new_empty(y.shape if need_res and residual is not None else (0,), dtype=io_dtype),
            y.new_empty(y.shape if need_gate and gate is not None else (0,), dtype=io_dtype),
            y.new_empty(lambda_skip.shape if residual is not None else (0,)))


def _setup(ctx, inputs, output):
    y, residual, gate, lambda_skip, activation, out_bf16 = inputs
    ctx.activation = activation
    ctx.has = (residual is not None, gate is not None, lambda_skip is not None)
    ctx.save_for_backward(y, residual, gate, lambda_skip)


def _backward(ctx, dout):
    y, residual, gate, lambda_skip = ctx.saved_tensors
    has_res, has_gate, has_lam = ctx.has
    residual = residual if has_res else None
    gate = gate if has_gate else None
    lambda_skip = lambda_skip if has_lam else None
    need_res = has_res and ctx.needs_input_grad[1]
    need_gate = has_gate and ctx.needs_input_grad[2]
    if dout.dtype not in (torch.float32, torch.bfloat16):
        dout = dout.float()
    dy, dres, dgate, dlam = _lib.call(_tail_bwd_op, dout.contiguous(), y, residual, gate, lambda_skip,
                                      ctx.activation, need_res, need_gate)
    return (dy, dres if need_res else None, dgate if need_gate else None,
            dlam if has_res and ctx.needs_input_grad[3] else None, None, None)


_tail_op.register_autograd(_backward, setup_context=_setup)


def gate_skip_hip(y: torch.Tensor, residual: Optional[torch.Tensor], gate: Optional[torch.Tensor],
                  lambda_skip: Optional[torch.Tensor], activation: str = "silu",
                  out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """(y + lambda_skip * residual) * act(gate), [B, L, M] of ``out_dtype``.

    y: fp32 [B, L, M]. residual, gate: [B, L, M] of one dtype (fp32 or bf16) with
    rows that share one stride (views such as a half of the input projection are
    read in place), or None when the layer has no skip / no gate. lambda_skip:
    fp32 0-dim or [M] tensor, required with a residual. ``out_dtype`` bf16 gives
    the fp32 result rounded to nearest even -- what autocast hands the output
    projection -- without a separate cast; its gradient comes back in bf16.
    """
    if residual is not None and lambda_skip is None:
        raise ValueError("a residual needs lambda_skip")
    if residual is not None and gate is not None and residual.dtype != gate.dtype:
        raise TypeError(f"residual and gate must share a dtype; got {residual.dtype} and {gate.dtype}")
    if residual is not None and _sensor_rows(residual) is None:
        residual = residual.contiguous()
    if gate is not None and _sensor_rows(gate) is None:
        gate = gate.contiguous()
    lam = lambda_skip if residual is not None else None
    if lam is not None and (lam.dtype != torch.float32 or not lam.is_contiguous()):
        lam = lam.float().contiguous()
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"out_dtype must be float32 or bfloat16, got {out_dtype}")
    return _lib.call(_tail_op, y.float().contiguous(), residual, gate, lam, ACTIVATIONS[activation],
                     out_dtype == torch.bfloat16)
