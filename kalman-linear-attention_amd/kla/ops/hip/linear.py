"""A projection whose weight gradient is split over the tokens.

KLALayer's projections (``in_proj``, ``sensor_proj``, ``out_proj``; reference
``src/kla/layers/kla_layer.py:61``, ``:88``, ``:127``) are bias-free
``nn.Linear`` calls. In the backward torch forms the weight gradient
dW = dY^T X [n, k] as one GEMM reducing over all B*L tokens. At the layer's
training shapes (16384 tokens, n*k of 2 to 8 M) that product has only 32 to 72
output tiles of 256 x 256 for MI355X's 256 CUs, and runs at a third to two
thirds of the rate of the forward product.

:func:`linear` runs the same forward (``F.linear`` on the same bf16 operands)
and, in the backward, dX = dY W as torch does. dW becomes P token-chunk products
in one fp32-output batched GEMM, which gives P times the workgroups.
``kla_sum_parts`` then adds the partials in chunk order and rounds them to bf16
once. The result is torch's value up to the fp32 summation order inside the
GEMM, which torch does not fix either.
"""

from __future__ import annotations

import functools

import torch
import torch.nn.functional as F

from kla.ops.hip import _lib

# Token chunks per weight gradient: 4 took C4's three products from 657 to
# 446 us on MI355X (2 and 8 gained less once the partials' sum is counted).
_PARTS = 4
# Shortest token chunk worth a split.
_MIN_CHUNK = 2048


@functools.cache
def _cus(index: int) -> int:
    return torch.cuda.get_device_properties(index).multi_processor_count


def split_count(tokens: int, n: int, k: int, device: torch.device) -> int:
    """Token chunks for the weight gradient of an [n, k] projection over
    ``tokens`` rows: ``_PARTS`` when 256 x 256 output tiles would leave CUs idle
    and the chunks stay long, else 1 (one GEMM, as torch does)."""
    tiles = -(-n // 256) * -(-k // 256)
    if tokens % _PARTS or tokens < _PARTS * _MIN_CHUNK or tiles >= _cus(device.index or 0):
        return 1
    return _PARTS


def weight_grad_hip(dy: torch.Tensor, x: torch.Tensor, parts: int) -> torch.Tensor:
    """dY^T X for dy [T, n], x [T, k] (dense, bf16 or fp32, T divisible by
    ``parts``) as ``parts`` fp32 chunk products summed by ``kla_sum_parts``,
    rounded to dy's dtype."""
    T, n = dy.shape
    k = x.shape[1]
    if x.shape[0] != T or T % parts or dy.dtype != x.dtype:
        raise ValueError(f"weight_grad_hip: dy {tuple(dy.shape)} {dy.dtype}, x {tuple(x.shape)} {x.dtype}, "
                         f"{parts} parts")
    dy = dy.contiguous()
    x = x.contiguous()
    c = T // parts
    # The right operand is a plain contiguous batch (no transposed view).
    p = torch.bmm(dy.view(parts, c, n).transpose(1, 2), x.view(parts, c, k), out_dtype=torch.float32)
    out = torch.empty((n, k), dtype=dy.dtype, device=dy.device)
    code = _lib.KLA_DTYPE_BF16 if dy.dtype == torch.bfloat16 else _lib.KLA_DTYPE_F32
    _lib.check("kla_sum_parts", _lib.lib().kla_sum_parts(
        code, p.data_ptr(), parts, n * k, out.data_ptr(), torch.cuda.current_stream(dy.device).cuda_stream))
    return out


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, parts):
        ctx.save_for_backward(x, w)
        ctx.parts = parts
        return F.linear(x, w)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        n, k = w.shape
        dy2 = dy.reshape(-1, n)
        dx = dw = None
        if ctx.needs_input_grad[0]:
            # autograd's product for a linear layer's input gradient
            dx = dy2.mm(w).view(x.shape)
        if ctx.needs_input_grad[1]:
            dw = weight_grad_hip(dy2, x.reshape(-1, k), ctx.parts)
        return dx, dw, None


def linear(mod: torch.nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """``mod(x)`` for a bias-free ``nn.Linear`` on a ROCm GPU in bf16 (under
    bf16 autocast, or bf16 input and weight), with the weight gradient split
    over the tokens where :func:`split_count` says so; otherwise ``mod(x)``.
    The casts autocast would make are made here, so their backward is the same."""
    w = mod.weight
    if (mod.bias is not None or not x.is_cuda or not torch.is_grad_enabled()
            or not (x.requires_grad or w.requires_grad)):
        return mod(x)
    dt = (x.dtype, w.dtype)
    if torch.is_autocast_enabled("cuda"):
        if torch.get_autocast_dtype("cuda") != torch.bfloat16 or not all(
                d in (torch.float32, torch.bfloat16) for d in dt):
            return mod(x)
    elif dt != (torch.bfloat16, torch.bfloat16):
        return mod(x)
    n, k = w.shape
    parts = split_count(x.numel() // k if k else 0, n, k, x.device)
    if parts == 1:
        return mod(x)
    x, w = x.to(torch.bfloat16), w.to(torch.bfloat16)
    with torch.autocast("cuda", enabled=False):
        return _Linear.apply(x, w, parts)
