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

A projection whose output is split right away (``in_proj`` into z and the gate,
``sensor_proj`` into v, log sigma^2, k and q) goes through
:func:`linear_split`, which also replaces the split: it returns the pieces, and
its backward concatenates their gradients with ``kla_cat_cols`` for dX (with no
dX to form, each piece's gradient gives its rows of dW directly). Its weight is
taken in row blocks of whole 256-row tiles plus the rest (``sensor_proj``'s
4128 rows: 4096 + 32), each block one forward product and one split weight
gradient, so a ragged last tile row does not slow the whole product (C4's
sensor_proj forward 304 -> 231 us, weight gradient 370 -> 294 us on MI355X).
"""

from __future__ import annotations

import functools

import torch
import torch.nn.functional as F

from kla.ops.hip import _lib
from kla.ops.hip.split import _Like, cat_cols_hip

# At most this many token chunks per weight gradient, each at least this long.
_MAX_PARTS = 32
_MIN_CHUNK = 512


@functools.cache
def _cus(index: int) -> int:
    return torch.cuda.get_device_properties(index).multi_processor_count


def split_count(tokens: int, n: int, k: int, device: torch.device) -> int:
    """Token chunks for the weight gradient of an [n, k] projection over
    ``tokens`` rows: doubled from 1 while the 256 x 256 output tiles of all
    chunks are fewer than the CUs, the chunks divide the tokens evenly and stay
    at least ``_MIN_CHUNK`` long (at most ``_MAX_PARTS``). 1 means one GEMM, as
    torch does. C4's projections get 4 (in_proj), 8 (out_proj), 2 and 32
    (sensor_proj's two row blocks)."""
    tiles = -(-n // 256) * -(-k // 256)
    cus = _cus(device.index or 0)
    parts = 1
    while (tiles * parts < cus and parts < _MAX_PARTS and tokens % (2 * parts) == 0
           and tokens // (2 * parts) >= _MIN_CHUNK):
        parts *= 2
    return parts


def row_blocks(n: int) -> list[tuple[int, int]]:
    """[r0, r1) row blocks of an n-row weight: whole 256-row tiles, then the rest."""
    n1 = n - n % 256
    return [(0, n1), (n1, n)] if 0 < n1 < n else [(0, n)]


def _weight_grad_into(out: torch.Tensor, dy: torch.Tensor, r0: int, r1: int, x: torch.Tensor, parts: int):
    """out = dy[:, r0:r1]^T x for dy [T, n] (unit column stride, any row stride)
    and dense x [T, k], out a dense [r1 - r0, k] tensor of dy's dtype: ``parts``
    fp32 chunk products summed in chunk order by ``kla_sum_parts`` and rounded
    once, or torch's single product when ``parts`` is 1."""
    T = dy.shape[0]
    k = x.shape[1]
    g = dy[:, r0:r1]
    if parts == 1:
        torch.mm(g.t(), x, out=out)
        return
    c = T // parts
    ld = g.stride(0)
    # Chunk j of g^T: [r1 - r0, c] columns j c .. (j + 1) c - 1, read in place.
    # The right operand is a plain contiguous batch (no transposed view).
    gt = g.as_strided((parts, r1 - r0, c), (c * ld, 1, ld))
    p = torch.bmm(gt, x.view(parts, c, k), out_dtype=torch.float32)
    code = _lib.KLA_DTYPE_BF16 if dy.dtype == torch.bfloat16 else _lib.KLA_DTYPE_F32
    _lib.check("kla_sum_parts", _lib.lib().kla_sum_parts(
        code, p.data_ptr(), parts, (r1 - r0) * k, out.data_ptr(), _lib.stream(dy.device)))


def weight_grad_hip(dy: torch.Tensor, x: torch.Tensor, parts: int) -> torch.Tensor:
    """dY^T X for dy [T, n], x [T, k] (bf16 or fp32, T divisible by ``parts``)
    as ``parts`` fp32 chunk products summed by ``kla_sum_parts``, rounded to
    dy's dtype."""
    T, n = dy.shape
    if x.dim() != 2 or x.shape[0] != T or T % parts or dy.dtype != x.dtype:
        raise ValueError(f"weight_grad_hip: dy {tuple(dy.shape)} {dy.dtype}, x {tuple(x.shape)} {x.dtype}, "
                         f"{parts} parts")
    if dy.stride(1) != 1:
        dy = dy.contiguous()
    out = torch.empty((n, x.shape[1]), dtype=dy.dtype, device=dy.device)
    _weight_grad_into(out, dy, 0, n, x.contiguous(), parts)
    return out


def _backward(ctx, dy: torch.Tensor):
    """(dx, dw) of y = x w^T from dense dy [..., n]: dx = dy w (torch's product),
    dw per row block with the token split :func:`split_count` picks."""
    x, w = ctx.saved_tensors
    n, k = w.shape
    dy2 = dy.reshape(-1, n).contiguous()
    dx = dw = None
    if ctx.needs_input_grad[0]:
        dx = dy2.mm(w).view(x.shape)
    if ctx.needs_input_grad[1]:
        x2 = x.reshape(-1, k).contiguous()
        T = x2.shape[0]
        dw = torch.empty_like(w)
        for r0, r1 in ctx.blocks:
            _weight_grad_into(dw[r0:r1], dy2, r0, r1, x2, split_count(T, r1 - r0, k, dy.device))
    return dx, dw


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        ctx.blocks = row_blocks(w.shape[0])
        return F.linear(x, w)

    @staticmethod
    def backward(ctx, dy):
        return _backward(ctx, dy)


class _SplitLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, sizes):
        n = w.shape[0]
        blocks = _blocks_for(n, sizes) or [(0, n)]   # one block where a piece would straddle two
        ctx.save_for_backward(x, w)
        ctx.blocks, ctx.sizes = blocks, list(sizes)
        outs = [F.linear(x, w[r0:r1]) for r0, r1 in blocks]
        return _pieces(outs, blocks, sizes)

    @staticmethod
    def backward(ctx, *grads):
        x, w = ctx.saved_tensors
        if ctx.needs_input_grad[0]:
            dy = cat_cols_hip(list(grads), ctx.sizes, _Like(x.shape[:-1] + (w.shape[0],), w.dtype, w.device))
            dx, dw = _backward(ctx, dy)
            return dx, dw, None
        # Without dx each piece's gradient gives its own rows of dw: no concatenation.
        k = w.shape[1]
        x2 = x.reshape(-1, k).contiguous()
        T = x2.shape[0]
        dw = torch.empty_like(w)
        c0 = 0
        for g, size in zip(grads, ctx.sizes):
            if size == 0:
                continue   # an empty piece owns no rows of dw
            if g is None:
                dw[c0:c0 + size].zero_()
            else:
                g2 = g.to(w.dtype).reshape(-1, size)   # a view where the rows allow it
                if g2.stride(1) != 1:
                    g2 = g2.contiguous()
                _weight_grad_into(dw[c0:c0 + size], g2, 0, size, x2, split_count(T, size, k, w.device))
            c0 += size
        return None, dw, None


def _bf16_operands(mod: torch.nn.Linear, x: torch.Tensor):
    """(x, w) as the bf16 operands of mod(x) -- the casts autocast would make,
    made here so their backward is the same -- for a bias-free nn.Linear with a
    gradient to carry on a ROCm GPU under bf16 autocast (or with bf16 x and w);
    None otherwise."""
    w = mod.weight
    if (mod.bias is not None or not x.is_cuda or not torch.is_grad_enabled()
            or not (x.requires_grad or w.requires_grad)):
        return None
    dt = (x.dtype, w.dtype)
    if torch.is_autocast_enabled("cuda"):
        if torch.get_autocast_dtype("cuda") != torch.bfloat16 or not all(
                d in (torch.float32, torch.bfloat16) for d in dt):
            return None
    elif dt != (torch.bfloat16, torch.bfloat16):
        return None
    return x.to(torch.bfloat16), w.to(torch.bfloat16)


def linear(mod: torch.nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """``mod(x)``; for a bias-free ``nn.Linear`` in bf16 on a ROCm GPU whose
    weight gradient :func:`split_count` splits, the product with the split
    weight gradient."""
    n, k = mod.weight.shape
    ops = _bf16_operands(mod, x)
    if ops is None or split_count(x.numel() // k if k else 0, n, k, x.device) == 1:
        return mod(x)
    with torch.autocast("cuda", enabled=False):
        return _Linear.apply(*ops)


def _blocks_for(n: int, sizes: list[int]):
    """row_blocks(n) when each piece of ``sizes`` lies within one block (and there
    is more than one block), else None."""
    blocks = row_blocks(n)
    cuts = {sum(sizes[:i]) for i in range(len(sizes) + 1)}
    if len(blocks) == 1 or any(r0 not in cuts for r0, _ in blocks):
        return None
    return blocks


def _pieces(outs, blocks, sizes):
    """The pieces of ``sizes`` as column views of the blocks' outputs."""
    pieces, c0 = [], 0
    for size in sizes:
        b = max(i for i, (r0, _) in enumerate(blocks) if r0 <= c0)
        r0 = blocks[b][0]
        pieces.append(outs[b][..., c0 - r0:c0 - r0 + size])
        c0 += size
    return tuple(pieces)


# Fewest tokens for split_blocks: below, the second product's host cost (one
# more library call and the weight slices, ~20 us) outweighs what it saves on the
# GPU, and a layer of that size is bound by host time (C1, 2048 tokens).
_MIN_BLOCK_TOKENS = 8192


def split_blocks(mod: torch.nn.Linear, x: torch.Tensor, sizes: list[int]):
    """``torch.split(mod(x), sizes, dim=-1)`` as one product per row block of the
    weight (whole 256-row tiles, then the rest) where every piece lies within one
    block: hipBLASLt otherwise runs the ragged last tile row's kernel over the
    whole product (``sensor_proj`` [2080, 1024] in fp32 at 32768 tokens 1091 ->
    982 us on MI355X). Autograd goes through the weight slices. None where that
    does not apply (the caller splits ``mod(x)`` itself), including inputs of
    fewer than ``_MIN_BLOCK_TOKENS`` tokens."""
    w, b = mod.weight, mod.bias
    if not x.is_cuda or sum(sizes) != w.shape[0] or x.numel() < _MIN_BLOCK_TOKENS * w.shape[1]:
        return None
    blocks = _blocks_for(w.shape[0], sizes)
    if blocks is None:
        return None
    outs = [F.linear(x, w[r0:r1], None if b is None else b[r0:r1]) for r0, r1 in blocks]
    return _pieces(outs, blocks, sizes)


def linear_split(mod: torch.nn.Linear, x: torch.Tensor, sizes: list[int]):
    """``torch.split(mod(x), sizes, dim=-1)`` for a bias-free ``nn.Linear`` in
    bf16 on a ROCm GPU (at most four pieces): the weight in row blocks, the
    split weight gradient, the pieces' gradients concatenated on the GPU. None
    where that does not apply (the caller splits ``mod(x)`` itself)."""
    if len(sizes) > 4 or sum(sizes) != mod.weight.shape[0]:
        return None
    ops = _bf16_operands(mod, x)
    if ops is None:
        return None
    with torch.autocast("cuda", enabled=False):
        return _SplitLinear.apply(*ops, list(sizes))
