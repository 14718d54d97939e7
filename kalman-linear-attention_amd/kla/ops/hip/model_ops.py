"""Inference kernels for the sequence model around the KLA layers on MI355X.

One-token decode is bound by the number of kernel launches. RMSNorm
(reference ``src/kla/layers/common.py:45-55``) is six torch kernels and the
SwiGLU activation (``:120-123``) two; :func:`rms_norm_hip` and
:func:`swiglu_hip` are one HIP kernel each (``kla_rms_norm_fwd``,
``kla_swiglu_fwd``) with torch's values.

:func:`rows_linear_hip` is a linear layer on a few rows (the batch of a
one-token step) with the block's RMSNorm before it and the residual add or the
SwiGLU activation after it fused in (``kla_rows_linear_fwd``): a block's decode
step is then two such kernels per sublayer instead of a norm, a library GEMM and
an elementwise kernel or two.

None of them carries a gradient: the modules use them only when no gradient is
required, and keep the torch code otherwise.
"""

from __future__ import annotations

import weakref

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
        _lib.stream(x.device)))
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
        _lib.stream(h.device)))
    return out


# Weights whose rows do not start 16-byte aligned (e.g. [512, 1365]) -> a copy with
# the row stride rounded up to 4 elements, keyed on the weight's storage and
# version so that an in-place update refreshes it.
# Entries are keyed by id() (tensors compare elementwise, so they cannot be dict
# keys), hold a weak reference that confirms the identity, and are dropped when
# the weight is collected.
_ALIGNED_ROWS: dict[int, tuple] = {}


def _rows_aligned(w: torch.Tensor) -> torch.Tensor:
    """``w`` itself when every row starts 16-byte aligned, else a cached copy whose
    rows do (the row kernel then loads four k at a time: about twice as fast).
    Under stream capture a missing copy is not made (the kernel takes ``w`` as it is)."""
    if w.stride(0) % 4 == 0 and w.data_ptr() % 16 == 0:
        return w
    key = (w.data_ptr(), w._version)
    hit = _ALIGNED_ROWS.get(id(w))
    if hit is not None and hit[0]() is w and hit[1] == key:
        return hit[2]
    if w.is_cuda and torch.cuda.is_current_stream_capturing():
        return w
    n, k = w.shape
    view = torch.empty(n, (k + 3) // 4 * 4, dtype=w.dtype, device=w.device)[:, :k]
    view.copy_(w)
    if hit is None or hit[0]() is not w:
        weakref.finalize(w, _ALIGNED_ROWS.pop, id(w), None)
    _ALIGNED_ROWS[id(w)] = (weakref.ref(w), key, view)
    return view


def rows_linear_hip(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
                    norm_weight: torch.Tensor | None = None, eps: float = 0.0,
                    residual: torch.Tensor | None = None, swiglu: bool = False) -> torch.Tensor:
    """``epilogue(norm(x) @ weight.T + bias)`` for fp32 x [rows, k] (last dim contiguous).

    * ``norm_weight``: RMSNorm of each row first, ``(x * rsqrt(mean(x^2) + eps)) * norm_weight``;
    * ``residual`` [rows, n]: returns ``residual + (...)`` (the block's ``x + sublayer(x)``);
    * ``swiglu``: ``weight`` is [2 H, k]; returns ``silu(a[:, :H]) * a[:, H:]`` of the product a.

    The result is [rows, n] with its row stride rounded up to 4 elements (a view
    of a padded buffer when n is not a multiple of 4), so that it feeds the next
    row kernel with aligned rows.
    """
    if x.dim() != 2 or x.stride(-1) != 1:
        x = x.reshape(-1, x.shape[-1]).contiguous()
    w = _rows_aligned(weight if weight.stride(-1) == 1 else weight.contiguous())
    for name, t in (("x", x), ("weight", w), ("bias", bias), ("norm_weight", norm_weight), ("residual", residual)):
        if t is not None and t.dtype != torch.float32:
            raise TypeError(f"rows_linear_hip: {name} must be float32, got {t.dtype}")
    rows, k = x.shape
    n_w = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"rows_linear_hip: weight {tuple(w.shape)} does not match x {tuple(x.shape)}")
    n, glu_off, epi = n_w, 0, _lib.KLA_ROWS_PLAIN
    if swiglu:
        if n_w % 2:
            raise ValueError("rows_linear_hip: swiglu needs an even number of weight rows")
        n = glu_off = n_w // 2
        epi = _lib.KLA_ROWS_SWIGLU
    if residual is not None:
        if swiglu:
            raise ValueError("rows_linear_hip: residual and swiglu epilogues do not combine")
        if residual.shape != (rows, n) or residual.stride(-1) != 1:
            residual = residual.reshape(rows, n).contiguous()
        epi = _lib.KLA_ROWS_RESIDUAL
    b = bias.contiguous() if bias is not None else None
    g = norm_weight.contiguous() if norm_weight is not None else None
    y = torch.empty(rows, (n + 3) // 4 * 4, dtype=torch.float32, device=x.device)[:, :n]
    p = _lib.ptr
    _lib.check("kla_rows_linear_fwd", _lib.lib().kla_rows_linear_fwd(
        epi, p(x), x.stride(0), p(w), w.stride(0), p(b), p(g), float(eps),
        p(residual), residual.stride(0) if residual is not None else 0, p(y), y.stride(0),
        rows, n, k, glu_off, _lib.stream(x.device)))
    return y


def gather_rows_hip(weight: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """``weight[ids]`` (nn.Embedding) for int64 ids of any shape, fp32 or bf16 rows
    with a contiguous last dimension; an id outside [0, vocab) gives a row of NaN."""
    if weight.stride(-1) != 1:
        weight = weight.contiguous()
    flat = ids.reshape(-1)
    if flat.dtype != torch.int64 or not flat.is_contiguous():
        flat = flat.to(torch.int64).contiguous()
    dim = weight.shape[-1]
    out = torch.empty(flat.numel(), dim, dtype=weight.dtype, device=weight.device)
    _lib.check("kla_gather_rows", _lib.lib().kla_gather_rows(
        _code(weight), weight.data_ptr(), weight.stride(0), weight.shape[0], flat.data_ptr(), out.data_ptr(),
        out.stride(0), flat.numel(), dim, _lib.stream(weight.device)))
    return out.view(*ids.shape, dim)


def argmax_rows_hip(x: torch.Tensor) -> torch.Tensor:
    """``x.argmax(dim=-1, keepdim=True)`` for fp32 x [..., n] (int64, torch's order:
    NaN first, ties to the smaller index)."""
    if x.dtype != torch.float32:
        raise TypeError(f"argmax_rows_hip: expected float32, got {x.dtype}")
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    out = torch.empty(x2.shape[0], 1, dtype=torch.int64, device=x.device)
    nbytes = _lib.lib().kla_argmax_workspace_bytes(x2.shape[0], x2.shape[1])
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes else None
    _lib.check("kla_argmax_rows", _lib.lib().kla_argmax_rows(
        x2.data_ptr(), x2.stride(0), x2.shape[0], x2.shape[1], out.data_ptr(), 1,
        ws.data_ptr() if ws is not None else None, nbytes, _lib.stream(x.device)))
    return out.view(*x.shape[:-1], 1)


_CONV_ACT = {"identity": 0, "silu": 1, "gelu": 2, "relu": 3}


def rows_linear_conv_hip(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, *,
                         norm_weight: torch.Tensor | None, eps: float, conv_weight: torch.Tensor,
                         conv_bias: torch.Tensor | None, window: torch.Tensor, activation: str = "silu",
                         in_place: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """``norm(x) @ weight.T + bias`` for fp32 x [rows, k] with one token of the
    depthwise causal conv applied to the first ``D = conv_weight.shape[0]`` output
    columns: returns (y [rows, n], new window [rows, D, K - 1]). ``window`` is the
    conv state [rows, D, K - 1] (contiguous fp32); with ``in_place`` the new window
    is written over it and returned as the same tensor."""
    if x.dim() != 2 or x.stride(-1) != 1:
        x = x.reshape(-1, x.shape[-1]).contiguous()
    w = _rows_aligned(weight if weight.stride(-1) == 1 else weight.contiguous())
    rows, k = x.shape
    n = w.shape[0]
    D, K = conv_weight.shape
    cw = conv_weight.contiguous()
    if window.shape != (rows, D, K - 1) or not window.is_contiguous() or window.dtype != torch.float32:
        raise ValueError(f"rows_linear_conv_hip: window {tuple(window.shape)} is not a dense fp32 [rows, D, K-1]")
    win_out = window if in_place else torch.empty_like(window)
    y = torch.empty(rows, (n + 3) // 4 * 4, dtype=torch.float32, device=x.device)[:, :n]
    p = _lib.ptr
    g = norm_weight.contiguous() if norm_weight is not None else None
    _lib.check("kla_rows_linear_conv_fwd", _lib.lib().kla_rows_linear_conv_fwd(
        p(x), x.stride(0), p(w), w.stride(0), p(bias.contiguous() if bias is not None else None), p(g), float(eps),
        p(y), y.stride(0), rows, n, k, p(cw), p(conv_bias.contiguous() if conv_bias is not None else None),
        p(window), p(win_out), D, K, _CONV_ACT[activation], _lib.stream(x.device)))
    return y, win_out
