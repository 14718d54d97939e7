"""PyTorch custom ops over the MI355X scan kernels, with autograd.

Public, differentiable:

* :func:`mobius_scan` ``(A, B, C, D=None, lam0=None) -> lam`` -- the standalone
  Moebius precision scan, contract of the reference's ``tiled_mobius_scan``
  (src/kla/ops/kernels/triton/tiled_mobius_scan.py:301-306).
* :func:`affine_scan` ``(g, u, h0=None) -> h`` -- the standalone affine scan,
  contract of ``tiled_affine_scan`` (tiled_mobius_scan.py:309-311), plus an
  optional initial state ``h0`` (the reference folds it into ``u[:, 0]``).

Operands are [batch, steps, *lanes] with any trailing lane shape (the
reference's [B, L, M, S]); states are [batch, *lanes]. The Moebius scan runs in
float32 (other float inputs are cast, as the reference's GPU backends do). The
affine scan keeps float32 or bfloat16 sequence I/O (fp32 arithmetic and state).

Each op is a ``torch.library`` custom op (``kla_hip::*``) whose backward is the
hand-written exact adjoint kernel, registered with ``register_autograd``.
"""

from __future__ import annotations

from typing import Optional

import torch

from kla.ops.hip import _lib

_F32 = torch.float32
_BF16 = torch.bfloat16


def _dims(x: torch.Tensor) -> tuple[int, int, int]:
    if x.dim() < 2:
        raise ValueError(f"sequence operand must be [batch, steps, ...], got shape {tuple(x.shape)}")
    lanes = 1
    for d in x.shape[2:]:
        lanes *= d
    return x.shape[0], x.shape[1], lanes


def _require_device(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise NotImplementedError(
                "The hip KLA kernels need tensors on a ROCm GPU; use backend='torch' for CPU tensors."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"operands on different devices: {dev} and {t.device}")
    return dev


def _check_state(state: Optional[torch.Tensor], x: torch.Tensor, name: str) -> None:
    if state is None:
        return
    if tuple(state.shape) != (x.shape[0], *x.shape[2:]):
        raise ValueError(f"{name} must have shape {(x.shape[0], *x.shape[2:])}, got {tuple(state.shape)}")
    if state.dtype != _F32 or not state.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 tensor")


def _check_seq(ts, like: torch.Tensor, dtype: torch.dtype) -> None:
    for name, t in ts:
        if t is None:
            continue
        if t.shape != like.shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(like.shape)}")
        if t.dtype != dtype or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dtype} tensor")


# ================================================================== Moebius


@_lib.hip_op("kla_hip::mobius_scan")
def _mobius_scan_op(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, D: Optional[torch.Tensor],
                    lam0: Optional[torch.Tensor]) -> torch.Tensor:
    dev = _require_device(A, B, C, D, lam0)
    _check_seq((("A", A), ("B", B), ("C", C), ("D", D)), A, _F32)
    _check_state(lam0, A, "lam0")
    nb, nt, nl = _dims(A)
    lam = torch.empty_like(A)
    if lam.numel() == 0:
        return lam
    ws, stream = _lib.workspace(_lib.KLA_SCAN_MOBIUS_FWD, nb, nt, nl, dev)
    p = _lib.ptr
    _lib.check("kla_mobius_scan_fwd", _lib.lib().kla_mobius_scan_fwd(
        p(A), p(B), p(C), p(D), p(lam0), p(lam), nb, nt, nl, p(ws), ws.numel(), stream))
    return lam


@_mobius_scan_op.register_fake
def _(A, B, C, D, lam0):
    return torch.empty_like(A)


@_lib.hip_op("kla_hip::mobius_scan_backward")
def _mobius_scan_bwd_op(dlam: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                        D: Optional[torch.Tensor], lam0: Optional[torch.Tensor], lam: torch.Tensor
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (dA, dB, dC, dD, dlam0); dD / dlam0 are empty when D / lam0 is None."""
    dev = _require_device(dlam, A, B, C, D, lam0, lam)
    _check_seq((("dlam", dlam), ("A", A), ("B", B), ("C", C), ("D", D), ("lam", lam)), A, _F32)
    _check_state(lam0, A, "lam0")
    nb, nt, nl = _dims(A)
    dA, dB, dC = torch.empty_like(A), torch.empty_like(A), torch.empty_like(A)
    dD = torch.empty_like(A) if D is not None else A.new_empty(0)
    dlam0 = torch.empty_like(lam0) if lam0 is not None else A.new_empty(0)
    if nb * nl == 0:
        return dA, dB, dC, dD, dlam0
    ws, stream = _lib.workspace(_lib.KLA_SCAN_MOBIUS_BWD, nb, nt, nl, dev)
    p = _lib.ptr
    _lib.check("kla_mobius_scan_bwd", _lib.lib().kla_mobius_scan_bwd(
        p(dlam), p(A), p(B), p(C), p(D), p(lam0), p(lam), p(dA), p(dB), p(dC),
        p(dD) if D is not None else None, p(dlam0) if lam0 is not None else None,
        nb, nt, nl, p(ws), ws.numel(), stream))
    return dA, dB, dC, dD, dlam0


@_mobius_scan_bwd_op.register_fake
def _(dlam, A, B, C, D, lam0, lam):
    e = A.new_empty(0)
    return (torch.empty_like(A), torch.empty_like(A), torch.empty_like(A),
            torch.empty_like(A) if D is not None else e,
            torch.empty_like(lam0) if lam0 is not None else e)


def _mobius_setup(ctx, inputs, output):
    A, B, C, D, lam0 = inputs
    ctx.has_d = D is not None
    ctx.has_l0 = lam0 is not None
    ctx.save_for_backward(A, B, C, D, lam0, output)


def _mobius_backward(ctx, dlam):
    A, B, C, D, lam0, lam = ctx.saved_tensors
    dA, dB, dC, dD, dlam0 = _lib.call(_mobius_scan_bwd_op, dlam.contiguous(), A, B, C, D, lam0, lam)
    return dA, dB, dC, (dD if ctx.has_d else None), (dlam0 if ctx.has_l0 else None)


_mobius_scan_op.register_autograd(_mobius_backward, setup_context=_mobius_setup)


def mobius_scan(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, D: Optional[torch.Tensor] = None,
                lam0: Optional[torch.Tensor] = None) -> torch.Tensor:
    """lam_t = (A_t lam_{t-1} + B_t) / max(C_t lam_{t-1} + D_t, 1e-12), lam_{-1} = lam0 (default 1).

    A, B, C, D: [batch, steps, *lanes]; lam0: [batch, *lanes]. D=None means D == 1
    (the KLA leaf), and saves reading a tensor of ones. Returns lam (float32).
    """
    A, B, C = (t.to(_F32).contiguous() for t in (A, B, C))
    D = None if D is None else D.to(_F32).contiguous()
    lam0 = None if lam0 is None else lam0.to(_F32).contiguous()
    return _lib.call(_mobius_scan_op, A, B, C, D, lam0)


# =================================================================== affine


def _io_dtype(t: torch.Tensor) -> int:
    if t.dtype == _F32:
        return _lib.KLA_DTYPE_F32
    if t.dtype == _BF16:
        return _lib.KLA_DTYPE_BF16
    raise TypeError(f"affine scan I/O must be float32 or bfloat16, got {t.dtype}")


@_lib.hip_op("kla_hip::affine_scan")
def _affine_scan_op(g: torch.Tensor, u: torch.Tensor, h0: Optional[torch.Tensor]) -> torch.Tensor:
    dev = _require_device(g, u, h0)
    _check_seq((("g", g), ("u", u)), g, g.dtype)
    _check_state(h0, g, "h0")
    code = _io_dtype(g)
    nb, nt, nl = _dims(g)
    h = torch.empty_like(g)
    if h.numel() == 0:
        return h
    ws, stream = _lib.workspace(_lib.KLA_SCAN_AFFINE_FWD, nb, nt, nl, dev)
    p = _lib.ptr
    _lib.check("kla_affine_scan_fwd", _lib.lib().kla_affine_scan_fwd(
        code, p(g), p(u), p(h0), p(h), nb, nt, nl, p(ws), ws.numel(), stream))
    return h


@_affine_scan_op.register_fake
def _(g, u, h0):
    return torch.empty_like(g)


@_lib.hip_op("kla_hip::affine_scan_backward")
def _affine_scan_bwd_op(dh: torch.Tensor, g: torch.Tensor, h: torch.Tensor, h0: Optional[torch.Tensor]
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (dg, du, dh0); dh0 is empty when h0 is None."""
    dev = _require_device(dh, g, h, h0)
    _check_seq((("dh", dh), ("g", g), ("h", h)), g, g.dtype)
    _check_state(h0, g, "h0")
    code = _io_dtype(g)
    nb, nt, nl = _dims(g)
    dg, du = torch.empty_like(g), torch.empty_like(g)
    dh0 = torch.empty_like(h0) if h0 is not None else g.new_empty(0, dtype=_F32)
    if nb * nl == 0:
        return dg, du, dh0
    ws, stream = _lib.workspace(_lib.KLA_SCAN_AFFINE_BWD, nb, nt, nl, dev)
    p = _lib.ptr
    _lib.check("kla_affine_scan_bwd", _lib.lib().kla_affine_scan_bwd(
        code, p(dh), p(g), p(h), p(h0), p(dg), p(du), p(dh0) if h0 is not None else None,
        nb, nt, nl, p(ws), ws.numel(), stream))
    return dg, du, dh0


@_affine_scan_bwd_op.register_fake
def _(dh, g, h, h0):
    return (torch.empty_like(g), torch.empty_like(g),
            torch.empty_like(h0) if h0 is not None else g.new_empty(0, dtype=_F32))


def _affine_setup(ctx, inputs, output):
    g, u, h0 = inputs
    ctx.has_h0 = h0 is not None
    ctx.save_for_backward(g, h0, output)


def _affine_backward(ctx, dh):
    g, h0, h = ctx.saved_tensors
    dg, du, dh0 = _lib.call(_affine_scan_bwd_op, dh.to(g.dtype).contiguous(), g, h, h0)
    return dg, du, (dh0 if ctx.has_h0 else None)


_affine_scan_op.register_autograd(_affine_backward, setup_context=_affine_setup)


def affine_scan(g: torch.Tensor, u: torch.Tensor, h0: Optional[torch.Tensor] = None) -> torch.Tensor:
    """h_t = g_t h_{t-1} + u_t, h_{-1} = h0 (default 0).

    g, u: [batch, steps, *lanes], both float32 or both bfloat16 (float16 and
    float64 are cast to float32); h0: [batch, *lanes] (float32). Returns h in
    the I/O dtype; accumulation is float32.
    """
    if g.dtype != u.dtype or g.dtype not in (_F32, _BF16):
        g, u = g.to(_F32), u.to(_F32)
    g, u = g.contiguous(), u.contiguous()
    h0 = None if h0 is None else h0.to(_F32).contiguous()
    return _lib.call(_affine_scan_op, g, u, h0)
