"""One O(1) decode step of the KLA filter on MI355X (reference kla_step,
src/kla/ops/kla_ops.py:293-331), as a single HIP kernel instead of ~20 torch
elementwise launches. Forward only: the hip backend's ``kla_step`` runs the
torch formula when a gradient is required (decode runs under no_grad).
"""

from __future__ import annotations

import torch

from kla.ops.hip import _lib
from kla.ops.hip.scans import _require_device

_F32 = torch.float32


@_lib.hip_op("kla_hip::kla_step")
def _step_op(v: torch.Tensor, lambda_v: torch.Tensor, k: torch.Tensor, q: torch.Tensor, a: torch.Tensor,
             p: torch.Tensor, lam: torch.Tensor, eta: torch.Tensor, decode_from_prior: bool
             ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y [B, M], y_var [B, M], lam [B, M, S], eta [B, M, S]) after one step; a
    d_state above 256 runs as the fused scan's state groups."""
    dev = _require_device(v, lambda_v, k, q, a, p, lam, eta)
    B, M = v.shape
    S = k.shape[1]
    for name, t, shape in (("lambda_v", lambda_v, (B, M)), ("k", k, (B, S)), ("q", q, (B, S)), ("a", a, (M, S)),
                           ("p", p, (M, S)), ("lam", lam, (B, M, S)), ("eta", eta, (B, M, S))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {shape}")
    from kla.ops.hip.fused import MAX_STATE, state_groups

    if S > MAX_STATE:
        # The scan's state groups: each a step of its own lanes, the read-outs summed in group order.
        y = y_var = None
        lam_out, eta_out = torch.empty_like(lam), torch.empty_like(eta)
        for s0, n in state_groups(S):
            part = [t[..., s0:s0 + n].contiguous() for t in (k, q, a, p, lam, eta)]
            yg, yvg, lg, eg = _step_one(v, lambda_v, *part, decode_from_prior, dev)
            y, y_var = (yg, yvg) if y is None else (y.add_(yg), y_var.add_(yvg))
            lam_out[..., s0:s0 + n] = lg
            eta_out[..., s0:s0 + n] = eg
        return y, y_var, lam_out, eta_out
    return _step_one(v, lambda_v, k, q, a, p, lam, eta, decode_from_prior, dev)


def _step_one(v, lambda_v, k, q, a, p, lam, eta, decode_from_prior, dev):
    """One kla_step_fwd launch (d_state <= 256)."""
    B, M = v.shape
    S = k.shape[1]
    y, y_var = v.new_empty(B, M), v.new_empty(B, M)
    lam_out, eta_out = torch.empty_like(lam), torch.empty_like(eta)
    if B * M * S == 0:
        return y.zero_(), y_var.zero_(), lam_out, eta_out   # sums over no state lanes
    pt = _lib.ptr
    _lib.check("kla_step_fwd", _lib.lib().kla_step_fwd(
        pt(v), pt(lambda_v), pt(k), pt(q), pt(a), pt(p), pt(lam), pt(eta), pt(y), pt(y_var), pt(lam_out),
        pt(eta_out), int(decode_from_prior), B, M, S, _lib.stream(dev)))
    return y, y_var, lam_out, eta_out


@_step_op.register_fake
def _(v, lambda_v, k, q, a, p, lam, eta, decode_from_prior):
    return v.new_empty(v.shape), v.new_empty(v.shape), torch.empty_like(lam), torch.empty_like(eta)


def kla_step_hip(v, lambda_v, k, q, a, p, lam, eta, decode_from_prior: bool = False):
    # a, p: any shape that broadcasts to [M, S], as the torch formula takes them.
    a, p = a.expand(v.shape[-1], k.shape[-1]), p.expand(v.shape[-1], k.shape[-1])
    v, lambda_v, k, q, a, p, lam, eta = (t.to(_F32).contiguous() for t in (v, lambda_v, k, q, a, p, lam, eta))
    return _lib.call(_step_op, v, lambda_v, k, q, a, p, lam, eta, bool(decode_from_prior))
