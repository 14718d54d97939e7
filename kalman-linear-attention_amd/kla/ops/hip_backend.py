"""The ``"hip"`` KLA backend: the KLA scan on MI355X kernels.

Fused path (``kernel="fused"``, the default): the whole filter in one kernel
per direction (:mod:`kla.ops.hip.fused`); nothing of shape [B, L, M, S] is
materialised, and the backward is the exact adjoint. A d_state above 256 runs as
consecutive groups of at most 256 state lanes whose read-outs are summed.

Composed path (``kernel="composed"``): the per-(b, l, m, s) glue -- sufficient
statistics, Moebius leaves, the gain alpha, posterior and read-out -- is torch
elementwise work, and the two recurrences run on the hand-written HIP scans
(:func:`kla.ops.hip.mobius_scan`, :func:`kla.ops.hip.affine_scan`), whose
backward passes are the exact adjoint kernels. The arrangement follows the
reference's composed Triton path (src/kla/ops/triton_backend.py:143-171) with
two differences: the constant leaf D = 1 is never materialised (the kernel
takes D = NULL), and the initial information eta0 enters the affine kernel as
its initial state instead of being folded into r_0 (the same value).

Contract (reference kla_ops.py:486-541): returns (y [B, L, M] fp32, y_var
[B, L, M] fp32, KLAState(lam [B, M, S], eta [B, M, S])), accepts an initial
state, supports ``decode_from_prior``, and differentiates through everything
including the returned state. Inputs are computed in float32.
"""

from __future__ import annotations

from typing import Optional

import torch

from kla.ops.kla_ops import EPS, KLAState, _broadcast_ap, _readout, _sufficient_stats, init_state


def kla_scan_hip(
    v: torch.Tensor,
    lambda_v: torch.Tensor,
    k: torch.Tensor,
    q: torch.Tensor,
    a: torch.Tensor,
    p: torch.Tensor,
    initial_state: Optional[KLAState] = None,
    decode_from_prior: bool = False,
    kernel: str = "auto",
):
    """KLA scan on the MI355X kernels. ``kernel``: "auto", "fused" or "composed"."""
    from kla.ops.hip import affine_scan, mobius_scan
    from kla.ops.hip.fused import kla_scan_fused

    if kernel not in ("auto", "fused", "composed"):
        raise ValueError(f"Unknown hip kernel {kernel!r}; expected 'auto', 'fused' or 'composed'")
    if not v.is_cuda:
        raise NotImplementedError("The hip KLA backend requires tensors on a ROCm GPU; use backend='torch'.")
    if kernel in ("auto", "fused"):
        lam0 = eta0 = None
        if initial_state is not None:
            lam0, eta0 = initial_state.lam, initial_state.eta
        y, y_var, lam, eta = kla_scan_fused(v, lambda_v, k, q, a, p, lam0, eta0, decode_from_prior)
        return y, y_var, KLAState(lam=lam, eta=eta)

    v, lambda_v, k, q = (t.float() for t in (v, lambda_v, k, q))
    Bn, L, M = v.shape
    S = k.shape[2]
    if initial_state is None:
        initial_state = init_state(Bn, M, S, device=v.device)
    lam0 = initial_state.lam.float().contiguous()
    eta0 = initial_state.eta.float().contiguous()
    if L == 0:
        # No steps: empty read-outs, and the state leaves as it came in.
        empty = v.new_zeros(Bn, 0, M)
        return empty, empty.clone(), KLAState(lam=lam0, eta=eta0)

    phi, r = _sufficient_stats(v, lambda_v, k)
    a_, p_ = _broadcast_ap(a.float(), p.float(), phi)
    a2 = (a_ * a_).clamp_min(EPS)

    # Precision: lam_t = (A lam' + phi) / (C lam' + 1), A = (1 + p phi)/a^2, C = p/a^2.
    leaf_a = (1.0 + p_ * phi) / a2
    leaf_c = (p_ / a2).expand_as(phi)
    lam = mobius_scan(leaf_a, phi, leaf_c, None, lam0)
    var = 1.0 / lam.clamp_min(EPS)

    # Information: eta_t = alpha_t eta_{t-1} + r_t, alpha_t = a / max(a^2 + p lam_{t-1}, EPS).
    lam_prev = torch.cat((lam0.unsqueeze(1), lam[:, :-1]), dim=1)
    alpha = a_ / (a2 + p_ * lam_prev).clamp_min(EPS)
    eta = affine_scan(alpha, r, eta0)

    mean = eta * var
    if decode_from_prior:
        mean = a_ * mean
        var = a2 * var + p_
    y, y_var = _readout(mean, var, q)
    return y, y_var, KLAState(lam=lam[:, -1], eta=eta[:, -1])
