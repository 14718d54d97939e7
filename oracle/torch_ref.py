"""torch (CPU) restatement of the reference's pure-PyTorch scan path (test oracle).

This is "the reference's own pure-PyTorch/CPU scan": the doubling (Hillis-Steele)
scan of src/kla/ops/scan.py:29-45 over the trace-normalised Moebius combine and
the affine combine of src/kla/ops/kla_ops.py:76-123, assembled as in
kla_scan_torch (kla_ops.py:188-290). Gradients come from torch autograd through
those elementwise ops, so they do not depend on any hand-written adjoint.

Uses:
* parity reference for the GPU kernels in fp32 (same algorithm, same dtype as
  the reference CPU path) and, in float64, a second opinion beside
  :mod:`oracle.scans`;
* :func:`kla_scan_stepwise`, the same filter one step at a time: the float64
  reference where the prefix form loses precision (a precision near zero);
* the timed ``cpu_baseline`` of ``bench.py`` (kind "port").
"""

from __future__ import annotations

import torch

EPS = 1e-12
P_MIN = 1e-12


def doubling_scan(combine, xs, dim=1):
    """Inclusive scan by doubling (restates scan.py:29-45)."""
    ys = tuple(xs)
    n = ys[0].size(dim)
    off = 1
    while off < n:
        lo = tuple(t.narrow(dim, 0, n - off) for t in ys)
        hi = tuple(t.narrow(dim, off, n - off) for t in ys)
        comb = combine(lo, hi)
        ys = tuple(torch.cat((t.narrow(dim, 0, off), c), dim=dim) for t, c in zip(ys, comb))
        off *= 2
    return ys


def sequential_scan(combine, xs, dim=1):
    """Inclusive scan by a python loop (restates scan.py:48-59)."""
    n = xs[0].size(dim)
    state = tuple(t.select(dim, 0) for t in xs)
    outs = [state]
    for i in range(1, n):
        state = combine(state, tuple(t.select(dim, i) for t in xs))
        outs.append(state)
    return tuple(torch.stack([o[j] for o in outs], dim=dim) for j in range(len(xs)))


def mobius_combine_tracenorm(left, right):
    """kla_ops.py:76-116."""
    a1, b1, c1, d1 = left
    a2, b2, c2, d2 = right
    a = a2 * a1 + b2 * c1
    b = a2 * b1 + b2 * d1
    c = c2 * a1 + d2 * c1
    d = c2 * b1 + d2 * d1
    inv = 1.0 / (a + d).clamp_min(EPS)
    return a * inv, b * inv, c * inv, d * inv


def mobius_combine_log(left, right):
    """kla_ops.py:64-73."""
    a1, b1, c1, d1 = left
    a2, b2, c2, d2 = right
    return (
        torch.logaddexp(a2 + a1, b2 + c1),
        torch.logaddexp(a2 + b1, b2 + d1),
        torch.logaddexp(c2 + a1, d2 + c1),
        torch.logaddexp(c2 + b1, d2 + d1),
    )


def affine_combine(left, right):
    """kla_ops.py:119-123."""
    a1, b1 = left
    a2, b2 = right
    return a2 * a1, a2 * b1 + b2


def mobius_scan(A, B, C, D=None, lam0=None, scan=doubling_scan):
    """Standalone Moebius scan on [B, T, ...] via the reference's CPU algorithm.

    Scan of the trace-normalised combine, then lam = (pA lam0 + pB)/max(pC lam0 + pD, EPS)
    (kla_ops.py:244-251). Differentiable through autograd.
    """
    if D is None:
        D = torch.ones_like(A)
    if lam0 is None:
        lam0 = torch.ones_like(A[:, 0])
    pA, pB, pC, pD = scan(mobius_combine_tracenorm, (A, B, C, D), dim=1)
    l0 = lam0.unsqueeze(1)
    return (pA * l0 + pB) / (pC * l0 + pD).clamp_min(EPS)


def affine_scan(g, u, h0=None, scan=doubling_scan):
    """Standalone affine scan h_t = g_t h_{t-1} + u_t via the reference's CPU algorithm
    (kla_ops.py:279-280). Differentiable through autograd."""
    pg, pu = scan(affine_combine, (g, u), dim=1)
    if h0 is None:
        return pu
    return pg * h0.unsqueeze(1) + pu


def kla_scan_torch(v, lambda_v, k, q, a, p, lam0=None, eta0=None, decode_from_prior=False,
                   mobius_impl="linear", scan=doubling_scan):
    """Restates kla_scan_torch (kla_ops.py:188-290). Returns (y, y_var, lam_fin, eta_fin).

    dtype is taken from ``v`` (float32 or float64); no widening is done here.
    """
    Bn, L, M = v.shape
    S = k.shape[2]
    dt = v.dtype
    lam0 = torch.ones(Bn, M, S, dtype=dt) if lam0 is None else lam0
    eta0 = torch.zeros(Bn, M, S, dtype=dt) if eta0 is None else eta0
    phi = lambda_v.unsqueeze(-1) * (k * k).unsqueeze(-2)
    if mobius_impl == "log":
        phi = phi.clamp_min(EPS)
    r = (v * lambda_v).unsqueeze(-1) * k.unsqueeze(-2)
    a_ = a.view(1, 1, M, S).to(dt)
    p_ = p.view(1, 1, M, S).clamp_min(P_MIN).to(dt)
    a2 = (a_ * a_).clamp_min(EPS)
    if mobius_impl == "linear":
        A = ((1.0 + p_ * phi) / a2).expand_as(phi)
        C = (p_ / a2).expand_as(phi)
        pA, pB, pC, pD = scan(mobius_combine_tracenorm, (A, phi, C, torch.ones_like(phi)), dim=1)
        l0 = lam0.unsqueeze(1)
        lam = (pA * l0 + pB) / (pC * l0 + pD).clamp_min(EPS)
        var = 1.0 / lam.clamp_min(EPS)
    elif mobius_impl == "log":
        la2 = a2.log()
        lA = (torch.log1p(p_ * phi) - la2).expand_as(phi)
        lB = phi.log()
        lC = (p_.log() - la2).expand_as(phi)
        lD = torch.zeros_like(phi)
        pA, pB, pC, pD = scan(mobius_combine_log, (lA, lB, lC, lD), dim=1)
        ll0 = lam0.clamp_min(EPS).log().unsqueeze(1)
        log_lam = torch.logaddexp(pA + ll0, pB) - torch.logaddexp(pC + ll0, pD)
        lam = log_lam.exp()
        var = (-log_lam).exp()
    else:
        raise ValueError(mobius_impl)
    lam_prev = torch.cat((lam0.unsqueeze(1), lam[:, :-1]), dim=1)
    alpha = a_ / (a2 + p_ * lam_prev).clamp_min(EPS)
    pAl, pR = scan(affine_combine, (alpha, r), dim=1)
    eta = pAl * eta0.unsqueeze(1) + pR
    mean = eta * var
    if decode_from_prior:
        mean = a_ * mean
        var = a2 * var + p_
    y = torch.einsum("blms,bls->blm", mean, q)
    y_var = torch.einsum("blms,bls->blm", var, q * q)
    return y, y_var, lam[:, -1], eta[:, -1]


def kla_scan_stepwise(v, lambda_v, k, q, a, p, lam0=None, eta0=None, decode_from_prior=False):
    """kla_scan_torch's filter (kla_ops.py:188-290) applied one step at a time:
    the same leaves, guards and read-out (phi not floored, p at P_MIN, a^2 at
    EPS, every denominator at EPS), each Moebius leaf and affine leaf applied to
    the running state instead of composed into prefixes. Differentiable through
    autograd. Where the trace-normalised prefixes lose precision (a state near
    zero under strong decay: the normalised D entry of a prefix falls toward or
    below EPS, and the prefix read-out's max(C lam0 + D, EPS) departs from the
    filter) this form stays exact; elsewhere the two agree to rounding."""
    Bn, L, M = v.shape
    S = k.shape[2]
    dt = v.dtype
    lam = torch.ones(Bn, M, S, dtype=dt) if lam0 is None else lam0
    eta = torch.zeros(Bn, M, S, dtype=dt) if eta0 is None else eta0
    a_ = a.view(1, M, S).to(dt)
    p_ = p.view(1, M, S).clamp_min(P_MIN).to(dt)
    a2 = (a_ * a_).clamp_min(EPS)
    ys, yvs = [], []
    for t in range(L):
        phi = lambda_v[:, t].unsqueeze(-1) * (k[:, t] * k[:, t]).unsqueeze(-2)
        r = (v[:, t] * lambda_v[:, t]).unsqueeze(-1) * k[:, t].unsqueeze(-2)
        A = (1.0 + p_ * phi) / a2
        C = p_ / a2
        alpha = a_ / (a2 + p_ * lam).clamp_min(EPS)
        lam = (A * lam + phi) / (C * lam + 1.0).clamp_min(EPS)
        eta = alpha * eta + r
        var = 1.0 / lam.clamp_min(EPS)
        mean = eta * var
        if decode_from_prior:
            mean = a_ * mean
            var = a2 * var + p_
        ys.append(torch.einsum("bms,bs->bm", mean, q[:, t]))
        yvs.append(torch.einsum("bms,bs->bm", var, q[:, t] * q[:, t]))
    return torch.stack(ys, 1), torch.stack(yvs, 1), lam, eta
