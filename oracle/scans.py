"""numpy restatement of the standalone Moebius and affine scans (test oracle).

Arrays are [batch, steps, lanes] (lanes may be any trailing shape; it is
flattened); states are [batch, lanes]. Every function loops over time only and
is vectorised over (batch, lanes), so the headline shape (8, 4096, 2048) runs in
about a second in float64.

References (vaisakh-shaj/kalman-linear-attention):
  forward, per-step form   src/kla/ops/kernels/mps/lane_mobius_scan.metal:37-62, :64-90
  forward, prefix form     src/kla/ops/kla_ops.py:76-116 (_mobius_combine_tracenorm),
                           :244-251 (leaves, scan, apply to lam0);
                           src/kla/ops/kernels/triton/tiled_mobius_scan.py:44-111
  Moebius backward         src/kla/ops/kernels/triton/tiled_mobius_scan.py:266-279
  affine forward/backward  src/kla/ops/kernels/triton/tiled_mobius_scan.py:161-203, :282-298,
                           :247-254 (_reverse_affine)
"""

from __future__ import annotations

import numpy as np

EPS = 1e-12  # kla_ops.py:43


def _seq(x, dtype):
    x = np.asarray(x, dtype=dtype)
    return x.reshape(x.shape[0], x.shape[1], -1)


def _state(x, like, fill, dtype):
    if x is None:
        return np.full((like.shape[0], like.shape[2]), fill, dtype=dtype)
    return np.asarray(x, dtype=dtype).reshape(like.shape[0], like.shape[2])


# --------------------------------------------------------------------- Moebius


def mobius_scan_fwd(A, B, C, D=None, lam0=None, dtype=np.float64):
    """lam_t = (A_t lam_{t-1} + B_t) / max(C_t lam_{t-1} + D_t, EPS), lam_{-1} = lam0 (default 1).

    Per-step application (lane_mobius_scan.metal:37-62). Mathematically equal to
    the reference's prefix form (see :func:`mobius_scan_fwd_prefix`).
    """
    A, B, C = (_seq(x, dtype) for x in (A, B, C))
    D = np.ones_like(A) if D is None else _seq(D, dtype)
    x = _state(lam0, A, 1.0, dtype).copy()
    lam = np.empty_like(A)
    for t in range(A.shape[1]):
        x = (A[:, t] * x + B[:, t]) / np.maximum(C[:, t] * x + D[:, t], EPS)
        lam[:, t] = x
    return lam


def mobius_combine_tracenorm(left, right):
    """R.L / max(tr(R.L), EPS) for 2x2 maps stored as 4-tuples (kla_ops.py:76-116)."""
    a1, b1, c1, d1 = left
    a2, b2, c2, d2 = right
    a = a2 * a1 + b2 * c1
    b = a2 * b1 + b2 * d1
    c = c2 * a1 + d2 * c1
    d = c2 * b1 + d2 * d1
    inv = 1.0 / np.maximum(a + d, EPS)
    return a * inv, b * inv, c * inv, d * inv


def mobius_scan_fwd_prefix(A, B, C, D=None, lam0=None, dtype=np.float64):
    """The reference's form: trace-normalised inclusive prefix products, applied to lam0.

    kla_ops.py:244-251 / tiled_mobius_scan.py:44-111:
    lam_t = (pA lam0 + pB) / max(pC lam0 + pD, EPS), (pA..pD) = prefix_t.
    """
    A, B, C = (_seq(x, dtype) for x in (A, B, C))
    D = np.ones_like(A) if D is None else _seq(D, dtype)
    l0 = _state(lam0, A, 1.0, dtype)
    acc = None
    lam = np.empty_like(A)
    for t in range(A.shape[1]):
        leaf = (A[:, t], B[:, t], C[:, t], D[:, t])
        acc = leaf if acc is None else mobius_combine_tracenorm(acc, leaf)
        pA, pB, pC, pD = acc
        lam[:, t] = (pA * l0 + pB) / np.maximum(pC * l0 + pD, EPS)
    return lam


def mobius_scan_bwd(dlam, A, B, C, D=None, lam0=None, lam=None, dtype=np.float64):
    """Exact adjoint of :func:`mobius_scan_fwd` (tiled_mobius_scan.py:266-279).

    lam_prev = [lam0, lam_0..lam_{T-2}];  den = max(C lam_prev + D, EPS);
    gain = (A D - B C) / den^2;  nu_t = dlam_t + gain_{t+1} nu_{t+1};
    dA = nu lam_prev / den, dB = nu / den, dC = -nu lam lam_prev / den,
    dD = -nu lam / den, dlam0 = nu_0 gain_0.
    Returns (dA, dB, dC, dD, dlam0); dD is None when D is None.
    """
    has_d = D is not None
    A, B, C, dlam = (_seq(x, dtype) for x in (A, B, C, dlam))
    D = np.ones_like(A) if D is None else _seq(D, dtype)
    l0 = _state(lam0, A, 1.0, dtype)
    lam = mobius_scan_fwd(A, B, C, D, l0, dtype) if lam is None else _seq(lam, dtype)
    T = A.shape[1]
    lam_prev = np.concatenate([l0[:, None], lam[:, :-1]], axis=1)
    den = np.maximum(C * lam_prev + D, EPS)
    gain = (A * D - B * C) / (den * den)
    nu = np.empty_like(A)
    acc = np.zeros_like(l0)
    for t in range(T - 1, -1, -1):
        acc = dlam[:, t] + (gain[:, t + 1] * acc if t + 1 < T else 0.0)
        nu[:, t] = acc
    q = nu / den
    dA = q * lam_prev
    dB = q
    dC = -q * lam * lam_prev
    dD = -q * lam if has_d else None
    dlam0 = nu[:, 0] * gain[:, 0] if T > 0 else np.zeros_like(l0)
    return dA, dB, dC, dD, dlam0


# ---------------------------------------------------------------------- affine


def affine_scan_fwd(g, u, h0=None, dtype=np.float64):
    """h_t = g_t h_{t-1} + u_t, h_{-1} = h0 (default 0) (tiled_mobius_scan.py:161-203)."""
    g, u = _seq(g, dtype), _seq(u, dtype)
    x = _state(h0, g, 0.0, dtype).copy()
    h = np.empty_like(g)
    for t in range(g.shape[1]):
        x = g[:, t] * x + u[:, t]
        h[:, t] = x
    return h


def affine_scan_bwd(dh, g, h, h0=None, dtype=np.float64):
    """Exact adjoint of :func:`affine_scan_fwd` (tiled_mobius_scan.py:291-298).

    mu_t = dh_t + g_{t+1} mu_{t+1};  dg_t = mu_t h_{t-1} (h_{-1} = h0);  du = mu;
    dh0 = g_0 mu_0. ``h`` is the forward's output. Returns (dg, du, dh0).
    """
    dh, g, h = _seq(dh, dtype), _seq(g, dtype), _seq(h, dtype)
    x0 = _state(h0, g, 0.0, dtype)
    T = g.shape[1]
    mu = np.empty_like(g)
    acc = np.zeros_like(x0)
    for t in range(T - 1, -1, -1):
        acc = dh[:, t] + (g[:, t + 1] * acc if t + 1 < T else 0.0)
        mu[:, t] = acc
    h_prev = np.concatenate([x0[:, None], h[:, :-1]], axis=1)
    dg = mu * h_prev
    dh0 = g[:, 0] * mu[:, 0] if T > 0 else np.zeros_like(x0)
    return dg, mu.copy(), dh0
