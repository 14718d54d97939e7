"""numpy float64 restatement of the full KLA scan (test oracle).

Shapes follow the reference (src/kla/ops/kla_ops.py:23-28):
    v, lambda_v [B, L, M];  k, q [B, L, S];  a, p [M, S];  state [B, M, S].

Two independent formulations of the same filter:

* :func:`kla_scan_sequential` -- the information form, one ``kla_step`` per
  token (kla_ops.py:293-331 stepped by kla_scan_reference, :334-362), with the
  reference's guards: p floored at P_MIN, a^2 at EPS, phi at EPS, the predict
  denominator at EPS, and var = 1/max(lam, EPS).
* :func:`kalman_filter_covariance` -- the textbook covariance form of the same
  per-(m, s) scalar model x_t = a x_{t-1} + w (Var p), v_t = k_t x_t + e
  (Var 1/lambda_v): P- = a^2 P + p, K = P- k / (k^2 P- + 1/lambda_v),
  mean = a mean + K (v - k a mean), P = (1 - K k) P-. It shares no algebra with
  the information form beyond the model, which is what makes it a pin.
"""

from __future__ import annotations

import numpy as np

EPS = 1e-12
P_MIN = 1e-12


def _f64(*xs):
    return tuple(None if x is None else np.asarray(x, dtype=np.float64) for x in xs)


def kla_scan_sequential(v, lambda_v, k, q, a, p, lam0=None, eta0=None, decode_from_prior=False):
    """Returns (y [B,L,M], y_var [B,L,M], lam_fin [B,M,S], eta_fin [B,M,S]).

    Restates kla_step (kla_ops.py:293-331) applied along the sequence
    (kla_scan_reference, kla_ops.py:334-362).
    """
    v, lambda_v, k, q, a, p, lam0, eta0 = _f64(v, lambda_v, k, q, a, p, lam0, eta0)
    Bn, L, M = v.shape
    S = k.shape[2]
    lam = np.ones((Bn, M, S)) if lam0 is None else lam0.copy()
    eta = np.zeros((Bn, M, S)) if eta0 is None else eta0.copy()
    a_ = a[None]
    p_ = np.maximum(p, P_MIN)[None]
    a2 = np.maximum(a_ * a_, EPS)
    y = np.empty((Bn, L, M))
    y_var = np.empty((Bn, L, M))
    for t in range(L):
        phi = np.maximum(lambda_v[:, t, :, None] * (k[:, t, None, :] ** 2), EPS)
        r = (v[:, t] * lambda_v[:, t])[:, :, None] * k[:, t, None, :]
        denom = np.maximum(a2 + p_ * lam, EPS)
        lam = lam / denom + phi
        eta = (a_ / denom) * eta + r
        var = 1.0 / np.maximum(lam, EPS)
        mean = eta * var
        if decode_from_prior:
            mean = a_ * mean
            var = a2 * var + p_
        y[:, t] = np.einsum("bms,bs->bm", mean, q[:, t])
        y_var[:, t] = np.einsum("bms,bs->bm", var, q[:, t] ** 2)
    return y, y_var, lam, eta


def kalman_filter_covariance(v, lambda_v, k, q, a, p, lam0=None, eta0=None):
    """Textbook covariance-form filter; returns (y, y_var, lam_fin, eta_fin).

    Valid where no guard of the information form binds (p > 0, a != 0, phi > 0);
    the state comes back in information form (lam = 1/P, eta = mean/P).
    """
    v, lambda_v, k, q, a, p, lam0, eta0 = _f64(v, lambda_v, k, q, a, p, lam0, eta0)
    Bn, L, M = v.shape
    S = k.shape[2]
    P = np.ones((Bn, M, S)) if lam0 is None else 1.0 / lam0
    mean = np.zeros((Bn, M, S)) if eta0 is None else eta0 * P
    y = np.empty((Bn, L, M))
    y_var = np.empty((Bn, L, M))
    for t in range(L):
        kk = k[:, t, None, :]
        obs_var = 1.0 / lambda_v[:, t, :, None]
        m_pred = a[None] * mean
        P_pred = a[None] ** 2 * P + p[None]
        K = P_pred * kk / (kk * kk * P_pred + obs_var)
        mean = m_pred + K * (v[:, t, :, None] - kk * m_pred)
        P = (1.0 - K * kk) * P_pred
        y[:, t] = np.einsum("bms,bs->bm", mean, q[:, t])
        y_var[:, t] = np.einsum("bms,bs->bm", P, q[:, t] ** 2)
    return y, y_var, 1.0 / P, mean / P
