"""The algebra of the time-split forward, in float64 on the CPU.

The fused kernels' time split (csrc/fused_kla.hpp fused_chunk_map_kernel,
chunk_starts_kernel) rests on one identity: in homogeneous coordinates
lam = N / D, eta = W / D, a filter step (reference kla_step,
src/kla/ops/kla_ops.py:293-331, with phi unfloored as in the scan)

    N' = A N + phi D,   D' = C N + D,   W' = g W + r D'
    A = (1 + p phi) / a^2,  C = p / a^2,  g = a / a^2

is linear, so a chunk of steps composes to one 3x3 map [[n0, n1, 0],
[d0, d1, 0], [w0, w1, w2]], and the state entering every chunk follows from
the maps alone. Here the maps are built exactly as the kernel builds them
(leaf times map, rescaled by a power of two after every step) and chained as
chunk_starts_kernel chains them, and the chunk-boundary states are compared
with the float64 sequential filter (oracle.kla.kla_scan_sequential), for
random inputs, with and without an initial state. A plausible slip (W taking
the pre-step denominator D instead of D') fails these checks.
"""

import numpy as np
import pytest

from oracle import kla as okla


def _inputs(B, L, M, S, seed):
    r = np.random.default_rng(seed)
    return (r.standard_normal((B, L, M)), r.random((B, L, M)) * 3 + 0.05, r.standard_normal((B, L, S)) * 0.6,
            r.standard_normal((B, L, S)), r.random((M, S)) * 0.5 + 0.45, r.random((M, S)) * 0.05 + 0.01)


def chunk_maps(v, lv, k, a, p):
    """[B, M, S, 7] maps of whole sequences v, lv [B, T, M], k [B, T, S]."""
    B, T, M = v.shape
    S = k.shape[2]
    p = np.maximum(p, okla.P_MIN)
    a2 = np.maximum(a * a, okla.EPS)
    C, g = p / a2, a / a2
    n0, n1, d0, d1 = (np.full((B, M, S), x) for x in (1.0, 0.0, 0.0, 1.0))
    w0, w1, w2 = np.zeros((B, M, S)), np.zeros((B, M, S)), np.ones((B, M, S))
    for t in range(T):
        phi = lv[:, t, :, None] * k[:, t, None, :] ** 2
        r = (v[:, t] * lv[:, t])[:, :, None] * k[:, t, None, :]
        A = (1 + p * phi) / a2
        e0, e1 = C * n0 + d0, C * n1 + d1
        m0, m1 = A * n0 + phi * d0, A * n1 + phi * d1
        x0, x1, x2 = g * w0 + r * e0, g * w1 + r * e1, g * w2
        scale = 2.0 ** -np.frexp(m0 + e1)[1]
        n0, n1, d0, d1, w0, w1, w2 = (z * scale for z in (m0, m1, e0, e1, x0, x1, x2))
    return np.stack([n0, n1, d0, d1, w0, w1, w2], -1)


# chunk_starts_kernel guards a map's denominator against zero and subnormals only
# (FLT_MIN): a rescaled map's d1 can be a normal number far below EPS.
DEN_MIN = float(np.finfo(np.float32).tiny)


def chain(maps, lam0, eta0, den_min=DEN_MIN):
    """States entering each chunk: maps [B, nc, M, S, 7] -> lam, eta [B, nc, M, S]."""
    nc = maps.shape[1]
    lam, eta = lam0.copy(), eta0.copy()
    lams, etas = [], []
    for c in range(nc):
        lams.append(lam)
        etas.append(eta)
        n0, n1, d0, d1, w0, w1, w2 = np.moveaxis(maps[:, c], -1, 0)
        den = np.maximum(d0 * lam + d1, den_min)
        lam, eta = (n0 * lam + n1) / den, (w0 * lam + w1 + w2 * eta) / den
    return np.stack(lams, 1), np.stack(etas, 1), lam, eta


@pytest.mark.parametrize("B,L,M,S,nc", [(2, 96, 3, 4, 4), (1, 120, 2, 5, 8), (3, 64, 4, 2, 2)])
@pytest.mark.parametrize("with_state", [False, True])
def test_chunk_maps_reproduce_the_sequential_filter(B, L, M, S, nc, with_state):
    v, lv, k, q, a, p = _inputs(B, L, M, S, seed=B * L + nc)
    r = np.random.default_rng(1)
    lam0 = r.random((B, M, S)) * 2 + 0.3 if with_state else np.ones((B, M, S))
    eta0 = r.standard_normal((B, M, S)) if with_state else np.zeros((B, M, S))
    Lc = L // nc
    maps = np.stack([chunk_maps(v[:, c * Lc:(c + 1) * Lc], lv[:, c * Lc:(c + 1) * Lc], k[:, c * Lc:(c + 1) * Lc],
                                a, p) for c in range(nc)], 1)
    lams, etas, lam_fin, eta_fin = chain(maps, lam0, eta0)
    for c in range(nc + 1):
        _, _, want_l, want_e = okla.kla_scan_sequential(v[:, :c * Lc], lv[:, :c * Lc], k[:, :c * Lc],
                                                        q[:, :c * Lc], a, p, lam0, eta0)
        got_l = lams[:, c] if c < nc else lam_fin
        got_e = etas[:, c] if c < nc else eta_fin
        np.testing.assert_allclose(got_l, want_l, rtol=1e-12, atol=1e-12, err_msg=f"lam entering chunk {c}")
        np.testing.assert_allclose(got_e, want_e, rtol=1e-11, atol=1e-11, err_msg=f"eta entering chunk {c}")


def test_dropping_the_coupling_term_is_caught():
    """The W row's r * D' term carries the information leaf; the same chain with
    r * D (the old denominator) misses the precision's effect on alpha and is far
    off: the check above would fail for it."""
    v, lv, k, q, a, p = _inputs(1, 40, 2, 3, seed=5)
    good = chunk_maps(v, lv, k, a, p)
    _, _, want_l, want_e = okla.kla_scan_sequential(v, lv, k, q, a, p)
    lam, eta = chain(good[:, None], np.ones((1, 2, 3)), np.zeros((1, 2, 3)))[2:]
    np.testing.assert_allclose(eta, want_e, rtol=1e-11, atol=1e-11)
    # A plausible slip: W' = g W + r D (pre-step denominator).
    B, T, M = v.shape
    a2 = np.maximum(a * a, okla.EPS)
    C, g = np.maximum(p, okla.P_MIN) / a2, a / a2
    n, d, w = np.ones((1, 2, 3)), np.ones((1, 2, 3)), np.zeros((1, 2, 3))
    for t in range(T):
        phi = lv[:, t, :, None] * k[:, t, None, :] ** 2
        r = (v[:, t] * lv[:, t])[:, :, None] * k[:, t, None, :]
        A = (1 + np.maximum(p, okla.P_MIN) * phi) / a2
        n, d, w = A * n + phi * d, C * n + d, g * w + r * d
    assert np.abs(w / d - want_e).max() > 1e-3


def test_cold_lane_over_a_whole_chunk_keeps_its_state():
    """lam0 = 0 under decay (a = 0.8, p = 0.03) with a lane whose phi is 4e-12 for the
    whole first chunk of 128 steps: the chunk's map, rescaled to a trace in
    [0.5, 1), has d1 below 1e-12 (a normal float32), and the state entering chunk 1
    is lam = n1 / d1 ~ 12. The chain follows the sequential filter (whose phi
    floor stays idle at this k); the same chain with its denominator floored at
    EPS (the slip this guards against) leaves lam far lower."""
    B, L, M, S, Lc = 1, 256, 2, 3, 128
    v, lv, k, q, _, _ = _inputs(B, L, M, S, seed=9)
    lv[:, :Lc] = 1.0
    k[:, :Lc, 0] = 2e-6   # phi = 4e-12: above the sequential filter's EPS floor
    a, p = np.full((M, S), 0.8), np.full((M, S), 0.03)
    lam0, eta0 = np.zeros((B, M, S)), np.zeros((B, M, S))
    maps = np.stack([chunk_maps(v[:, c * Lc:(c + 1) * Lc], lv[:, c * Lc:(c + 1) * Lc], k[:, c * Lc:(c + 1) * Lc],
                                a, p) for c in range(2)], 1)
    assert maps[0, 0, :, 0, 3].max() < 1e-12 < maps[0, 0, :, 0, 3].min() * 1e6, "d1 of the cold lane's map"
    _, _, want_l, want_e = okla.kla_scan_sequential(v[:, :Lc], lv[:, :Lc], k[:, :Lc], q[:, :Lc], a, p, lam0, eta0)
    _, _, fin_l, fin_e = okla.kla_scan_sequential(v, lv, k, q, a, p, lam0, eta0)
    assert want_l[0, 0, 0] > 1.0
    lams, etas, lam_fin, eta_fin = chain(maps, lam0, eta0)
    np.testing.assert_allclose(lams[:, 1], want_l, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(etas[:, 1], want_e, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(lam_fin, fin_l, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(eta_fin, fin_e, rtol=1e-9, atol=1e-12)
    bad = chain(maps, lam0, eta0, den_min=okla.EPS)[0][:, 1]
    assert abs(bad[0, 0, 0] - want_l[0, 0, 0]) > 0.5 * want_l[0, 0, 0]
