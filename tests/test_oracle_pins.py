"""Pins of the CPU oracle (oracle/) against mathematics it does not share code with.

The reference ships no golden vectors for the scan path, so every oracle
function is pinned here by something independent of its own formula:

* Moebius forward    constant-leaf fixed point (root of C x^2 + (D - A) x - B = 0);
                     the C = 0 reduction to an affine recurrence with a closed form;
                     identity leaves; KLA leaves against the textbook covariance-form
                     Kalman filter; the reference's trace-normalised prefix form.
* Moebius backward   central finite differences (float64); torch autograd through the
                     doubling-scan restatement (no hand-written adjoint involved).
* affine forward     closed forms for constant g, g = 1 (cumsum) and g = 0.
* affine backward    finite differences; the g = 1 closed form (reverse cumsum).
* KLA scan           sequential information form vs covariance-form filter; the scalar
                     steady state (closed-form root of the stationary Riccati equation);
                     the torch doubling restatement vs the sequential one; gradcheck;
                     the torch stepwise restatement vs the sequential one, gradcheck,
                     and a held zero precision.
* trace-norm combine the invariants of reference tests/test_mobius_impl.py:116-146.

Each pin is a function returning an error measure, and ``test_planted_mistakes``
swaps a plausible mistake into the oracle (an operand swap, a dropped term, a
wrong sign, an off-by-one) and checks that some pin then fails.
"""

import numpy as np
import pytest
import torch

from oracle import kla as okla
from oracle import scans, torch_ref

# ----------------------------------------------------------------- inputs


def _mobius_leaves(B, T, N, seed):
    r = np.random.default_rng(seed)
    A = np.exp(-np.log1p(np.exp(r.standard_normal((B, T, N)))))
    Bm = np.log1p(np.exp(r.standard_normal((B, T, N))))
    C = np.log1p(np.exp(r.standard_normal((B, T, N))))
    D = 0.5 + r.random((B, T, N))
    lam0 = 0.2 + r.random((B, N))
    return A, Bm, C, D, lam0


def _kla_inputs(B, L, M, S, seed, dtype=np.float64):
    r = np.random.default_rng(seed)
    v = r.standard_normal((B, L, M))
    lambda_v = r.random((B, L, M)) + 0.5
    k = r.standard_normal((B, L, S)) * 0.5
    q = r.standard_normal((B, L, S)) * 0.5
    a = r.random((M, S)) * 0.5 + 0.4
    p = r.random((M, S)) * 0.05 + 0.01
    return tuple(x.astype(dtype) for x in (v, lambda_v, k, q, a, p))


def _rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-300))


# ---------------------------------------------------------- pin functions
# Each takes the implementation under test and returns an error (0 = exact).


def pin_mobius_fixed_point(fwd):
    """Constant leaf [[A,B],[C,D]] (entries > 0): lam_t -> the positive root of
    C x^2 + (D - A) x - B = 0, from any positive start."""
    A, Bm, C, D = 0.7, 0.3, 0.4, 1.2
    T = 400
    leaf = lambda v: np.full((1, T, 1), v)  # noqa: E731
    lam = fwd(leaf(A), leaf(Bm), leaf(C), leaf(D), np.array([[5.0]]))
    star = ((A - D) + np.sqrt((A - D) ** 2 + 4 * Bm * C)) / (2 * C)
    return abs(lam[0, -1, 0] - star) / star


def pin_mobius_affine_reduction(fwd):
    """C = 0: lam_t = g lam_{t-1} + u with g = A/D, u = B/D; constant g, u has the
    closed form g^(t+1) lam0 + u (1 - g^(t+1)) / (1 - g)."""
    T = 37
    A, Bm, D = 0.9, 0.25, 1.5
    g, u = A / D, Bm / D
    ones = np.ones((2, T, 3))
    lam0 = np.array([[0.5, 1.0, 2.0], [3.0, 0.1, 7.0]])
    lam = fwd(A * ones, Bm * ones, 0 * ones, D * ones, lam0)
    t = np.arange(1, T + 1)[None, :, None]
    want = g**t * lam0[:, None, :] + u * (1 - g**t) / (1 - g)
    return _rel(lam, want)


def pin_mobius_identity(fwd):
    """Identity leaves keep lam0."""
    ones, zeros = np.ones((2, 9, 4)), np.zeros((2, 9, 4))
    lam0 = np.arange(1, 9, dtype=np.float64).reshape(2, 4)
    lam = fwd(ones, zeros, zeros, ones, lam0)
    return _rel(lam, np.broadcast_to(lam0[:, None, :], lam.shape))


def pin_mobius_kalman(fwd):
    """KLA leaves A = (1 + p phi)/a^2, B = phi, C = p/a^2, D = 1 reproduce the
    posterior precision 1/P of the textbook covariance-form filter."""
    v, lambda_v, k, q, a, p = _kla_inputs(2, 30, 3, 2, seed=5)
    phi = lambda_v[..., None] * (k * k)[:, :, None, :]
    a2 = (a * a)[None, None]
    A = (1 + p * phi) / a2
    C = np.broadcast_to(p / a2, phi.shape)
    lam0 = np.full((2, 3 * 2), 1.7)
    lam = fwd(A.reshape(2, 30, -1), phi.reshape(2, 30, -1), C.reshape(2, 30, -1),
              np.ones((2, 30, 6)), lam0)
    # Covariance form, per step (P0 = 1/lam0), written out with no Moebius algebra.
    P = 1.0 / lam0.reshape(2, 3, 2)
    out = np.empty((2, 30, 3, 2))
    for t in range(30):
        P_pred = a**2 * P + p
        kk = k[:, t, None, :]
        R = 1.0 / lambda_v[:, t, :, None]
        K = P_pred * kk / (kk * kk * P_pred + R)
        P = (1 - K * kk) * P_pred
        out[:, t] = 1.0 / P
    return _rel(lam, out.reshape(2, 30, -1))


def pin_affine_closed_forms(fwd):
    T = 40
    ones = np.ones((2, T, 3))
    h0 = np.array([[0.3, -1.0, 2.0], [0.0, 4.0, -0.5]])
    t = np.arange(1, T + 1)[None, :, None]
    err = 0.0
    g, u = 0.8, 0.6
    err = max(err, _rel(fwd(g * ones, u * ones, h0), g**t * h0[:, None, :] + u * (1 - g**t) / (1 - g)))
    uu = np.random.default_rng(0).standard_normal((2, T, 3))
    err = max(err, _rel(fwd(ones, uu, h0), h0[:, None, :] + np.cumsum(uu, axis=1)))
    err = max(err, _rel(fwd(0 * ones, uu, h0), uu))
    return err


def _fd_grad(f, x, eps=1e-6):
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp, xm = x.copy(), x.copy()
        xp[i] += eps
        xm[i] -= eps
        g[i] = (f(xp) - f(xm)) / (2 * eps)
    return g


def pin_mobius_bwd_fd(bwd):
    """Every Moebius gradient against central differences of sum(dlam * lam)."""
    A, Bm, C, D, lam0 = _mobius_leaves(2, 6, 2, seed=11)
    dlam = np.random.default_rng(12).standard_normal(A.shape)
    ins = [A, Bm, C, D, lam0]

    def loss(i, x):
        args = list(ins)
        args[i] = x
        return float(np.sum(dlam * scans.mobius_scan_fwd(*args)))

    got = bwd(dlam, A, Bm, C, D, lam0, scans.mobius_scan_fwd(A, Bm, C, D, lam0))
    return max(_rel(got[i], _fd_grad(lambda x, i=i: loss(i, x), ins[i])) for i in range(5))


def pin_mobius_bwd_autograd(bwd):
    """Against torch autograd through the reference's doubling-scan form (D = None)."""
    A, Bm, C, _, lam0 = _mobius_leaves(2, 33, 3, seed=13)
    dlam = np.random.default_rng(14).standard_normal(A.shape)
    ts = [torch.tensor(x, requires_grad=True) for x in (A, Bm, C, lam0)]
    lam = torch_ref.mobius_scan(ts[0], ts[1], ts[2], None, ts[3])
    lam.backward(torch.tensor(dlam))
    got = bwd(dlam, A, Bm, C, None, lam0, scans.mobius_scan_fwd(A, Bm, C, None, lam0))
    want = [t.grad.numpy() for t in ts]
    return max(_rel(got[i], want[j]) for i, j in ((0, 0), (1, 1), (2, 2), (4, 3)))


def pin_affine_bwd_fd(bwd):
    r = np.random.default_rng(21)
    g = r.random((2, 7, 3)) * 0.9 + 0.05
    u = r.standard_normal((2, 7, 3))
    h0 = r.standard_normal((2, 3))
    dh = r.standard_normal((2, 7, 3))
    h = scans.affine_scan_fwd(g, u, h0)
    dg, du, dh0 = bwd(dh, g, h, h0)
    fg = _fd_grad(lambda x: float(np.sum(dh * scans.affine_scan_fwd(x, u, h0))), g)
    fu = _fd_grad(lambda x: float(np.sum(dh * scans.affine_scan_fwd(g, x, h0))), u)
    f0 = _fd_grad(lambda x: float(np.sum(dh * scans.affine_scan_fwd(g, u, x))), h0)
    return max(_rel(dg, fg), _rel(du, fu), _rel(dh0, f0))


def pin_affine_bwd_cumsum(bwd):
    """g = 1: mu_t = sum_{s >= t} dh_s, dg_t = mu_t h_{t-1}, dh0 = mu_0."""
    r = np.random.default_rng(22)
    T = 25
    g = np.ones((2, T, 3))
    u = r.standard_normal((2, T, 3))
    h0 = r.standard_normal((2, 3))
    dh = r.standard_normal((2, T, 3))
    h = h0[:, None, :] + np.cumsum(u, axis=1)
    mu = np.flip(np.cumsum(np.flip(dh, 1), 1), 1)
    h_prev = np.concatenate([h0[:, None, :], h[:, :-1]], axis=1)
    dg, du, dh0 = bwd(dh, g, h, h0)
    return max(_rel(du, mu), _rel(dg, mu * h_prev), _rel(dh0, mu[:, 0]))


def pin_kla_covariance(seq):
    """Sequential information form vs the covariance-form filter (independent algebra)."""
    v, lambda_v, k, q, a, p = _kla_inputs(2, 40, 4, 3, seed=31)
    lam0 = np.full((2, 4, 3), 2.0)
    eta0 = np.random.default_rng(32).standard_normal((2, 4, 3))
    got = seq(v, lambda_v, k, q, a, p, lam0, eta0)
    want = okla.kalman_filter_covariance(v, lambda_v, k, q, a, p, lam0, eta0)
    return max(_rel(x, w) for x, w in zip(got, want))


def pin_kla_steady_state(seq):
    """Constant phi = Lambda^v k^2: lam converges to the positive root of the
    stationary information Riccati equation p x^2 + (a^2 - 1 - p phi) x - phi a^2 = 0."""
    L, M, S = 300, 2, 2
    a = np.array([[0.5, 0.9], [0.7, 0.95]])
    p = np.array([[0.05, 0.01], [0.2, 0.003]])
    k = np.full((1, L, S), 0.8)
    lambda_v = np.full((1, L, M), 1.5)
    v = np.zeros((1, L, M))
    q = np.ones((1, L, S))
    _, _, lam, _ = seq(v, lambda_v, k, q, a, p)
    phi = 1.5 * 0.8**2
    bq = a**2 - 1 - p * phi
    star = (-bq + np.sqrt(bq**2 + 4 * p * phi * a**2)) / (2 * p)
    return _rel(lam[0], star)


# ------------------------------------------------------------------ tests


def test_mobius_forward_pins():
    assert pin_mobius_fixed_point(scans.mobius_scan_fwd) < 1e-12
    assert pin_mobius_affine_reduction(scans.mobius_scan_fwd) < 1e-12
    assert pin_mobius_identity(scans.mobius_scan_fwd) == 0.0
    assert pin_mobius_kalman(scans.mobius_scan_fwd) < 1e-12


def test_mobius_prefix_form_matches_per_step():
    """The reference's trace-normalised prefix-product form (kla_ops.py:244-251)."""
    A, Bm, C, D, lam0 = _mobius_leaves(3, 64, 5, seed=3)
    assert _rel(scans.mobius_scan_fwd_prefix(A, Bm, C, D, lam0), scans.mobius_scan_fwd(A, Bm, C, D, lam0)) < 1e-12
    assert pin_mobius_fixed_point(scans.mobius_scan_fwd_prefix) < 1e-12
    assert pin_mobius_kalman(scans.mobius_scan_fwd_prefix) < 1e-12


def test_mobius_backward_pins():
    assert pin_mobius_bwd_fd(scans.mobius_scan_bwd) < 1e-6
    assert pin_mobius_bwd_autograd(scans.mobius_scan_bwd) < 1e-12


def test_affine_pins():
    assert pin_affine_closed_forms(scans.affine_scan_fwd) < 1e-12
    assert pin_affine_bwd_fd(scans.affine_scan_bwd) < 1e-7
    assert pin_affine_bwd_cumsum(scans.affine_scan_bwd) < 1e-12


def test_affine_torch_restatement():
    r = np.random.default_rng(4)
    g, u, h0 = r.random((2, 50, 3)), r.standard_normal((2, 50, 3)), r.standard_normal((2, 3))
    h = torch_ref.affine_scan(torch.tensor(g), torch.tensor(u), torch.tensor(h0))
    assert _rel(h.numpy(), scans.affine_scan_fwd(g, u, h0)) < 1e-12


def test_kla_pins():
    assert pin_kla_covariance(okla.kla_scan_sequential) < 1e-10
    assert pin_kla_steady_state(okla.kla_scan_sequential) < 1e-10
    # The covariance filter itself satisfies the same closed form.
    cov = lambda *a: okla.kalman_filter_covariance(*a)  # noqa: E731
    assert pin_kla_steady_state(cov) < 1e-10


@pytest.mark.parametrize("decode_from_prior", [False, True])
def test_torch_restatement_matches_sequential(decode_from_prior):
    """oracle.torch_ref.kla_scan_torch (doubling scans of trace-normalised products,
    the reference's CPU algorithm) against the sequential float64 filter."""
    args = _kla_inputs(2, 64, 5, 3, seed=41)
    lam0 = np.full((2, 5, 3), 1.3)
    eta0 = np.random.default_rng(42).standard_normal((2, 5, 3))
    want = okla.kla_scan_sequential(*args, lam0, eta0, decode_from_prior=decode_from_prior)
    for impl in ("linear", "log"):
        got = torch_ref.kla_scan_torch(*(torch.tensor(x) for x in args), torch.tensor(lam0), torch.tensor(eta0),
                                       decode_from_prior=decode_from_prior, mobius_impl=impl)
        for x, w in zip(got, want):
            assert _rel(x.numpy(), w) < 1e-9, impl


@pytest.mark.parametrize("decode_from_prior", [False, True])
def test_stepwise_restatement_matches_sequential(decode_from_prior):
    """oracle.torch_ref.kla_scan_stepwise (kla_scan_torch's leaves applied one step
    at a time, in torch) against the sequential float64 filter, with k away from
    zero so that filter's phi floor never acts; and its gradients by central
    differences."""
    args = _kla_inputs(2, 64, 5, 3, seed=43)
    lam0 = np.full((2, 5, 3), 0.9)
    eta0 = np.random.default_rng(44).standard_normal((2, 5, 3))
    want = okla.kla_scan_sequential(*args, lam0, eta0, decode_from_prior=decode_from_prior)
    got = torch_ref.kla_scan_stepwise(*(torch.tensor(x) for x in args), torch.tensor(lam0), torch.tensor(eta0),
                                      decode_from_prior=decode_from_prior)
    for x, w in zip(got, want):
        assert _rel(x.numpy(), w) < 1e-12
    r = np.random.default_rng(52)
    B, L, M, S = 1, 6, 2, 2
    ins = (r.standard_normal((B, L, M)), r.random((B, L, M)) + 0.5, r.standard_normal((B, L, S)) * 0.5,
           r.standard_normal((B, L, S)) * 0.5, r.random((M, S)) * 0.4 + 0.5, r.random((M, S)) * 0.04 + 0.02,
           r.random((B, M, S)) + 0.5, r.standard_normal((B, M, S)))
    ts = tuple(torch.tensor(x, requires_grad=True) for x in ins)
    assert torch.autograd.gradcheck(
        lambda *a: torch_ref.kla_scan_stepwise(*a, decode_from_prior=decode_from_prior), ts,
        eps=1e-6, atol=1e-5, rtol=1e-3)


def test_stepwise_holds_a_zero_precision():
    """From lam0 = 0 with k = 0 the precision stays exactly 0 (phi = 0, lam idn = 0)
    and var = 1/max(lam, EPS) is clamped; the first step with k != 0 gives
    lam = phi = lambda_v k^2 exactly, the filter's update from an uninformative
    prior."""
    B, L, M, S = 1, 5, 2, 3
    r = np.random.default_rng(53)
    v, lv = torch.tensor(r.standard_normal((B, L, M))), torch.tensor(r.random((B, L, M)) + 0.5)
    k = torch.zeros(B, L, S, dtype=torch.float64)
    k[:, 3:] = torch.tensor(r.standard_normal((B, 2, S)))
    q = torch.tensor(r.standard_normal((B, L, S)))
    a, p = torch.tensor(r.random((M, S)) * 0.4 + 0.5), torch.tensor(r.random((M, S)) * 0.04 + 0.02)
    zero = torch.zeros(B, M, S, dtype=torch.float64)
    _, y_var, _, _ = torch_ref.kla_scan_stepwise(v, lv, k, q, a, p, zero, zero.clone())
    assert torch.allclose(y_var[:, :3], (q[:, :3] ** 2).sum(-1).unsqueeze(-1).expand(B, 3, M) / torch_ref.EPS)
    _, _, lam, _ = torch_ref.kla_scan_stepwise(v[:, :4], lv[:, :4], k[:, :4], q[:, :4], a, p, zero, zero.clone())
    assert torch.equal(lam, lv[:, 3].unsqueeze(-1) * (k[:, 3] ** 2).unsqueeze(-2))


def test_doubling_matches_sequential_scan():
    r = np.random.default_rng(7)
    xs = tuple(torch.tensor(r.random((2, 37, 3)) + 0.1) for _ in range(4))
    d = torch_ref.doubling_scan(torch_ref.mobius_combine_tracenorm, xs)
    s = torch_ref.sequential_scan(torch_ref.mobius_combine_tracenorm, xs)
    for a, b in zip(d, s):
        assert _rel(a.numpy(), b.numpy()) < 1e-12


def test_gradcheck_torch_restatement():
    """Central differences vs autograd through the torch restatement (reference
    tests/test_gradcheck.py:60-109 in spirit): pins every gradient of the full scan."""
    r = np.random.default_rng(51)
    B, L, M, S = 1, 6, 2, 2
    ins = (r.standard_normal((B, L, M)), r.random((B, L, M)) + 0.5, r.standard_normal((B, L, S)) * 0.5,
           r.standard_normal((B, L, S)) * 0.5, r.random((M, S)) * 0.4 + 0.5, r.random((M, S)) * 0.04 + 0.02)
    ts = tuple(torch.tensor(x, requires_grad=True) for x in ins)
    lam0 = torch.full((B, M, S), 2.0, dtype=torch.float64)
    eta0 = torch.full((B, M, S), 0.3, dtype=torch.float64)

    def f(*a):
        y, y_var, lam, eta = torch_ref.kla_scan_torch(*a, lam0, eta0)
        return y, y_var, lam, eta

    assert torch.autograd.gradcheck(f, ts, eps=1e-6, atol=1e-5, rtol=1e-3)


def test_tracenorm_invariants():
    """After any number of compositions: A, D in [0, 1] with A + D = 1, entries >= 0,
    B C <= 1/4 (reference tests/test_mobius_impl.py:116-146)."""
    g = torch.Generator().manual_seed(0)
    scale = torch.logspace(-6, 6, 64, dtype=torch.float64).unsqueeze(-1)
    acc = tuple((torch.rand(64, 4, generator=g, dtype=torch.float64) + 1e-3) * scale for _ in range(4))
    for _ in range(20):
        acc = torch_ref.mobius_combine_tracenorm(acc, acc)
        A, Bm, Cm, D = acc
        assert torch.stack(acc).isfinite().all()
        assert (torch.stack(acc) >= 0).all()
        assert (Bm * Cm <= 0.25 + 1e-12).all()
    assert torch.allclose(acc[0] + acc[3], torch.ones_like(acc[0]))


# ------------------------------------------------------- planted mistakes


def _mutant_mobius_swap_bc(A, B, C, D=None, lam0=None, dtype=np.float64):
    return scans.mobius_scan_fwd(A, C, B, D, lam0, dtype)


def _mutant_mobius_off_by_one(A, B, C, D=None, lam0=None, dtype=np.float64):
    lam = scans.mobius_scan_fwd(A, B, C, D, lam0, dtype)
    # Publishes the prior instead of the posterior: lam_{t-1} at t.
    l0 = np.ones_like(lam[:, 0]) if lam0 is None else np.asarray(lam0, dtype).reshape(lam[:, 0].shape)
    return np.concatenate([l0[:, None], lam[:, :-1]], axis=1)


def _mutant_mobius_bwd_no_gain(dlam, A, B, C, D=None, lam0=None, lam=None, dtype=np.float64):
    # Drops the carried term: nu_t = dlam_t.
    out = list(scans.mobius_scan_bwd(dlam, A, B, C, D, lam0, lam, dtype))
    A_, B_, C_, dl = (np.asarray(x, dtype) for x in (A, B, C, dlam))
    D_ = np.ones_like(A_) if D is None else np.asarray(D, dtype)
    l0 = np.ones_like(A_[:, 0]) if lam0 is None else np.asarray(lam0, dtype)
    lm = scans.mobius_scan_fwd(A_, B_, C_, D_, l0)
    lp = np.concatenate([l0[:, None], lm[:, :-1]], axis=1)
    den = np.maximum(C_ * lp + D_, 1e-12)
    qv = dl / den
    out[0], out[1] = qv * lp, qv
    return tuple(out)


def _mutant_mobius_bwd_sign(dlam, A, B, C, D=None, lam0=None, lam=None, dtype=np.float64):
    dA, dB, dC, dD, dl0 = scans.mobius_scan_bwd(dlam, A, B, C, D, lam0, lam, dtype)
    return dA, dB, -dC, dD, dl0


def _mutant_affine_transpose(g, u, h0=None, dtype=np.float64):
    return scans.affine_scan_fwd(u, g, h0, dtype)


def _mutant_affine_bwd_shift(dh, g, h, h0=None, dtype=np.float64):
    # Off by one step: dg_t = mu_t h_t instead of mu_t h_{t-1}.
    dg, du, dh0 = scans.affine_scan_bwd(dh, g, h, h0, dtype)
    return du * np.asarray(h, dtype), du, dh0


def _mutant_kla_drop_value_precision(v, lambda_v, k, q, a, p, lam0=None, eta0=None, decode_from_prior=False):
    # Dropped term: r = v k instead of (v Lambda^v) k.
    return okla.kla_scan_sequential(np.asarray(v) / np.asarray(lambda_v), lambda_v, k, q, a, p, lam0, eta0,
                                    decode_from_prior)


@pytest.mark.parametrize(
    "pin, mutant",
    [
        (pin_mobius_fixed_point, _mutant_mobius_swap_bc),
        (pin_mobius_kalman, _mutant_mobius_swap_bc),
        (pin_mobius_affine_reduction, _mutant_mobius_off_by_one),
        (pin_mobius_kalman, _mutant_mobius_off_by_one),
        (pin_mobius_bwd_fd, _mutant_mobius_bwd_no_gain),
        (pin_mobius_bwd_autograd, _mutant_mobius_bwd_no_gain),
        (pin_mobius_bwd_fd, _mutant_mobius_bwd_sign),
        (pin_affine_closed_forms, _mutant_affine_transpose),
        (pin_affine_bwd_fd, _mutant_affine_bwd_shift),
        (pin_affine_bwd_cumsum, _mutant_affine_bwd_shift),
        (pin_kla_covariance, _mutant_kla_drop_value_precision),
    ],
)
def test_planted_mistakes(pin, mutant):
    """A pin that cannot see a plausible mistake pins nothing."""
    assert pin(mutant) > 1e-3
