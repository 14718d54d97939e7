"""KLA scan ops and the backend dispatcher.

The KLA scan is a Kalman filter in information form, run independently on every
(channel m, state s) lane (reference src/kla/ops/kla_ops.py:1-32):

    predict   lam-_t = lam_{t-1} / (a^2 + p lam_{t-1})
    update    lam_t  = lam-_t + phi_t,       phi_t = Lambda^v_t k_t^2
    gain      alpha_t = a / (a^2 + p lam_{t-1})
    info      eta_t  = alpha_t eta_{t-1} + r_t,   r_t = (v_t Lambda^v_t) k_t
    read-out  y[m] = sum_s q[s] eta/lam,   y_var[m] = sum_s q[s]^2 / lam

Shapes: v, lambda_v [B, L, M]; k, q [B, L, S]; a, p [M, S]; state [B, M, S].

The precision recurrence is a Moebius map lam -> (A lam + B)/(C lam + D) with
leaf A = (1 + p phi)/a^2, B = phi, C = p/a^2, D = 1, scanned as trace-normalised
2x2 products; the information vector is a first-order affine recurrence.

Backends (``kla_scan(..., backend=...)``):
  torch          this module's pure-torch path (CPU or GPU)
  hip            MI355X kernels (see :mod:`kla.ops.hip_backend`): the fused scan
  hip_fused      pinned to the fused kernels (any d_state: groups of <= 256 lanes)
  hip_composed   pinned to the composed path (HIP scans + torch glue)
  triton*, cuda*, mps*  names kept from the reference registry for config
                 compatibility; their kernels are not part of this build and
                 they raise NotImplementedError naming a backend that works.
"""

from __future__ import annotations

import functools
from typing import NamedTuple, Optional

import torch

from kla.ops.scan import resolve_scan, sequential_scan  # noqa: F401

EPS = 1e-12
P_MIN = 1e-12  # floor on the process noise p


class KLAState(NamedTuple):
    """Filter state carried across calls: posterior precision and information vector."""

    lam: torch.Tensor  # [B, M, S]
    eta: torch.Tensor  # [B, M, S]


def init_state(batch: int, d_model: int, d_state: int, device=None, dtype=torch.float32) -> KLAState:
    """Standard-normal prior: precision 1, information 0 (reference kla_ops.py:54-61)."""
    return KLAState(
        lam=torch.ones(batch, d_model, d_state, device=device, dtype=dtype),
        eta=torch.zeros(batch, d_model, d_state, device=device, dtype=dtype),
    )


# --------------------------------------------------------------- combinators


def _mobius_combine_log(left, right):
    """Compose 2x2 maps held as (log A, log B, log C, log D) (reference kla_ops.py:64-73)."""
    la1, lb1, lc1, ld1 = left
    la2, lb2, lc2, ld2 = right
    return (
        torch.logaddexp(la2 + la1, lb2 + lc1),
        torch.logaddexp(la2 + lb1, lb2 + ld1),
        torch.logaddexp(lc2 + la1, ld2 + lc1),
        torch.logaddexp(lc2 + lb1, ld2 + ld1),
    )


def _mobius_combine_tracenorm(left, right):
    """right . left as a 2x2 product, divided by its trace (reference kla_ops.py:76-116).

    The map lam -> (A lam + B)/(C lam + D) does not change when all four entries
    are scaled together, so dividing by the trace only keeps the entries O(1).
    Every leaf has non-negative entries (A, C > 0, B = phi >= 0, D = 1) and such
    matrices are closed under products, so the trace stays positive whatever
    order the scan combines in; with A + D = 1 after normalisation and a
    positive determinant (the leaf's is 1/a^2), B C = A D - det < 1/4.
    """
    a1, b1, c1, d1 = left
    a2, b2, c2, d2 = right
    pa = a2 * a1 + b2 * c1
    pb = a2 * b1 + b2 * d1
    pc = c2 * a1 + d2 * c1
    pd = c2 * b1 + d2 * d1
    scale = 1.0 / (pa + pd).clamp_min(EPS)
    return pa * scale, pb * scale, pc * scale, pd * scale


def _affine_combine(left, right):
    """Compose x -> a x + b maps: later (a2, b2) after earlier (a1, b1) (kla_ops.py:119-123)."""
    a1, b1 = left
    a2, b2 = right
    return a2 * a1, a2 * b1 + b2


# ---------------------------------------------------------------------- glue


def _compute_dtype(*tensors: torch.Tensor) -> tuple:
    """Widen bf16/fp16 to float32; keep float32 and float64 (reference kla_ops.py:126-137).

    float64 passes through so torch.autograd.gradcheck can run against the torch path.
    """
    return tuple(t if t.dtype in (torch.float32, torch.float64) else t.float() for t in tensors)


def _state_dtype(t: torch.Tensor) -> torch.dtype:
    return t.dtype if t.dtype in (torch.float32, torch.float64) else torch.float32


def _sufficient_stats(v, lambda_v, k, floor: bool = False):
    """phi = Lambda^v (x) k^2 and r = (v Lambda^v) (x) k, both [B, L, M, S] (kla_ops.py:145-178).

    ``floor`` clamps phi at EPS. The linear Moebius scan does not need it (phi
    only appears as B and inside A), and the clamp would zero the gradient where
    it binds, so it is used only by the log-space combine, which takes log(phi).
    """
    phi = lambda_v.unsqueeze(-1) * (k * k).unsqueeze(-2)
    r = (v * lambda_v).unsqueeze(-1) * k.unsqueeze(-2)
    return (phi.clamp_min(EPS) if floor else phi), r


def _broadcast_ap(a, p, like):
    """[M, S] -> [1, 1, M, S], with p floored at P_MIN (kla_ops.py:181-185)."""
    a4 = a.view(1, 1, *a.shape)
    p4 = p.view(1, 1, *p.shape)
    return a4.to(like), p4.clamp_min(P_MIN).to(like)


def _readout(mean, var, q):
    """y[b,l,m] = sum_s q mean, y_var = sum_s q^2 var (kla_ops.py:288-289)."""
    y = torch.einsum("blms,bls->blm", mean, q)
    y_var = torch.einsum("blms,bls->blm", var, q * q)
    return y, y_var


# ---------------------------------------------------------------- torch path


def kla_scan_torch(
    v: torch.Tensor,
    lambda_v: torch.Tensor,
    k: torch.Tensor,
    q: torch.Tensor,
    a: torch.Tensor,
    p: torch.Tensor,
    initial_state: Optional[KLAState] = None,
    scan_impl: str = "auto",
    decode_from_prior: bool = False,
    mobius_impl: str = "linear",
):
    """Parallel-scan torch implementation. Returns (y, y_var, final_state).

    Same contract as the reference (kla_ops.py:188-290). ``scan_impl`` chooses how
    the scans are parallelised ("auto" becomes "doubling" when grad is off, since
    associative_scan compiles per sequence length); ``mobius_impl`` chooses how
    the precision map is represented while composed ("linear" or "log").
    """
    if mobius_impl not in ("linear", "log"):
        raise ValueError(f"Unknown mobius_impl {mobius_impl!r}; expected 'linear' or 'log'")
    v, lambda_v, k, q = _compute_dtype(v, lambda_v, k, q)
    dtype = v.dtype
    Bn, L, M = v.shape
    S = k.shape[2]
    if initial_state is None:
        initial_state = init_state(Bn, M, S, device=v.device, dtype=dtype)
    lam0 = initial_state.lam.to(dtype)
    eta0 = initial_state.eta.to(dtype)

    if scan_impl == "auto" and not torch.is_grad_enabled():
        scan_impl = "doubling"
    scan = resolve_scan(scan_impl)

    phi, r = _sufficient_stats(v, lambda_v, k, floor=(mobius_impl == "log"))
    a_, p_ = _broadcast_ap(a, p, phi)
    a2 = (a_ * a_).clamp_min(EPS)

    if mobius_impl == "linear":
        leaf_a = ((1.0 + p_ * phi) / a2).expand_as(phi)
        leaf_c = (p_ / a2).expand_as(phi)
        leaf_d = torch.ones_like(phi)
        pa, pb, pc, pd = scan(_mobius_combine_tracenorm, (leaf_a, phi, leaf_c, leaf_d), dim=1)
        l0 = lam0.unsqueeze(1)
        lam = (pa * l0 + pb) / (pc * l0 + pd).clamp_min(EPS)
        var = 1.0 / lam.clamp_min(EPS)
    else:
        log_a2 = a2.log()
        log_leaves = (
            (torch.log1p(p_ * phi) - log_a2).expand_as(phi),
            phi.log(),
            (p_.log() - log_a2).expand_as(phi),
            torch.zeros_like(phi),
        )
        pa, pb, pc, pd = scan(_mobius_combine_log, log_leaves, dim=1)
        log_l0 = lam0.clamp_min(EPS).log().unsqueeze(1)
        log_lam = torch.logaddexp(pa + log_l0, pb) - torch.logaddexp(pc + log_l0, pd)
        lam = log_lam.exp()
        var = (-log_lam).exp()

    lam_prev = torch.cat((lam0.unsqueeze(1), lam[:, :-1]), dim=1)
    alpha = a_ / (a2 + p_ * lam_prev).clamp_min(EPS)
    p_alpha, p_r = scan(_affine_combine, (alpha, r), dim=1)
    eta = p_alpha * eta0.unsqueeze(1) + p_r

    mean = eta * var
    if decode_from_prior:
        mean = a_ * mean
        var = a2 * var + p_
    y, y_var = _readout(mean, var, q)
    return y, y_var, KLAState(lam=lam[:, -1], eta=eta[:, -1])


def kla_step(
    v: torch.Tensor,  # [B, M]
    lambda_v: torch.Tensor,  # [B, M]
    k: torch.Tensor,  # [B, S]
    q: torch.Tensor,  # [B, S]
    a: torch.Tensor,  # [M, S]
    p: torch.Tensor,  # [M, S]
    state: KLAState,
    decode_from_prior: bool = False,
    *,
    backend: str = "torch",
):
    """One filter step for O(1) decode. Returns (y [B, M], y_var [B, M], new_state).

    Reference kla_ops.py:293-331; phi is floored at EPS here, as there.
    ``backend`` names the family the caller runs on (the layer passes its
    config's): the "hip" family (and "auto" on a ROCm GPU) uses the one-kernel
    MI355X step when no gradient is required; every other case is the torch
    formula below.
    """
    if backend != "torch" and _step_on_hip(backend, v) and not (
            torch.is_grad_enabled() and any(t.requires_grad for t in (v, lambda_v, k, q, a, p, *state))):
        from kla.ops.hip.step import kla_step_hip

        y, y_var, lam, eta = kla_step_hip(v, lambda_v, k, q, a, p, state.lam, state.eta, decode_from_prior)
        return y, y_var, KLAState(lam=lam, eta=eta)
    v, lambda_v, k, q = _compute_dtype(v, lambda_v, k, q)
    dtype = v.dtype
    phi = (lambda_v.unsqueeze(-1) * (k * k).unsqueeze(-2)).clamp_min(EPS)
    r = (v * lambda_v).unsqueeze(-1) * k.unsqueeze(-2)
    a_ = a.to(dtype).unsqueeze(0)
    p_ = p.to(dtype).unsqueeze(0).clamp_min(P_MIN)
    a2 = (a_ * a_).clamp_min(EPS)

    denom = (a2 + p_ * state.lam).clamp_min(EPS)
    lam = state.lam / denom + phi
    eta = (a_ / denom) * state.eta + r
    var = 1.0 / lam.clamp_min(EPS)
    mean = eta * var
    if decode_from_prior:
        mean = a_ * mean
        var = a2 * var + p_
    y = torch.einsum("bms,bs->bm", mean, q)
    y_var = torch.einsum("bms,bs->bm", var, q * q)
    return y, y_var, KLAState(lam=lam, eta=eta)


def _step_on_hip(backend: str, x: torch.Tensor) -> bool:
    """Whether work of ``backend`` on ``x`` runs on the MI355X kernels: a
    hip-family backend (or "auto" resolving to one) and fp32/bf16 tensors on a
    ROCm GPU. A hip-family backend whose library is missing or stale raises
    here instead of running torch code in its place."""
    if not x.is_cuda or x.dtype == torch.float64:
        return False
    if backend == "auto":
        backend = _resolve_auto(x)
    if backend.split("_", 1)[0] != "hip":
        return False
    if not _HIP_LIB_LOADED:
        from kla.ops.hip import _lib

        _lib.lib()   # RuntimeError when libkla_hip.so is missing or built for another ABI
        _HIP_LIB_LOADED.append(True)
    return True


# Non-empty once _step_on_hip has loaded libkla_hip.so (the load is then skipped).
_HIP_LIB_LOADED: list = []


def kla_scan_reference(v, lambda_v, k, q, a, p, initial_state: Optional[KLAState] = None,
                       decode_from_prior: bool = False):
    """Sequential reference: :func:`kla_step` along the sequence (kla_ops.py:334-362)."""
    Bn, L, M = v.shape
    S = k.shape[2]
    state = initial_state or init_state(Bn, M, S, device=v.device, dtype=_state_dtype(v))
    ys, yvars = [], []
    for t in range(L):
        y_t, yv_t, state = kla_step(v[:, t], lambda_v[:, t], k[:, t], q[:, t], a, p, state,
                                    decode_from_prior=decode_from_prior)
        ys.append(y_t)
        yvars.append(yv_t)
    return torch.stack(ys, dim=1), torch.stack(yvars, dim=1), state


# ----------------------------------------------------------------- registry


def _backend_torch(*args, scan_impl="auto", mobius_impl="linear", **kwargs):
    return kla_scan_torch(*args, scan_impl=scan_impl, mobius_impl=mobius_impl, **kwargs)


def _backend_hip(*args, **kwargs):
    """MI355X kernels, default path (see :mod:`kla.ops.hip_backend`)."""
    from kla.ops.hip_backend import kla_scan_hip

    return kla_scan_hip(*args, **kwargs)


def _backend_hip_fused(*args, **kwargs):
    """MI355X kernels, pinned to the fused scan (one kernel per direction)."""
    from kla.ops.hip_backend import kla_scan_hip

    return kla_scan_hip(*args, kernel="fused", **kwargs)


def _backend_hip_composed(*args, **kwargs):
    """MI355X kernels, pinned to the composed path (HIP scans + torch glue)."""
    from kla.ops.hip_backend import kla_scan_hip

    return kla_scan_hip(*args, kernel="composed", **kwargs)


def _not_in_this_build(name: str):
    def backend(*args, **kwargs):
        raise NotImplementedError(
            f"The {name!r} backend's kernels (CUDA/Triton/Metal) are not part of this MI355X "
            "build; use backend='hip' on a ROCm GPU, or 'torch' (or 'auto')."
        )

    backend.__name__ = f"_backend_{name}"
    return backend


# Family name = that family's default implementation; "<family>_<impl>" pins one
# (reference kla_ops.py:425-442). "auto" is the only device-dependent name.
_BACKENDS = {
    "torch": _backend_torch,
    "hip": _backend_hip,
    "hip_fused": _backend_hip_fused,
    "hip_composed": _backend_hip_composed,
    "triton": _not_in_this_build("triton"),
    "triton_fused": _not_in_this_build("triton_fused"),
    "triton_composed": _not_in_this_build("triton_composed"),
    "cuda": _not_in_this_build("cuda"),
    "cuda_v2_2": _not_in_this_build("cuda_v2_2"),
    "cuda_v2_1": _not_in_this_build("cuda_v2_1"),
    "mps": _not_in_this_build("mps"),
    "mps_fused": _not_in_this_build("mps_fused"),
    "mps_tiled": _not_in_this_build("mps_tiled"),
    "mps_composed": _not_in_this_build("mps_composed"),
}


@functools.cache
def _hip_available() -> bool:
    """True on a ROCm build of torch with libkla_hip.so present and loadable."""
    if getattr(torch.version, "hip", None) is None:
        return False
    try:
        from kla.ops.hip import _lib

        _lib.lib()
    except Exception:
        return False
    return True


# Device attribute -> backend "auto" picks there, if its kernels load.
_AUTO = (("is_cuda", "hip", _hip_available),)


def _resolve_auto(x: torch.Tensor) -> str:
    """Backend "auto" picks for tensors on ``x``'s device (kla_ops.py:472-483).

    Device in, backend out; nothing about the call is consulted, so a backend
    that cannot serve a request raises rather than being swapped out silently.
    """
    for attr, backend, available in _AUTO:
        if getattr(x, attr) and available():
            return backend
    return "torch"


def kla_scan(
    v: torch.Tensor,
    lambda_v: torch.Tensor,
    k: torch.Tensor,
    q: torch.Tensor,
    a: torch.Tensor,
    p: torch.Tensor,
    *,
    initial_state: Optional[KLAState] = None,
    backend: str = "auto",
    scan_impl: str = "auto",
    decode_from_prior: bool = False,
    mobius_impl: str = "linear",
):
    """Dispatch the KLA scan to ``backend`` (reference kla_ops.py:486-541).

    Returns (y [B, L, M], y_var [B, L, M], KLAState(lam [B, M, S], eta [B, M, S])).
    ``scan_impl`` and ``mobius_impl`` only reach the torch backend.
    """
    if backend == "auto":
        backend = _resolve_auto(v)
    try:
        fn = _BACKENDS[backend]
    except KeyError:
        raise ValueError(f"Unknown backend {backend!r}; expected one of {sorted(_BACKENDS)}") from None
    if backend == "torch":
        return fn(v, lambda_v, k, q, a, p, initial_state=initial_state, scan_impl=scan_impl,
                  decode_from_prior=decode_from_prior, mobius_impl=mobius_impl)
    return fn(v, lambda_v, k, q, a, p, initial_state=initial_state,
              decode_from_prior=decode_from_prior)


def backend_names() -> tuple:
    """Every name ``kla_scan`` accepts, read off the dispatch table."""
    return tuple(_BACKENDS)


def default_device() -> str:
    """The accelerator ``resolve_backend`` assumes by default."""
    if torch.cuda.is_available():
        return "cuda"
    if torch.backends.mps.is_available():
        return "mps"
    return "cpu"


def resolve_backend(device=None) -> str:
    """The backend ``backend="auto"`` resolves to for tensors on ``device``."""
    if device is None:
        device = default_device()
    return _resolve_auto(torch.empty(0, device=device))
