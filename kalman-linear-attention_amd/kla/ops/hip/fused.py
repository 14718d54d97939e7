"""The fused KLA scan on MI355X: one kernel per direction, no [B, L, M, S] tensors.

:func:`kla_scan_fused` computes what the reference's ``kla_scan_torch``
(src/kla/ops/kla_ops.py:188-290) computes -- y, y_var [B, L, M] and the final
state (lam, eta) [B, M, S] -- from v, lambda_v [B, L, M], k, q [B, L, S] and the
static a, p [M, S], with an optional initial state and ``decode_from_prior``.
It is a ``torch.library`` custom op (``kla_hip::kla_scan_fused``) whose backward
is the hand-written exact adjoint kernel (checkpoint replay), giving gradients
for all six inputs and for the initial state, including gradients that arrive
through the returned final state.

:func:`kla_scan_fused_sensors` is the same scan fed by the layer's sensor
projection directly (``kla_hip::kla_scan_fused_sensors``): v and log sigma^2 are
read as the projection's strided bf16 or fp32 columns, and the precision
lambda_v is formed inside the kernels.
"""

from __future__ import annotations

import ctypes
import functools
import math
from typing import Optional

import torch

from kla.ops.hip import _lib
from kla.ops.hip.scans import _require_device

_F32 = torch.float32
# d_state one fused launch takes: a channel's S lanes in one 256-thread
# workgroup. kla_scan_fused runs a larger d_state as groups of this many lanes
# (state_groups); the sensor-fed variant and the decode steps stop here.
MAX_STATE = 256
# The time-split forward (inference only): grids below _split_below(SP)
# workgroups per CU are split, into chunks of at least MIN_CHUNK steps, up to
# about SPLIT_TO workgroups per CU. Measured on MI355X: the chunk-map pass costs
# about what the forward costs, so a split pays only where the whole grid leaves
# CUs or issue slots idle -- below one workgroup per CU up to 64 lanes per
# channel (one workgroup keeps a CU busy), below two for 128 and 256 (whose
# channels span several waves and wait on each other); chunks shorter than 128
# steps lose to the map pass and the walk over chunks.
SPLIT_TO, MIN_CHUNK = 8, 128


def _split_below(sp: int) -> int:
    return 1 if sp <= 64 else 2


@functools.cache
def _cus(index: int) -> int:
    return torch.cuda.get_device_properties(index).multi_processor_count


def time_chunks(B: int, L: int, M: int, S: int, cus: int) -> int:
    """Chunks the time-split forward cuts each sequence into (1: no split). The
    grid is B x channel groups (256 / SP channels a workgroup, SP = S rounded up
    to a power of two, at least 4); below _split_below(SP) workgroups per CU the
    chunk count doubles while the grid stays below SPLIT_TO per CU, the chunks
    divide L evenly and stay MIN_CHUNK steps or longer."""
    sp, base = _grid(B, M, S)
    if base >= _split_below(sp) * cus:
        return 1
    nc = 1
    while base * nc * 2 <= SPLIT_TO * cus and L % (2 * nc) == 0 and L // (2 * nc) >= MIN_CHUNK:
        nc *= 2
    return nc


def _grid(B: int, M: int, S: int) -> tuple[int, int]:
    """(SP, workgroups) of the fused kernels' plain grid: SP = S rounded up to a
    power of two (at least 4), 256 / SP channels a workgroup, B x channel groups.
    One launch's plan: S is at most MAX_STATE (a wider state plans per group)."""
    if S > MAX_STATE:
        raise ValueError(f"one fused launch takes d_state <= {MAX_STATE} (got {S}); plan each of state_groups(S)")
    sp = 4
    while sp < S:
        sp *= 2
    return sp, B * -(-M // (256 // sp))


def train_chunks(B: int, L: int, M: int, S: int, cus: int) -> int:
    """Chunks the time-split training pair (the forward that keeps checkpoints and
    the backward) cuts each sequence into (1: no split). The backward holds two
    workgroups per CU and the split costs about 1.7 backwards of work (the chunk
    maps' replay and composition, then the backward itself), so it pays below one
    workgroup per CU: the chunk count doubles while the grid stays below two per
    CU, the chunks divide L into whole 16-step checkpoint blocks (the forward's
    checkpoints are then the same memory on the chunk view) and last at least
    MIN_CHUNK steps."""
    _, base = _grid(B, M, S)
    if base >= cus:
        return 1
    nc = 1
    while base * nc < 2 * cus and L % (32 * nc) == 0 and L // (2 * nc) >= MIN_CHUNK:
        nc *= 2
    return nc


def _split_forward(sn, k, q, a, p, lam0, eta0, y, y_var, lam_fin, eta_fin, decode_from_prior, B, L, M, S, nc,
                   dev, ck_lam=None, ck_eta=None):
    """The time-split forward: kla_fused_chunk_maps on the [B * nc, L / nc] view,
    kla_chunk_starts, then the fused forward on the view from those starts (with
    the checkpoints when given: [B, n_ck, M, S] is the view's [B * nc, n_ck / nc,
    M, S] when L / nc is a multiple of 16). Writes lam_fin, eta_fin [B, M, S], the
    state after each sequence's last chunk (from the chunk maps, by
    kla_chunk_starts). The maps and the chunk starts share one buffer; every
    chunk's final state (unused) then lands in the maps' part, no longer read."""
    lib, pt = _lib.lib(), _lib.ptr
    stream = _lib.stream(dev)
    Bp, Lc = B * nc, L // nc
    lanes = Bp * M * S
    buf = torch.empty(10 * lanes, dtype=_F32, device=dev)   # maps [Bp, M, S, 8], then two [Bp, M, S]
    maps = pt(buf)
    lam_st, eta_st = maps + 32 * lanes, maps + 36 * lanes
    _lib.check("kla_fused_chunk_maps", lib.kla_fused_chunk_maps(
        ctypes.byref(sn), pt(k), pt(a), pt(p), maps, Bp, Lc, M, S, stream))
    _lib.check("kla_chunk_starts", lib.kla_chunk_starts(
        maps, pt(lam0), pt(eta0), lam_st, eta_st, pt(lam_fin), pt(eta_fin), B, nc, M, S, stream))
    _lib.check("kla_fused_scan_sensors_fwd", lib.kla_fused_scan_sensors_fwd(
        ctypes.byref(sn), pt(k), pt(q), pt(a), pt(p), lam_st, eta_st, pt(y), pt(y_var), maps, maps + 4 * lanes,
        pt(ck_lam), pt(ck_eta), int(decode_from_prior), Bp, Lc, M, S, stream))


def _split_backward(bwd, dy, dy_var, dlam_fin, deta_fin, sn, k, q, a, p, ck_lam, ck_eta, decode_from_prior,
                    B, L, M, S, nc, dev):
    """The time-split backward: kla_fused_adjoint_maps on the [B * nc, L / nc]
    view, kla_adjoint_ends, then ``bwd(batch, steps, dlam_fin, deta_fin, dlam0,
    deta0, workspace, nbytes)`` -- the backward entry point on the view, with every
    chunk's adjoint entering from its end. Returns (dlam0, deta0) [B, M, S], the
    first chunks' initial-state gradients."""
    lib, pt = _lib.lib(), _lib.ptr
    stream = _lib.stream(dev)
    Bp, Lc = B * nc, L // nc
    f32 = dict(dtype=_F32, device=dev)
    maps = torch.empty(Bp, M, S, 8, **f32)
    _lib.check("kla_fused_adjoint_maps", lib.kla_fused_adjoint_maps(
        pt(dy), pt(dy_var), ctypes.byref(sn), pt(k), pt(q), pt(a), pt(p), pt(ck_lam), pt(ck_eta), pt(maps),
        int(decode_from_prior), Bp, Lc, M, S, stream))
    gl_end, ge_end = torch.empty(B, nc, M, S, **f32), torch.empty(B, nc, M, S, **f32)
    _lib.check("kla_adjoint_ends", lib.kla_adjoint_ends(
        pt(maps), pt(dlam_fin), pt(deta_fin), pt(gl_end), pt(ge_end), B, nc, M, S, stream))
    dlam0, deta0 = torch.empty(B, nc, M, S, **f32), torch.empty(B, nc, M, S, **f32)
    nbytes = int(lib.kla_fused_workspace_bytes(Bp, Lc, M, S))
    ws, _ = _lib.scratch(nbytes, dev)
    bwd(Bp, Lc, gl_end, ge_end, dlam0, deta0, ws, nbytes)
    return dlam0[:, 0].contiguous(), deta0[:, 0].contiguous()


def _dense_sensors(v: torch.Tensor, lambda_v: torch.Tensor) -> "_lib.Sensors":
    """Dense fp32 [B, L, M] v and lambda_v as a sensor descriptor."""
    M = v.shape[2]
    return _lib.Sensors(v=_lib.ptr(v), ld_v=M, obs=_lib.ptr(lambda_v), ld_obs=M, dtype=_lib.KLA_DTYPE_F32,
                        log_var=0, obs_var_min=0.0, obs_var_max=math.inf)


def _f32(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.to(_F32).contiguous()


def _dynamics(a: torch.Tensor, p: torch.Tensor, M: int, S: int) -> tuple[torch.Tensor, torch.Tensor]:
    """a, p as dense fp32 [M, S]: the reference's torch path takes any shape that
    broadcasts to [M, S] (kla_ops.py:181-185 views them as [1, 1, *shape]); the
    gradient flows back through the expansion."""
    if a.dim() > 2 or p.dim() > 2:
        raise ValueError(f"a and p must broadcast to [M, S] = [{M}, {S}]; got {tuple(a.shape)}, {tuple(p.shape)}")
    return _f32(a.expand(M, S)), _f32(p.expand(M, S))


def _check(v, lambda_v, k, q, a, p, lam0, eta0, max_state: Optional[int] = MAX_STATE):
    if v.dim() != 3 or k.dim() != 3:
        raise ValueError(f"v must be [B, L, M] and k [B, L, S]; got {tuple(v.shape)} and {tuple(k.shape)}")
    B, L, M = v.shape
    S = k.shape[2]
    if max_state is not None and S > max_state:
        raise NotImplementedError(f"the fused hip kernel supports d_state <= {max_state} (got {S}); "
                                  "use backend='hip_composed'")
    for name, t, shape in (("lambda_v", lambda_v, (B, L, M)), ("k", k, (B, L, S)), ("q", q, (B, L, S)),
                           ("a", a, (M, S)), ("p", p, (M, S)), ("lam0", lam0, (B, M, S)),
                           ("eta0", eta0, (B, M, S))):
        if t is not None and tuple(t.shape) != shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {shape}")
    return B, L, M, S


def state_groups(S: int) -> list[tuple[int, int]]:
    """(first lane, lanes) of the state groups a d_state above MAX_STATE runs as:
    MAX_STATE lanes each, the remainder last. The filter's lanes are independent
    but for the read-out's sum over s, so each group is a whole fused scan of its
    own lanes (k, q, a, p and the state sliced along s) and y, y_var -- and in the
    backward dv, dlambda_v -- are the groups' sums, added in group order."""
    return [(s0, min(MAX_STATE, S - s0)) for s0 in range(0, S, MAX_STATE)]


def _lanes(t: Optional[torch.Tensor], s0: int, n: int) -> Optional[torch.Tensor]:
    return None if t is None else t[..., s0:s0 + n].contiguous()


def _ck_group(ck: torch.Tensor, B: int, n_ck: int, M: int, s0: int, n: int) -> torch.Tensor:
    """Group (s0, n)'s checkpoints: the grouped forward keeps each group's [B, n_ck,
    M, n] checkpoints as one contiguous block of the [B, n_ck, M, S] buffer, in
    group order (the buffer is opaque to everything but the backward)."""
    unit = B * n_ck * M
    return ck.view(-1)[unit * s0:unit * (s0 + n)].view(B, n_ck, M, n)


def _fwd_one(v, lambda_v, k, q, a, p, lam0, eta0, decode_from_prior, save, dev, ck_lam, ck_eta):
    """One fused forward over d_state <= MAX_STATE into the given checkpoint
    buffers (used when ``save``); returns (y, y_var, lam_fin, eta_fin)."""
    B, L, M = v.shape
    S = k.shape[2]
    y = v.new_empty(B, L, M)
    y_var = v.new_empty(B, L, M)
    lam_fin = v.new_empty(B, M, S)
    eta_fin = v.new_empty(B, M, S)
    if B * M * S == 0:
        # No lanes: the read-outs sum over no state lanes (zero where B, L, M leave entries).
        return y.zero_(), y_var.zero_(), lam_fin, eta_fin
    cus = _cus(dev.index or 0)
    nc = train_chunks(B, L, M, S, cus) if save else time_chunks(B, L, M, S, cus)
    if nc > 1:
        _split_forward(_dense_sensors(v, lambda_v), k, q, a, p, lam0, eta0, y, y_var, lam_fin, eta_fin,
                       decode_from_prior, B, L, M, S, nc, dev,
                       ck_lam=ck_lam if save else None, ck_eta=ck_eta if save else None)
        return y, y_var, lam_fin, eta_fin
    stream = _lib.stream(dev)
    pt = _lib.ptr
    _lib.check("kla_fused_scan_fwd", _lib.lib().kla_fused_scan_fwd(
        pt(v), pt(lambda_v), pt(k), pt(q), pt(a), pt(p), pt(lam0), pt(eta0), pt(y), pt(y_var),
        pt(lam_fin), pt(eta_fin), pt(ck_lam) if save else None, pt(ck_eta) if save else None,
        int(decode_from_prior), B, L, M, S, stream))
    return y, y_var, lam_fin, eta_fin


@_lib.hip_op("kla_hip::kla_scan_fused")
def _fused_fwd_op(v: torch.Tensor, lambda_v: torch.Tensor, k: torch.Tensor, q: torch.Tensor, a: torch.Tensor,
                  p: torch.Tensor, lam0: Optional[torch.Tensor], eta0: Optional[torch.Tensor],
                  decode_from_prior: bool, save: bool
                  ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns (y, y_var, lam_fin, eta_fin, ck_lam, ck_eta); the checkpoints are
    empty unless ``save``. d_state above MAX_STATE runs as state_groups(S)."""
    dev = _require_device(v, lambda_v, k, q, a, p, lam0, eta0)
    B, L, M, S = _check(v, lambda_v, k, q, a, p, lam0, eta0, max_state=None)
    n_ck = int(_lib.lib().kla_fused_checkpoints(L))
    ck_lam = v.new_empty(B, n_ck, M, S) if save else v.new_empty(0)
    ck_eta = v.new_empty(B, n_ck, M, S) if save else v.new_empty(0)
    if S <= MAX_STATE:
        return (*_fwd_one(v, lambda_v, k, q, a, p, lam0, eta0, decode_from_prior, save, dev, ck_lam, ck_eta),
                ck_lam, ck_eta)
    y = y_var = None
    lam_fin, eta_fin = v.new_empty(B, M, S), v.new_empty(B, M, S)
    for s0, n in state_groups(S):
        cl = _ck_group(ck_lam, B, n_ck, M, s0, n) if save else ck_lam
        ce = _ck_group(ck_eta, B, n_ck, M, s0, n) if save else ck_eta
        yg, yvg, lf, ef = _fwd_one(v, lambda_v, _lanes(k, s0, n), _lanes(q, s0, n), _lanes(a, s0, n),
                                   _lanes(p, s0, n), _lanes(lam0, s0, n), _lanes(eta0, s0, n), decode_from_prior,
                                   save, dev, cl, ce)
        y, y_var = (yg, yvg) if y is None else (y.add_(yg), y_var.add_(yvg))
        lam_fin[..., s0:s0 + n] = lf
        eta_fin[..., s0:s0 + n] = ef
    return y, y_var, lam_fin, eta_fin, ck_lam, ck_eta


@_fused_fwd_op.register_fake
def _(v, lambda_v, k, q, a, p, lam0, eta0, decode_from_prior, save):
    B, L, M = v.shape
    S = k.shape[2]
    n_ck = (L + 15) // 16
    ck = v.new_empty(B, n_ck, M, S) if save else v.new_empty(0)
    return (v.new_empty(B, L, M), v.new_empty(B, L, M), v.new_empty(B, M, S), v.new_empty(B, M, S), ck,
            torch.empty_like(ck))


def _bwd_one(dy, dy_var, dlam_fin, deta_fin, v, lambda_v, k, q, a, p, ck_lam, ck_eta, decode_from_prior, dev):
    """One fused backward over d_state <= MAX_STATE; returns (dv, dlambda_v, dk,
    dq, da, dp, dlam0, deta0)."""
    B, L, M = v.shape
    S = k.shape[2]
    dv, dlv = torch.empty_like(v), torch.empty_like(lambda_v)
    dk, dq = torch.empty_like(k), torch.empty_like(q)
    da, dp = torch.empty_like(a), torch.empty_like(p)
    dlam0, deta0 = v.new_empty(B, M, S), v.new_empty(B, M, S)
    if B * M * S == 0:
        # No lanes: every gradient with entries (dk, dq over no channels, da, dp over no batch rows) is zero.
        for t in (dv, dlv, dk, dq, da, dp):
            t.zero_()
        return dv, dlv, dk, dq, da, dp, dlam0, deta0
    pt = _lib.ptr

    def bwd(batch, steps, lam_fin_grad, eta_fin_grad, lam0_grad, eta0_grad, ws, nbytes):
        stream = _lib.stream(dev)
        _lib.check("kla_fused_scan_bwd", _lib.lib().kla_fused_scan_bwd(
            pt(dy), pt(dy_var), pt(lam_fin_grad), pt(eta_fin_grad), pt(v), pt(lambda_v), pt(k), pt(q), pt(a),
            pt(p), pt(ck_lam), pt(ck_eta), pt(dv), pt(dlv), pt(dk), pt(dq), pt(da), pt(dp), pt(lam0_grad),
            pt(eta0_grad), int(decode_from_prior), batch, steps, M, S, pt(ws), nbytes, stream))

    nc = train_chunks(B, L, M, S, _cus(dev.index or 0))
    if nc > 1:
        dlam0, deta0 = _split_backward(bwd, dy, dy_var, dlam_fin, deta_fin, _dense_sensors(v, lambda_v), k, q, a,
                                       p, ck_lam, ck_eta, decode_from_prior, B, L, M, S, nc, dev)
        return dv, dlv, dk, dq, da, dp, dlam0, deta0
    nbytes = int(_lib.lib().kla_fused_workspace_bytes(B, L, M, S))
    ws, _ = _lib.scratch(nbytes, dev)
    bwd(B, L, dlam_fin, deta_fin, dlam0, deta0, ws, ws.numel())
    return dv, dlv, dk, dq, da, dp, dlam0, deta0


@_lib.hip_op("kla_hip::kla_scan_fused_backward")
def _fused_bwd_op(dy: torch.Tensor, dy_var: Optional[torch.Tensor], dlam_fin: Optional[torch.Tensor],
                  deta_fin: Optional[torch.Tensor],
                  v: torch.Tensor, lambda_v: torch.Tensor, k: torch.Tensor, q: torch.Tensor, a: torch.Tensor,
                  p: torch.Tensor, ck_lam: torch.Tensor, ck_eta: torch.Tensor, decode_from_prior: bool
                  ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                             torch.Tensor, torch.Tensor]:
    """Returns (dv, dlambda_v, dk, dq, da, dp, dlam0, deta0). dy_var, dlam_fin,
    deta_fin None: zero (without dy_var the kernel skips the variance read-out's
    adjoint). d_state above MAX_STATE runs as the forward's state_groups(S)."""
    dev = _require_device(dy, dy_var, dlam_fin, deta_fin, v, lambda_v, k, q, a, p, ck_lam, ck_eta)
    B, L, M, S = _check(v, lambda_v, k, q, a, p, None, None, max_state=None)
    if S <= MAX_STATE:
        return _bwd_one(dy, dy_var, dlam_fin, deta_fin, v, lambda_v, k, q, a, p, ck_lam, ck_eta,
                        decode_from_prior, dev)
    n_ck = int(_lib.lib().kla_fused_checkpoints(L))
    dv = dlv = None
    dk, dq = torch.empty_like(k), torch.empty_like(q)
    da, dp = torch.empty_like(a), torch.empty_like(p)
    dlam0, deta0 = v.new_empty(B, M, S), v.new_empty(B, M, S)
    for s0, n in state_groups(S):
        g = _bwd_one(dy, dy_var, _lanes(dlam_fin, s0, n), _lanes(deta_fin, s0, n), v, lambda_v,
                     _lanes(k, s0, n), _lanes(q, s0, n), _lanes(a, s0, n), _lanes(p, s0, n),
                     _ck_group(ck_lam, B, n_ck, M, s0, n), _ck_group(ck_eta, B, n_ck, M, s0, n),
                     decode_from_prior, dev)
        dv, dlv = (g[0], g[1]) if dv is None else (dv.add_(g[0]), dlv.add_(g[1]))
        for out, part in zip((dk, dq, da, dp, dlam0, deta0), g[2:]):
            out[..., s0:s0 + n] = part
    return dv, dlv, dk, dq, da, dp, dlam0, deta0


@_fused_bwd_op.register_fake
def _(dy, dy_var, dlam_fin, deta_fin, v, lambda_v, k, q, a, p, ck_lam, ck_eta, decode_from_prior):
    B, L, M = v.shape
    S = k.shape[2]
    return (torch.empty_like(v), torch.empty_like(lambda_v), torch.empty_like(k), torch.empty_like(q),
            torch.empty_like(a), torch.empty_like(p), v.new_empty(B, M, S), v.new_empty(B, M, S))


def _setup(ctx, inputs, output):
    v, lambda_v, k, q, a, p, lam0, eta0, decode_from_prior, save = inputs
    _, _, _, _, ck_lam, ck_eta = output
    if not save:
        raise RuntimeError("kla_scan_fused was run without checkpoints but a gradient is required")
    ctx.prior = decode_from_prior
    ctx.has_lam0, ctx.has_eta0 = lam0 is not None, eta0 is not None
    ctx.save_for_backward(v, lambda_v, k, q, a, p, ck_lam, ck_eta)
    # Unused outputs arrive as None, not zeros: an unused y_var selects the
    # kernel without the variance adjoint, an unused final state reads nothing.
    ctx.set_materialize_grads(False)


def _backward(ctx, dy, dy_var, dlam_fin, deta_fin, _dck_lam, _dck_eta):
    v, lambda_v, k, q, a, p, ck_lam, ck_eta = ctx.saved_tensors

    def f32(t):
        return None if t is None else t.to(_F32).contiguous()

    dv, dlv, dk, dq, da, dp, dlam0, deta0 = _lib.call(_fused_bwd_op,
        torch.zeros_like(v) if dy is None else f32(dy), f32(dy_var), f32(dlam_fin), f32(deta_fin), v, lambda_v,
        k, q, a, p, ck_lam, ck_eta, ctx.prior)
    return (dv, dlv, dk, dq, da, dp, dlam0 if ctx.has_lam0 else None, deta0 if ctx.has_eta0 else None,
            None, None)


_fused_fwd_op.register_autograd(_backward, setup_context=_setup)


def kla_scan_fused(v, lambda_v, k, q, a, p, lam0=None, eta0=None, decode_from_prior: bool = False):
    """(y, y_var, lam_fin, eta_fin) of the KLA scan, computed by the fused kernels.

    All inputs are cast to contiguous float32 (the reference's GPU backends
    compute in float32 too). Checkpoints for the backward are kept only when a
    gradient can be required.
    """
    a, p = _dynamics(a, p, v.shape[-1], k.shape[-1])
    v, lambda_v, k, q, lam0, eta0 = (_f32(t) for t in (v, lambda_v, k, q, lam0, eta0))
    save = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (v, lambda_v, k, q, a, p, lam0, eta0))
    y, y_var, lam_fin, eta_fin, _, _ = _lib.call(_fused_fwd_op, v, lambda_v, k, q, a, p, lam0, eta0,
                                                  bool(decode_from_prior), save)
    return y, y_var, lam_fin, eta_fin


# ------------------------------------------------------- sensors from the projection
#
# The layer's sensor read-out (reference src/kla/layers/kla_layer.py:194-231) ends
# in v.float() and lambda_v = 1 / min(softplus(log sigma^2) + obs_var_min,
# obs_var_max), each an elementwise pass over [B, L, M] with its own backward.
# kla_scan_fused_sensors hands the projection's v and log sigma^2 columns to the
# kernels as they are (bf16 or fp32, strided rows); the kernels form lambda_v
# while staging and write dv, d log sigma^2 in the projection's dtype.


def _sensor_rows(t: torch.Tensor) -> Optional[int]:
    """Row stride ld of a [B, L, M] view whose element (b, t, m) sits at
    (b * L + t) * ld + m, or None if the view is not laid out that way."""
    B, L, M = t.shape
    if M > 1 and t.stride(2) != 1:
        return None
    if L == 1:
        ld = t.stride(0) if B > 1 else M
    else:
        ld = t.stride(1)
        if B > 1 and t.stride(0) != L * ld:
            return None
    return ld if ld >= M else None


def _sensor_desc(v: torch.Tensor, obs: torch.Tensor, lds: tuple[int, int], log_var: bool, obs_var_min: float,
                 obs_var_max: float) -> "_lib.Sensors":
    return _lib.Sensors(v=_lib.ptr(v), ld_v=lds[0], obs=_lib.ptr(obs), ld_obs=lds[1],
                        dtype=_lib.KLA_DTYPE_BF16 if v.dtype == torch.bfloat16 else _lib.KLA_DTYPE_F32,
                        log_var=int(log_var), obs_var_min=obs_var_min, obs_var_max=obs_var_max)


def _check_sensors(v, obs) -> tuple[int, int]:
    """(ld_v, ld_obs), the row strides of the two sensor operands; raises if
    their dtypes or layouts are not ones the kernels read."""
    if v.dtype != obs.dtype or v.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"v and the precision operand must both be float32 or both bfloat16; "
                        f"got {v.dtype} and {obs.dtype}")
    lds = _sensor_rows(v), _sensor_rows(obs)
    if None in lds:
        raise ValueError("sensor operands must be [B, L, M] rows with a contiguous last dimension")
    return lds


@_lib.hip_op("kla_hip::kla_scan_fused_sensors")
def _sensors_fwd_op(v: torch.Tensor, obs: torch.Tensor, k: torch.Tensor, q: torch.Tensor, a: torch.Tensor,
                    p: torch.Tensor, lam0: Optional[torch.Tensor], eta0: Optional[torch.Tensor], log_var: bool,
                    obs_var_min: float, obs_var_max: float, decode_from_prior: bool, save: bool, with_var: bool
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(y, y_var, lam_fin, eta_fin, ck_lam, ck_eta) from strided v and log sigma^2
    (or lambda_v) of one dtype; the checkpoints are empty unless ``save``, and
    y_var is empty (and not computed) unless ``with_var``."""
    dev = _require_device(v, obs, k, q, a, p, lam0, eta0)
    B, L, M, S = _check(v, obs, k, q, a, p, lam0, eta0)
    lds = _check_sensors(v, obs)
    f32 = dict(dtype=_F32, device=dev)
    y = torch.empty(B, L, M, **f32)
    y_var = torch.empty(B, L, M, **f32) if with_var else torch.empty(0, **f32)
    lam_fin, eta_fin = torch.empty(B, M, S, **f32), torch.empty(B, M, S, **f32)
    n_ck = int(_lib.lib().kla_fused_checkpoints(L))
    ck_lam = torch.empty(B, n_ck, M, S, **f32) if save else torch.empty(0, **f32)
    ck_eta = torch.empty(B, n_ck, M, S, **f32) if save else torch.empty(0, **f32)
    if B * M * S == 0:
        # No lanes: the read-outs sum over no state lanes (zero where B, L, M leave entries).
        return y.zero_(), y_var.zero_(), lam_fin, eta_fin, ck_lam, ck_eta
    sn = _sensor_desc(v, obs, lds, log_var, obs_var_min, obs_var_max)
    cus = _cus(dev.index or 0)
    nc = train_chunks(B, L, M, S, cus) if save else time_chunks(B, L, M, S, cus)
    if nc > 1:
        _split_forward(sn, k, q, a, p, lam0, eta0, y, y_var if with_var else None, lam_fin, eta_fin,
                       decode_from_prior, B, L, M, S, nc, dev,
                       ck_lam=ck_lam if save else None, ck_eta=ck_eta if save else None)
        return y, y_var, lam_fin, eta_fin, ck_lam, ck_eta
    pt = _lib.ptr
    _lib.check("kla_fused_scan_sensors_fwd", _lib.lib().kla_fused_scan_sensors_fwd(
        ctypes.byref(sn), pt(k), pt(q), pt(a), pt(p), pt(lam0), pt(eta0), pt(y), pt(y_var) if with_var else None,
        pt(lam_fin),
        pt(eta_fin), pt(ck_lam) if save else None, pt(ck_eta) if save else None, int(decode_from_prior),
        B, L, M, S, _lib.stream(dev)))
    return y, y_var, lam_fin, eta_fin, ck_lam, ck_eta


@_sensors_fwd_op.register_fake
def _(v, obs, k, q, a, p, lam0, eta0, log_var, obs_var_min, obs_var_max, decode_from_prior, save, with_var):
    B, L, M = v.shape
    S = k.shape[2]
    n_ck = (L + 15) // 16
    f = dict(dtype=_F32)
    ck = k.new_empty(B, n_ck, M, S, **f) if save else k.new_empty(0, **f)
    y_var = k.new_empty(B, L, M, **f) if with_var else k.new_empty(0, **f)
    return (k.new_empty(B, L, M, **f), y_var, k.new_empty(B, M, S, **f), k.new_empty(B, M, S, **f), ck,
            torch.empty_like(ck))


@_lib.hip_op("kla_hip::kla_scan_fused_sensors_backward")
def _sensors_bwd_op(dy: torch.Tensor, dy_var: Optional[torch.Tensor], dlam_fin: Optional[torch.Tensor],
                    deta_fin: Optional[torch.Tensor],
                    v: torch.Tensor, obs: torch.Tensor, k: torch.Tensor, q: torch.Tensor, a: torch.Tensor,
                    p: torch.Tensor, ck_lam: torch.Tensor, ck_eta: torch.Tensor, log_var: bool,
                    obs_var_min: float, obs_var_max: float, decode_from_prior: bool
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                               torch.Tensor, torch.Tensor]:
    """(dv, dobs, dk, dq, da, dp, dlam0, deta0); dv and dobs dense in the sensors' dtype.
    dy_var, dlam_fin, deta_fin None: zero (without dy_var the variance read-out's
    adjoint is skipped)."""
    dev = _require_device(dy, dy_var, dlam_fin, deta_fin, v, obs, k, q, a, p, ck_lam, ck_eta)
    B, L, M, S = _check(v, obs, k, q, a, p, None, None)
    lds = _check_sensors(v, obs)
    dv = torch.empty(B, L, M, dtype=v.dtype, device=dev)
    dobs = torch.empty(B, L, M, dtype=v.dtype, device=dev)
    dk, dq = torch.empty_like(k), torch.empty_like(q)
    da, dp = torch.empty_like(a), torch.empty_like(p)
    dlam0, deta0 = k.new_empty(B, M, S), k.new_empty(B, M, S)
    if B * M * S == 0:
        # No lanes: every gradient with entries (dk, dq over no channels, da, dp over no batch rows) is zero.
        for t in (dv, dobs, dk, dq, da, dp):
            t.zero_()
        return dv, dobs, dk, dq, da, dp, dlam0, deta0
    sn = _sensor_desc(v, obs, lds, log_var, obs_var_min, obs_var_max)
    pt = _lib.ptr

    def bwd(batch, steps, lam_fin_grad, eta_fin_grad, lam0_grad, eta0_grad, ws, nbytes):
        stream = _lib.stream(dev)
        _lib.check("kla_fused_scan_sensors_bwd", _lib.lib().kla_fused_scan_sensors_bwd(
            pt(dy), pt(dy_var), pt(lam_fin_grad), pt(eta_fin_grad), ctypes.byref(sn), pt(k), pt(q), pt(a), pt(p),
            pt(ck_lam), pt(ck_eta), pt(dv), pt(dobs), pt(dk), pt(dq), pt(da), pt(dp), pt(lam0_grad),
            pt(eta0_grad), int(decode_from_prior), batch, steps, M, S, pt(ws), nbytes, stream))

    nc = train_chunks(B, L, M, S, _cus(dev.index or 0))
    if nc > 1:
        dlam0, deta0 = _split_backward(bwd, dy, dy_var, dlam_fin, deta_fin, sn, k, q, a, p, ck_lam, ck_eta,
                                       decode_from_prior, B, L, M, S, nc, dev)
        return dv, dobs, dk, dq, da, dp, dlam0, deta0
    nbytes = int(_lib.lib().kla_fused_workspace_bytes(B, L, M, S))
    ws, _ = _lib.scratch(nbytes, dev)
    bwd(B, L, dlam_fin, deta_fin, dlam0, deta0, ws, ws.numel())
    return dv, dobs, dk, dq, da, dp, dlam0, deta0


@_sensors_bwd_op.register_fake
def _(dy, dy_var, dlam_fin, deta_fin, v, obs, k, q, a, p, ck_lam, ck_eta, log_var, obs_var_min, obs_var_max,
      decode_from_prior):
    B, L, M = v.shape
    S = k.shape[2]
    return (v.new_empty(B, L, M), v.new_empty(B, L, M), torch.empty_like(k), torch.empty_like(q),
            torch.empty_like(a), torch.empty_like(p), k.new_empty(B, M, S), k.new_empty(B, M, S))


def _sensors_setup(ctx, inputs, output):
    v, obs, k, q, a, p, lam0, eta0, log_var, obs_var_min, obs_var_max, decode_from_prior, save, with_var = inputs
    _, _, _, _, ck_lam, ck_eta = output
    if not save:
        raise RuntimeError("kla_scan_fused_sensors was run without checkpoints but a gradient is required")
    ctx.opts = (log_var, obs_var_min, obs_var_max, decode_from_prior)
    ctx.has_lam0, ctx.has_eta0 = lam0 is not None, eta0 is not None
    ctx.save_for_backward(v, obs, k, q, a, p, ck_lam, ck_eta)
    ctx.set_materialize_grads(False)


def _sensors_backward(ctx, dy, dy_var, dlam_fin, deta_fin, _dck_lam, _dck_eta):
    v, obs, k, q, a, p, ck_lam, ck_eta = ctx.saved_tensors

    def f32(t):
        return None if t is None or t.numel() == 0 else t.to(_F32).contiguous()

    B, L, M = v.shape
    dy = k.new_zeros(B, L, M) if dy is None else f32(dy)
    dv, dobs, dk, dq, da, dp, dlam0, deta0 = _lib.call(_sensors_bwd_op,
        dy, f32(dy_var), f32(dlam_fin), f32(deta_fin), v, obs, k, q, a, p, ck_lam, ck_eta, *ctx.opts)
    return (dv, dobs, dk, dq, da, dp, dlam0 if ctx.has_lam0 else None, deta0 if ctx.has_eta0 else None,
            None, None, None, None, None, None)


_sensors_fwd_op.register_autograd(_sensors_backward, setup_context=_sensors_setup)


def kla_scan_fused_sensors(v, obs, k, q, a, p, lam0=None, eta0=None, *, log_var: bool = True,
                           obs_var_min: float = 1e-4, obs_var_max: Optional[float] = None,
                           decode_from_prior: bool = False, with_var: bool = True):
    """(y, y_var, lam_fin, eta_fin) of the KLA scan with the layer's sensor read-out fused in.

    v and obs are [B, L, M] -- views such as column slices of the sensor
    projection are read in place. With ``log_var`` obs is log sigma^2 and
    lambda_v = 1 / min(softplus(obs) + obs_var_min, obs_var_max) is formed in
    the kernel, as KLALayer._project_sensors forms it (reference
    kla_layer.py:224-230); otherwise obs is lambda_v. bf16 sensors stay bf16 and
    their gradients come back in bf16; fp32 otherwise. k, q, a, p and the state
    are computed in fp32. With ``with_var=False`` y_var is not computed and comes
    back as None.
    """
    if v.dtype != obs.dtype or v.dtype not in (torch.float32, torch.bfloat16):
        v, obs = v.float(), obs.float()
    if _sensor_rows(v) is None:
        v = v.contiguous()
    if _sensor_rows(obs) is None:
        obs = obs.contiguous()
    a, p = _dynamics(a, p, v.shape[-1], k.shape[-1])
    k, q, lam0, eta0 = (_f32(t) for t in (k, q, lam0, eta0))
    save = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (v, obs, k, q, a, p, lam0, eta0))
    ov_max = math.inf if obs_var_max is None else float(obs_var_max)
    y, y_var, lam_fin, eta_fin, _, _ = _lib.call(_sensors_fwd_op, v, obs, k, q, a, p, lam0, eta0, bool(log_var),
                                                  float(obs_var_min), ov_max, bool(decode_from_prior), save,
                                                  bool(with_var))
    return y, (y_var if with_var else None), lam_fin, eta_fin
