"""The time-split forward of the fused KLA scan (inference at small batch).

Without a gradient to save for, the fused forward cuts each sequence into nc
chunks when the plain grid (batch x channel groups) would leave the CUs idle
(kla.ops.hip.fused.time_chunks): one pass composes each chunk's steps into a
3x3 map of the state in homogeneous coordinates (lam = N / D, eta = W / D), a
short walk chains the maps into every chunk's entering state, and the fused
forward runs on the [B * nc, L / nc] view from those states. This is the
chunked forward of the reference's tiled kernel
(src/kla/ops/kernels/mps/tiled_kla_scan.metal:1-35), with its two composition
rounds (precision, then information) folded into one.

Parity bar: the scan's fp32 tolerance against the float64 sequential filter,
|got - want| <= 1e-6 + 1e-5 |want| (check_scan), on chunk counts forced onto
small shapes (with and without an initial state, the prior read-out, bf16
sensors through softplus) and at C1's shape with the count the planner picks.
The map algebra itself is pinned on the CPU (tests/test_time_split_algebra.py).
"""

import pytest
import torch

from kla.ops import KLAState, kla_scan
from kla.ops.hip import fused
from test_gpu_backend import check_scan, make_inputs, oracle, random_state

pytestmark = pytest.mark.gpu


@pytest.fixture
def chunks(monkeypatch):
    """force(nc) makes the planner return nc for every call in the test."""

    def force(nc):
        monkeypatch.setattr(fused, "time_chunks", lambda B, L, M, S, cus: nc)

    return force


def _state(st, cuda):
    return None if st is None else KLAState(st.lam.to(cuda), st.eta.to(cuda))


@pytest.mark.parametrize("shape", [(2, 512, 9, 16), (1, 256, 3, 128), (1, 128, 2, 256), (3, 320, 70, 4)])
@pytest.mark.parametrize("nc", [2, 4, 16])
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("decode_from_prior", [False, True])
def test_forced_split_matches_oracle(cuda, chunks, shape, nc, with_state, decode_from_prior):
    B, L, M, S = shape
    if L % nc:
        pytest.skip("chunks must divide L")
    print(f"[time split] shape={shape} nc={nc} state={with_state} prior={decode_from_prior}", flush=True)
    chunks(nc)
    ins = make_inputs(B, L, M, S, seed=21)
    st = random_state(B, M, S, seed=4) if with_state else None
    y, y_var, fin = kla_scan(*(t.to(cuda) for t in ins), backend="hip_fused", decode_from_prior=decode_from_prior,
                             initial_state=_state(st, cuda))
    wy, wv, wl, we = oracle(ins, st, decode_from_prior)
    for name, got, want in (("y", y, wy), ("y_var", y_var, wv), ("lam", fin.lam, wl), ("eta", fin.eta, we)):
        check_scan(name, got, want)


@pytest.mark.parametrize("nc", [1, 4])
@pytest.mark.parametrize("with_var", [True, False])
def test_forced_split_of_bf16_sensors_matches_oracle(cuda, chunks, nc, with_var):
    """bf16 projection columns through softplus and the clamp (the layer's inference
    path, kla_layer.py:224-230), split and whole, against the float64 filter on the
    widened values."""
    import torch.nn.functional as F

    from kla.ops.hip.fused import kla_scan_fused_sensors

    B, L, M, S = 1, 512, 24, 16
    chunks(nc)
    _, _, k, q, a, p = make_inputs(B, L, M, S, seed=22)
    g = torch.Generator().manual_seed(23)
    proj = (torch.randn(B, L, 2 * M + 3, generator=g) * 1.5).to(torch.bfloat16)
    v, lv = proj[..., :M], proj[..., M + 1:2 * M + 1]
    ov_min, ov_max = 1e-4, 4.0
    lam_v = 1.0 / (F.softplus(lv.double()) + ov_min).clamp_max(ov_max)
    st = random_state(B, M, S, seed=6)
    wy, wv, wl, we = oracle((v.double(), lam_v, k, q, a, p), st)
    pj = proj.to(cuda)
    y, y_var, lam, eta = kla_scan_fused_sensors(pj[..., :M], pj[..., M + 1:2 * M + 1],
                                                *(t.to(cuda) for t in (k, q, a, p)), st.lam.to(cuda),
                                                st.eta.to(cuda), obs_var_min=ov_min, obs_var_max=ov_max,
                                                with_var=with_var)
    assert (y_var is None) == (not with_var)
    check_scan("y", y, wy)
    if with_var:
        check_scan("y_var", y_var, wv)
    check_scan("lam", lam, wl)
    check_scan("eta", eta, we)


def test_planner_splits_c1_and_matches_oracle(cuda, monkeypatch):
    """At C1's scan shape (B=2, L=1024, M=1024, S=16) the planner cuts 8 chunks
    (128 workgroups -> 1024); split outputs against the float64 filter on whole tensors,
    and the whole forward (taken when a gradient is to be saved for) to the same bar."""
    B, L, M, S = 2, 1024, 1024, 16
    assert fused.time_chunks(B, L, M, S, fused._cus(cuda.index or 0)) == 8
    calls = []
    split = fused._split_forward
    monkeypatch.setattr(fused, "_split_forward", lambda *a: calls.append(a[-2]) or split(*a))
    ins = make_inputs(B, L, M, S, seed=24)
    xs = [t.to(cuda) for t in ins]
    y, y_var, fin = kla_scan(*xs, backend="hip_fused")
    assert calls == [8]
    wy, wv, wl, we = oracle(ins)
    for name, got, want in (("y", y, wy), ("y_var", y_var, wv), ("lam", fin.lam, wl), ("eta", fin.eta, we)):
        check_scan(name, got, want)
    # With a gradient to save for, the forward runs whole: the same numbers to the same bar.
    ws = [t.clone().requires_grad_(True) for t in xs]
    y2, y_var2, fin2 = kla_scan(*ws, backend="hip_fused")
    for name, got, want in (("y", y2, wy), ("y_var", y_var2, wv), ("lam", fin2.lam, wl), ("eta", fin2.eta, we)):
        check_scan(name, got, want)
    assert calls == [8], "a forward that saves checkpoints runs whole"


def test_split_chunked_prefill_carries_state(cuda):
    """Two prefill pieces, each split, carry the state as one whole pass does."""
    B, L, M, S = 1, 1024, 64, 16
    ins = make_inputs(B, L, M, S, seed=25)
    xs = [t.to(cuda) for t in ins]
    assert fused.time_chunks(B, 512, M, S, fused._cus(cuda.index or 0)) > 1
    y1, _, st1 = kla_scan(*(t[:, :512] if t.dim() == 3 else t for t in xs), backend="hip_fused")
    y2, _, st2 = kla_scan(*(t[:, 512:] if t.dim() == 3 else t for t in xs), backend="hip_fused", initial_state=st1)
    wy, _, wl, we = oracle(ins)
    check_scan("y", torch.cat([y1, y2], 1), wy)
    check_scan("lam", st2.lam, wl)
    check_scan("eta", st2.eta, we)
