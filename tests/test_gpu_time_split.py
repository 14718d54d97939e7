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
    assert L % nc == 0, "chunks must divide L"
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
    and the forward that saves checkpoints for a gradient (cut by the training
    planner, into 4) to the same bar."""
    B, L, M, S = 2, 1024, 1024, 16
    cus = fused._cus(cuda.index or 0)
    assert fused.time_chunks(B, L, M, S, cus) == 8
    assert fused.train_chunks(B, L, M, S, cus) == 4
    calls = []
    split = fused._split_forward
    monkeypatch.setattr(fused, "_split_forward", lambda *a, **kw: calls.append(a[-2]) or split(*a, **kw))
    ins = make_inputs(B, L, M, S, seed=24)
    xs = [t.to(cuda) for t in ins]
    y, y_var, fin = kla_scan(*xs, backend="hip_fused")
    assert calls == [8]
    wy, wv, wl, we = oracle(ins)
    for name, got, want in (("y", y, wy), ("y_var", y_var, wv), ("lam", fin.lam, wl), ("eta", fin.eta, we)):
        check_scan(name, got, want)
    # With a gradient to save for, the training planner's 4 chunks: the same numbers to the same bar.
    ws = [t.clone().requires_grad_(True) for t in xs]
    y2, y_var2, fin2 = kla_scan(*ws, backend="hip_fused")
    for name, got, want in (("y", y2, wy), ("y_var", y_var2, wv), ("lam", fin2.lam, wl), ("eta", fin2.eta, we)):
        check_scan(name, got, want)
    assert calls == [8, 4]


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


# ------------------------------------------------------------ training (backward)
#
# With a gradient to save for, small grids split as well (kla.ops.hip.fused.
# train_chunks): the forward keeps its checkpoints on the chunk view (the same
# memory as the whole sequence's), a pass composes each chunk's adjoint steps
# into an affine map with an upper-triangular linear part, a walk over the maps
# from the end of each sequence gives every chunk the adjoint entering it from
# the right, and the fused backward runs on the view from those. Parity bar: the
# fused scan's against float64 autograd of the reference's torch path.


@pytest.fixture
def train_chunks(monkeypatch):
    """force(nc) makes the training planner return nc for every call in the test."""

    def force(nc):
        monkeypatch.setattr(fused, "train_chunks", lambda B, L, M, S, cus: nc)

    return force


# (shape, chunk count) pairs whose chunks hold whole 16-step checkpoint blocks.
_TRAIN_SPLITS = [(shape, nc)
                 for shape in [(2, 256, 9, 16), (1, 128, 3, 128), (3, 320, 70, 4), (1, 256, 2, 256), (2, 192, 5, 32)]
                 for nc in (2, 4, 8) if shape[1] % (16 * nc) == 0]


@pytest.mark.parametrize("shape,nc", _TRAIN_SPLITS)
@pytest.mark.parametrize("with_state", [False, True])
@pytest.mark.parametrize("decode_from_prior", [False, True])
@pytest.mark.parametrize("with_var", [True, False])
def test_forced_training_split_matches_float64_autograd(cuda, train_chunks, shape, nc, with_state,
                                                        decode_from_prior, with_var):
    from oracle import torch_ref

    B, L, M, S = shape
    print(f"[training split] shape={shape} nc={nc} state={with_state} prior={decode_from_prior} "
          f"var={with_var}", flush=True)
    train_chunks(nc)
    ins = make_inputs(B, L, M, S, seed=31)
    st = random_state(B, M, S, seed=32)
    g = torch.Generator().manual_seed(33)
    wy, wv = torch.randn(B, L, M, generator=g), torch.randn(B, L, M, generator=g)
    wl, we = torch.randn(B, M, S, generator=g), torch.randn(B, M, S, generator=g)

    def loss(y, y_var, lam, eta):
        w = [t.to(device=y.device, dtype=y.dtype) for t in (wy, wv, wl, we)]
        var_term = (w[1] * y_var).sum() if with_var else 0.0
        return (w[0] * y).sum() + var_term + (w[2] * lam).sum() + (w[3] * eta).sum()

    extra = (st.lam, st.eta) if with_state else ()
    xs = [t.double().requires_grad_(True) for t in ins + extra]
    ref = torch_ref.kla_scan_torch(*xs, decode_from_prior=decode_from_prior)
    loss(*ref).backward()
    gs = [t.to(cuda).requires_grad_(True) for t in ins + extra]
    state = KLAState(gs[6], gs[7]) if with_state else None
    y, y_var, fin = kla_scan(*gs[:6], backend="hip_fused", initial_state=state, decode_from_prior=decode_from_prior)
    for name, got, want in zip(("y", "y_var", "lam", "eta"), (y, y_var, fin.lam, fin.eta), ref):
        check_scan(name, got, want.detach().numpy())
    loss(y, y_var, fin.lam, fin.eta).backward()
    for name, got, want in zip(("v", "lambda_v", "k", "q", "a", "p", "lam0", "eta0"), gs, xs):
        check_scan("d" + name, got.grad, want.grad.numpy())


@pytest.mark.parametrize("nc", [2, 4])
def test_forced_training_split_of_sensors(cuda, train_chunks, nc):
    """The layer's training path (kla_scan_fused_sensors on projection columns):
    fp32 columns against float64 autograd of the read-out tail and the reference's
    filter, and bf16 columns equal to the fp32 run on the widened values bit for
    bit, as for the whole sequence (dv, d log sigma^2 rounded to bf16)."""
    import torch.nn.functional as F

    from kla.ops.hip.fused import kla_scan_fused_sensors
    from oracle import torch_ref

    B, L, M, S = 2, 256, 20, 16
    train_chunks(nc)
    _, _, k, q, a, p = make_inputs(B, L, M, S, seed=34)
    g = torch.Generator().manual_seed(35)
    proj16 = (torch.randn(B, L, 2 * M + 3, generator=g) * 1.5).to(torch.bfloat16)
    proj = proj16.float()
    st = random_state(B, M, S, seed=36)
    wy, wl = torch.randn(B, L, M, generator=g), torch.randn(B, M, S, generator=g)

    def views(t):
        return t[..., :M], t[..., M + 1:2 * M + 1]

    xs = [t.double().requires_grad_(True) for t in (proj, k, q, a, p, st.lam, st.eta)]
    v64, lv64 = views(xs[0])
    ref = torch_ref.kla_scan_torch(v64, 1.0 / (F.softplus(lv64) + 1e-4), *xs[1:])
    ((wy.double() * ref[0]).sum() + (wl.double() * ref[2]).sum()).backward()
    runs = []
    for pj in (proj, proj16):
        gs = [t.to(cuda).requires_grad_(True) for t in (pj, k, q, a, p, st.lam, st.eta)]
        y, _, lam, _ = kla_scan_fused_sensors(*views(gs[0]), *gs[1:], with_var=False)
        ((wy.to(cuda) * y).sum() + (wl.to(cuda) * lam).sum()).backward()
        runs.append([y, lam] + [t.grad for t in gs])
    check_scan("y", runs[0][0], ref[0].detach().numpy())
    check_scan("lam", runs[0][1], ref[2].detach().numpy())
    for name, got, want in zip(("dproj", "dk", "dq", "da", "dp", "dlam0", "deta0"), runs[0][2:], xs):
        check_scan(name, got, want.grad.numpy())
    f32, b16 = runs
    for i, name in enumerate(("y", "lam", "dproj", "dk", "dq", "da", "dp", "dlam0", "deta0")):
        want = f32[i].to(torch.bfloat16) if name == "dproj" else f32[i]
        assert torch.equal(b16[i], want), name


def test_training_planner_at_c1_matches_whole_backward(cuda, monkeypatch):
    """At C1's shape with gradients (B=2, L=1024, M=1024, S=16: 128 workgroups) the
    training planner cuts 4 chunks; every output and gradient of the split pair
    against the whole pair (the training planner forced to 1), at the scan's bar
    relative to the whole run."""
    B, L, M, S = 2, 1024, 1024, 16
    assert fused.train_chunks(B, L, M, S, fused._cus(cuda.index or 0)) == 4
    ins = [t.to(cuda) for t in make_inputs(B, L, M, S, seed=37)]
    st = random_state(B, M, S, seed=38)
    g = torch.Generator(device="cpu").manual_seed(39)
    wy, wv = torch.randn(B, L, M, generator=g).to(cuda), torch.randn(B, L, M, generator=g).to(cuda)
    runs = []
    for force in (None, 1):
        if force is not None:
            monkeypatch.setattr(fused, "train_chunks", lambda *a: 1)
        gs = [t.clone().requires_grad_(True) for t in ins + [st.lam.to(cuda), st.eta.to(cuda)]]
        y, y_var, fin = kla_scan(*gs[:6], backend="hip_fused", initial_state=KLAState(gs[6], gs[7]))
        ((wy * y).sum() + (wv * y_var).sum() + fin.lam.sum() + fin.eta.square().sum()).backward()
        runs.append([y, y_var, fin.lam, fin.eta] + [t.grad for t in gs])
    names = ("y", "y_var", "lam", "eta", "dv", "dlambda_v", "dk", "dq", "da", "dp", "dlam0", "deta0")
    for name, got, want in zip(names, *runs):
        check_scan(name, got, want.detach().double().cpu().numpy())


def _cold_start_inputs():
    """lam0 = 0, eta0 = 0 under decay (a = 0.8, p = 0.03) with state lane s = 0 of
    every channel nearly unobserved (phi = 4e-12, above the filter's EPS floor) for
    the whole first chunk of 128 steps: the chunk's composed map carries a
    denominator entry d1 below 1e-12, which chunk_starts_kernel must not floor at
    EPS (the map algebra of this case is pinned in tests/test_time_split_algebra.py).
    An EPS floor there leaves that lane's lam entering chunk 1 about 3x too low,
    which y, lam and eta of the second chunk show."""
    B, L, M, S = 1, 256, 8, 16
    v, lv, k, q, _, _ = make_inputs(B, L, M, S, seed=41)
    lv[:, :128] = 1.0
    k[:, :128, 0] = 2e-6
    # The cold lane is not read out while cold (its mean eta / lam ~ 1e5 would make
    # y ill-conditioned in fp32 over the first chunk); its state still enters chunk 1.
    q[:, :128, 0] = 0.0
    a, p = torch.full((M, S), 0.8), torch.full((M, S), 0.03)
    return (v, lv, k, q, a, p), KLAState(torch.zeros(B, M, S), torch.zeros(B, M, S))


def test_forced_split_from_a_cold_start_matches_oracle(cuda, chunks):
    ins, st = _cold_start_inputs()
    print("[time split] cold start, nc=2", flush=True)
    chunks(2)
    y, y_var, fin = kla_scan(*(t.to(cuda) for t in ins), backend="hip_fused", initial_state=_state(st, cuda))
    wy, wv, wl, we = oracle(ins, st)
    assert wl.min() > 0
    for name, got, want in (("y", y, wy), ("y_var", y_var, wv), ("lam", fin.lam, wl), ("eta", fin.eta, we)):
        check_scan(name, got, want)


def test_forced_training_split_from_a_cold_start_matches_float64_autograd(cuda, train_chunks):
    """The same inputs with gradients (2 training chunks) against float64 autograd of
    the step-by-step form of the reference's scan (torch_ref.kla_scan_stepwise: no
    phi floor, exact from lam0 = 0, where the doubling form's trace-normalised
    prefixes lose precision)."""
    from oracle import torch_ref

    ins, st = _cold_start_inputs()
    print("[training split] cold start, nc=2", flush=True)
    train_chunks(2)
    B, L, M, S = ins[2].shape[0], ins[2].shape[1], ins[0].shape[2], ins[2].shape[2]
    g = torch.Generator().manual_seed(42)
    wy, wl, we = torch.randn(B, L, M, generator=g), torch.randn(B, M, S, generator=g), torch.randn(B, M, S, generator=g)

    def loss(y, lam, eta):
        w = [t.to(device=y.device, dtype=y.dtype) for t in (wy, wl, we)]
        return (w[0] * y).sum() + (w[1] * lam).sum() + (w[2] * eta).sum()

    xs = [t.double().requires_grad_(True) for t in ins + (st.lam, st.eta)]
    ref = torch_ref.kla_scan_stepwise(*xs)
    loss(ref[0], ref[2], ref[3]).backward()
    gs = [t.to(cuda).requires_grad_(True) for t in ins + (st.lam, st.eta)]
    y, _, fin = kla_scan(*gs[:6], backend="hip_fused", initial_state=KLAState(gs[6], gs[7]))
    for name, got, want in zip(("y", "lam", "eta"), (y, fin.lam, fin.eta), (ref[0], ref[2], ref[3])):
        check_scan(name, got, want.detach().numpy())
    loss(y, fin.lam, fin.eta).backward()
    for name, got, want in zip(("v", "lambda_v", "k", "q", "a", "p", "lam0", "eta0"), gs, xs):
        check_scan("d" + name, got.grad, want.grad.numpy())
