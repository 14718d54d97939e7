"""Every compiled variant of the fused KLA kernels, run and checked.

The fused forward, backward, chunk-map and adjoint-map kernels are compiled per
(SP, PRIOR, BF16, VAR): SP the channel's lanes rounded up to a power of two
(4 ... 256), PRIOR the read-out from the prior (decode_from_prior), BF16 bf16
sensor columns, VAR whether the variance read-out (and its adjoint) runs. The
sensor-fed op reaches all of them: fp32 runs are checked against float64
autograd of the reference's torch algorithm behind the layer's sensor read-out
(softplus, clamp, reciprocal: reference kla_layer.py:224-230), and bf16 runs,
whose arithmetic is the fp32 path's on exactly widened values, must equal the
fp32 run on those values bit for bit (dv, d log sigma^2 rounded once to bf16).
Each case runs whole (split 1) and with the time split forced to two chunks:
for training the chunk maps, the adjoint maps and both walks; for inference
the chunk maps and the forward from the chunk starts.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import torch_ref
from test_gpu_backend import _projection, _views, check_scan, make_inputs, random_state

pytestmark = pytest.mark.gpu

# (SP, S): one state width per compiled lane count, ragged where it can be.
WIDTHS = [(4, 3), (8, 8), (16, 13), (32, 32), (64, 50), (128, 128), (256, 200)]
B, L, M = 1, 64, 3
OV_MIN, OV_MAX = 1e-4, 1.5


def _case(S, seed):
    _, _, k, q, a, p = make_inputs(B, L, M, S, seed=seed)
    st = random_state(B, M, S)
    g = torch.Generator().manual_seed(seed + 1)
    w = [torch.randn(B, L, M, generator=g), torch.randn(B, L, M, generator=g),
         torch.randn(B, M, S, generator=g), torch.randn(B, M, S, generator=g)]
    return k, q, a, p, st, w


def _loss(out, w, with_var):
    y, y_var, lam, eta = out
    ww = [t.to(device=y.device, dtype=y.dtype) for t in w]
    var_term = (ww[1] * y_var).sum() if with_var else 0.0
    return (ww[0] * y).sum() + var_term + (ww[2] * lam).sum() + (ww[3] * eta).sum()


def _force_split(monkeypatch, split):
    from kla.ops.hip import fused

    if split > 1:
        monkeypatch.setattr(fused, "train_chunks", lambda *a: split)
        monkeypatch.setattr(fused, "time_chunks", lambda *a: split)
    else:
        monkeypatch.setattr(fused, "train_chunks", lambda *a: 1)
        monkeypatch.setattr(fused, "time_chunks", lambda *a: 1)


def _run(cuda, proj, k, q, a, p, st, w, prior, with_var, grad):
    """(outputs, gradients of proj, k, q, a, p, lam0, eta0) of the sensor-fed op."""
    from kla.ops.hip.fused import kla_scan_fused_sensors

    xs = [t.to(cuda) for t in (proj, k, q, a, p, st.lam, st.eta)]
    if grad:
        xs = [t.requires_grad_(True) for t in xs]
    v, lv = _views(xs[0], M)
    with torch.set_grad_enabled(grad):
        out = kla_scan_fused_sensors(v, lv, *xs[1:], log_var=True, obs_var_min=OV_MIN, obs_var_max=OV_MAX,
                                     decode_from_prior=prior, with_var=with_var)
        if grad:
            _loss(out, w, with_var).backward()
    return out, ([t.grad for t in xs] if grad else None)


@pytest.mark.parametrize("split", [1, 2])
@pytest.mark.parametrize("with_var", [False, True])
@pytest.mark.parametrize("prior", [False, True])
@pytest.mark.parametrize("sp,S", WIDTHS)
def test_fp32_variant_matches_float64_autograd(cuda, monkeypatch, sp, S, prior, with_var, split):
    """fp32 sensors: y, y_var, the final state and every gradient (through the
    projection, the sensor transform, and the state) against float64 autograd."""
    print(f"[variants] fp32 SP={sp} S={S} prior={prior} var={with_var} split={split}", flush=True)
    _force_split(monkeypatch, split)
    k, q, a, p, st, w = _case(S, seed=3 * sp + 1)
    proj = _projection(B, L, M, S, seed=sp)
    xs = [t.double().requires_grad_(True) for t in (proj, k, q, a, p, st.lam, st.eta)]
    v64, lv64 = _views(xs[0], M)
    obs = (F.softplus(lv64) + OV_MIN).clamp_max(OV_MAX)
    ref = torch_ref.kla_scan_torch(v64, 1.0 / obs, *xs[1:], decode_from_prior=prior)
    _loss(ref, w, with_var).backward()
    out, grads = _run(cuda, proj, k, q, a, p, st, w, prior, with_var, grad=True)
    assert (out[1] is None) == (not with_var)
    for name, got, want in zip(("y", "y_var", "lam", "eta"), out, ref):
        if got is not None:
            check_scan(name, got, want.detach().numpy())
    for name, got, want in zip(("proj", "k", "q", "a", "p", "lam0", "eta0"), grads, xs):
        check_scan("d" + name, got, want.grad.numpy())


@pytest.mark.parametrize("split", [1, 2])
@pytest.mark.parametrize("with_var", [False, True])
@pytest.mark.parametrize("prior", [False, True])
@pytest.mark.parametrize("sp,S", WIDTHS)
def test_bf16_variant_equals_fp32_of_the_same_values(cuda, monkeypatch, sp, S, prior, with_var, split):
    """bf16 sensor columns against their exact fp32 widening: every fp32 output and
    gradient bit-identical, and the projection's gradient equal to the fp32 run's
    rounded to bf16 (nearest even)."""
    print(f"[variants] bf16 SP={sp} S={S} prior={prior} var={with_var} split={split}", flush=True)
    _force_split(monkeypatch, split)
    k, q, a, p, st, w = _case(S, seed=5 * sp + 2)
    proj16 = _projection(B, L, M, S, seed=sp + 100, dtype=torch.bfloat16)
    out16, g16 = _run(cuda, proj16, k, q, a, p, st, w, prior, with_var, grad=True)
    out32, g32 = _run(cuda, proj16.float(), k, q, a, p, st, w, prior, with_var, grad=True)
    for name, x, y in zip(("y", "y_var", "lam", "eta"), out16, out32):
        assert (x is None) == (y is None), name
        if x is not None:
            assert torch.equal(x, y), name
    assert g16[0].dtype == torch.bfloat16
    assert torch.equal(g16[0], g32[0].to(torch.bfloat16)), "dproj"
    for name, x, y in zip(("k", "q", "a", "p", "lam0", "eta0"), g16[1:], g32[1:]):
        assert torch.equal(x, y), "d" + name


@pytest.mark.parametrize("with_var", [False, True])
@pytest.mark.parametrize("prior", [False, True])
@pytest.mark.parametrize("sp,S", WIDTHS)
def test_inference_split_variants(cuda, monkeypatch, sp, S, prior, with_var):
    """Without gradients the time split runs the chunk maps and the forward from
    the chunk starts: fp32 against float64, bf16 bit-identical to fp32 on the
    same values."""
    print(f"[variants] inference split SP={sp} S={S} prior={prior} var={with_var}", flush=True)
    _force_split(monkeypatch, 2)
    k, q, a, p, st, w = _case(S, seed=7 * sp + 3)
    proj16 = _projection(B, L, M, S, seed=sp + 200, dtype=torch.bfloat16)
    out16, _ = _run(cuda, proj16, k, q, a, p, st, w, prior, with_var, grad=False)
    out32, _ = _run(cuda, proj16.float(), k, q, a, p, st, w, prior, with_var, grad=False)
    for name, x, y in zip(("y", "y_var", "lam", "eta"), out16, out32):
        assert (x is None) == (y is None), name
        if x is not None:
            assert torch.equal(x, y), name
    xs = [t.double() for t in (proj16.float(), k, q, a, p, st.lam, st.eta)]
    v64, lv64 = _views(xs[0], M)
    obs = (F.softplus(lv64) + OV_MIN).clamp_max(OV_MAX)
    ref = torch_ref.kla_scan_torch(v64, 1.0 / obs, *xs[1:], decode_from_prior=prior)
    for name, got, want in zip(("y", "y_var", "lam", "eta"), out32, ref):
        if got is not None:
            check_scan(name, got, want.numpy())
