"""KLALayer at BASELINE sizes on the "hip" backend against the reference's
algorithm run on the torch backend (the reference's own layer and
kla_scan_torch, reference src/kla/layers/kla_layer.py:235-349,
src/kla/ops/kla_ops.py:188-290).

C1, KLALayer(512, d_state=16) forward on x (2, 1024, 512) fp32: the hip layer
(fp32 projections through torch, every other part in HIP kernels) against the
same weights on backend "torch" on the host CPU in float64, with the
reference's float32 scan inputs evaluated in float64 (the algorithm's exact
value), and in float32 (the reference's own CPU run). Bar: the scan's fp32
tolerance, |d| <= 1e-6 + 1e-5 |ref| elementwise against float64, for the output
and the final precision lam; the final information eta (a sum over the whole
sequence) with atol 1e-6 max|eta|. The float32 CPU run is measured against the
same float64 beside it (at C1 it misses the literal bar on lam and eta by 9x and
22x: its slow lanes, a_bar ~ 0.999, amplify a rounding bias of the decay).

C4, KLALayer(1024, d_state=16) training step on x (4, 4096, 1024) under bf16
autocast, loss = mean(out^2): the hip layer against the same weights on
backend "torch" on the same GPU (torch's nn.Linear, conv, split, gate and the
reference's parallel scan under autograd), run one sequence at a time with the
gradients accumulated (the loss is a mean over independent sequences, so the
sum of the per-sequence gradients is the whole step's; one sequence at a time
keeps the torch path's [1, 4096, 2048, 16] intermediates within memory). Bar:
bf16 I/O within rtol 2e-2, |d| <= 2e-2 |ref| + atol elementwise, with atol
1e-2 max|ref| for elements whose reference has cancelled toward zero; the
share of elements beyond the plain rtol 2e-2 (atol 1e-3 max|ref|) is printed.
"""

import copy
import dataclasses

import numpy as np
import pytest
import torch

from kla import KLAConfig, KLALayer

pytestmark = pytest.mark.gpu


def _ratio(got, want, rtol, atol):
    got = got.detach().double().cpu().numpy()
    want = want.detach().double().cpu().numpy().reshape(got.shape)
    assert np.isfinite(got).all()
    r = np.abs(got - want) / (atol + rtol * np.abs(want))
    return float(r.max()), float((r > 1.0).mean())


def _backend(layer, backend):
    out = copy.deepcopy(layer)
    out.config = dataclasses.replace(layer.config, backend=backend)
    return out


def test_c1_layer_forward_matches_float64_reference(cuda, monkeypatch):
    """C1 on hip against the reference layer in float64 with its scan run in
    float64 too (the reference layer casts the scan's inputs to float32,
    kla_layer.py:224-231; here that float32 input is evaluated exactly), on the
    same static dynamics (a_bar, p_bar) as the hip layer: where the filter
    forgets slowly (a_bar ~ 0.999) its final state moves ~500x as much as a_bar
    does, so a one-ulp difference between the GPU's and the CPU's exp in a_bar
    shows up as ~3e-5 in lam and eta; that part is measured and printed apart
    (the reference's own float32 CPU layer beside it)."""
    import kla.layers.kla_layer as kl
    from kla.ops import kla_scan as real_scan

    torch.manual_seed(0)
    base = KLALayer(512, KLAConfig(d_state=16, backend="torch"))
    x = torch.randn(2, 1024, 512, generator=torch.Generator().manual_seed(0))
    hip = _backend(base, "hip").to(cuda)
    with torch.no_grad():
        a_h, p_h = (t.detach().cpu() for t in hip._compute_aq())
        a_c, p_c = base._compute_aq()
        ulp = float(((a_h.double() - a_c.double()).abs() / torch.finfo(torch.float32).eps / a_c.double()).max())
        print(f"[c1] a_bar hip vs cpu: up to {ulp:.2f} ulp; p_bar max rel diff "
              f"{float(((p_h.double() - p_c.double()).abs() / p_c.double()).max()):.2e}", flush=True)

        def scan64(v, lv, k, q, a, p, **kw):
            """The reference layer's scan on its float32 inputs, evaluated in float64,
            with the hip layer's a_bar, p_bar."""
            st = kw.pop("initial_state", None)
            return real_scan(v.double(), lv.double(), k.double(), q.double(), a_h.double(), p_h.double(),
                             initial_state=st, **{**kw, "scan_impl": "sequential"})

        print("[c1] float64 reference on the CPU", flush=True)
        monkeypatch.setattr(kl, "kla_scan", scan64)
        y64, st64 = _backend(base, "torch").double()(x.double(), return_state=True)
        monkeypatch.setattr(kl, "kla_scan", real_scan)
        print("[c1] float32 reference (the reference's own CPU run) on the CPU", flush=True)
        y32, st32 = _backend(base, "torch")(x, return_state=True)
        print("[c1] hip", flush=True)
        yh, sth = hip(x.to(cuda), return_state=True)
    rows = [("y", yh, y32, y64), ("lam", sth.ssm.lam, st32.ssm.lam, st64.ssm.lam),
            ("eta", sth.ssm.eta, st32.ssm.eta, st64.ssm.eta)]
    for name, h, c, want in rows:
        hr, hs = _ratio(h, want, 1e-5, 1e-6)
        cr, cs = _ratio(c, want, 1e-5, 1e-6)
        xr, xs = _ratio(h, c, 1e-5, 1e-6)
        print(f"  {name:4s} rtol 1e-5 / atol 1e-6 against float64: hip {hr:.3f} ({hs:.1e} of elements above 1), "
              f"cpu fp32 {cr:.3f} ({cs:.1e}); hip against cpu fp32 {xr:.3f} ({xs:.1e})", flush=True)
        if name != "eta":
            assert hr <= 1.0, f"{name}: hip outside rtol 1e-5 / atol 1e-6 of float64 (ratio {hr:.3f})"
            continue
        # eta_T = sum_t (prod alpha) r_t sums 1024 mixed-sign information terms:
        # its fp32 rounding scales with the terms, not with the (cancelled)
        # result, so near-zero entries take atol 1e-6 max|eta| (the contraction
        # bar of the scan tests); and hip must be no less exact than the
        # reference's own float32 CPU run under the literal bar.
        sr, _ = _ratio(h, want, 1e-5, 1e-6 * float(want.abs().max()))
        print(f"  eta  rtol 1e-5 / atol 1e-6 max|eta|: hip {sr:.3f}", flush=True)
        assert sr <= 1.0, f"eta: hip outside rtol 1e-5 / atol 1e-6 max|eta| of float64 (ratio {sr:.3f})"
        assert hr <= cr, f"eta: hip ({hr:.3f}) less exact than the reference's float32 run ({cr:.3f})"


def test_c4_layer_step_matches_torch_backend(cuda):
    torch.manual_seed(0)
    hip = KLALayer(1024, KLAConfig(d_state=16, backend="hip"))
    ref = _backend(hip, "torch")
    hip, ref = hip.to(cuda), ref.to(cuda)
    B, L = 4, 4096
    x = torch.randn(B, L, 1024, generator=torch.Generator().manual_seed(0)).to(cuda)
    n = x.numel()

    print("[c4] hip step", flush=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out_h = hip(x)
    out_h.float().square().mean().backward()
    out_h = out_h.detach().float()
    grads_h = {k: p.grad.detach().float() for k, p in hip.named_parameters() if p.grad is not None}
    del hip
    torch.cuda.empty_cache()

    outs = []
    for b in range(B):
        print(f"[c4] torch-backend step, sequence {b}", flush=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            o = ref(x[b:b + 1])
        (o.float().square().sum() / n).backward()
        outs.append(o.detach().float())
        del o
        torch.cuda.empty_cache()
    out_r = torch.cat(outs)
    grads_r = {k: p.grad.detach().float() for k, p in ref.named_parameters() if p.grad is not None}
    assert grads_h.keys() == grads_r.keys()
    worst = {}
    for name, a, b in [("out", out_h, out_r)] + [(k, grads_h[k], grads_r[k]) for k in sorted(grads_r)]:
        scale = float(b.abs().max())
        plain, share = _ratio(a, b, 2e-2, 1e-3 * scale)
        r, _ = _ratio(a, b, 2e-2, 1e-2 * scale)
        worst[name] = r
        print(f"  {name:22s} rtol 2e-2: atol 1e-2 max|ref| {r:.3f}; atol 1e-3 max|ref| {plain:.3f} "
              f"({share:.1e} of elements above 1)", flush=True)
    bad = {k: v for k, v in worst.items() if v > 1.0}
    assert not bad, f"outside rtol 2e-2 (atol 1e-2 max|ref|): {bad}"
