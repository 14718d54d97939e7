"""The k, q sensors in one kernel (kla_rows_linear_qk_fwd): the sensor
projection's last 2 S rows, the l2 norm over S and the clamp (reference
src/kla/layers/kla_layer.py:205-222), against float64 torch, and the inference
layer path that uses it against the torch backend."""

import pytest
import torch

from kla import KLAConfig, KLALayer
from kla.ops.hip import sensors

pytestmark = pytest.mark.gpu


def _reference(x, w, b, S, norm, clip):
    """(k, q) in float64 and, per row, the factor a product error is scaled by on
    the way out: 1 / ||row|| after the l2 norm (a short row's direction carries
    its components' fp32 rounding divided by its length), else 1."""
    a = x.double() @ w.double().t() + (b.double() if b is not None else 0.0)
    k, q = a[:, :S], a[:, S:]
    gk = gq = torch.ones(a.shape[0], 1, dtype=torch.float64)
    if norm:
        nk, nq = k.norm(dim=-1, keepdim=True).clamp_min(1e-12), q.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        k, q = k / nk, q / nq
        gk, gq = (1.0 / nk).clamp_min(1.0), (1.0 / nq).clamp_min(1.0)
    if clip is not None:
        k, q = k.clamp(-clip, clip), q.clamp(-clip, clip)
    return (k, gk), (q, gq)


@pytest.mark.parametrize("S", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("rows,K", [(1, 64), (37, 1000), (2048, 1024), (300, 21)])
@pytest.mark.parametrize("norm,clip", [(True, None), (True, 0.3), (False, 2.0), (False, None)])
def test_qk_project_matches_float64(cuda, S, rows, K, norm, clip):
    print(f"[qk project] S={S} rows={rows} K={K} norm={norm} clip={clip}", flush=True)
    g = torch.Generator().manual_seed(S * 1000 + rows + K)
    x = torch.randn(rows, K, generator=g)
    w = torch.randn(2 * S, K, generator=g) / K ** 0.5
    b = torch.randn(2 * S, generator=g) * 0.1
    rk, rq = _reference(x, w, b, S, norm, clip)
    k, q = sensors.qk_project_hip(x.to(cuda), w.to(cuda), b.to(cuda), S, norm=norm, clip=clip)
    # fp32 bar: 1e-6 + 1e-5 |want|, the absolute part scaled by the norm's 1 / ||row||.
    for got, (want, gain) in ((k, rk), (q, rq)):
        assert got.shape == (rows, S) and got.dtype == torch.float32
        err = (got.double().cpu() - want).abs() / (1e-6 * gain + 1e-5 * want.abs())
        assert err.max().item() <= 1.0, f"worst ratio {err.max().item():.3g}"


def test_layer_inference_takes_the_kernel_and_matches_torch(cuda, monkeypatch):
    """KLALayer(512, d_state=16) inference on hip runs the k, q sensors through
    qk_project_hip and agrees with the torch backend (float64 on the CPU)."""
    torch.manual_seed(0)
    layer = KLALayer(512, KLAConfig(d_state=16, backend="hip"))
    x = torch.randn(2, 256, 512, generator=torch.Generator().manual_seed(1))
    ref_layer = KLALayer(512, KLAConfig(d_state=16, backend="torch"))
    ref_layer.load_state_dict(layer.state_dict())
    with torch.no_grad():
        want = ref_layer.double()(x.double())
    calls = []
    orig = sensors.qk_project_hip
    monkeypatch.setattr(sensors, "qk_project_hip", lambda *a, **k: calls.append(1) or orig(*a, **k))
    layer.to(cuda)
    with torch.no_grad():
        got = layer(x.to(cuda)).double().cpu()
    assert calls, "the inference path did not run qk_project_hip"
    err = ((got - want).abs().max() / want.abs().max()).item()
    assert err < 1e-5, err


def test_training_and_autocast_forwards_keep_the_differentiable_path(cuda, monkeypatch):
    """The kernel has no backward and computes in fp32: a forward that records a
    gradient, or one under bf16 autocast, keeps the split product and the qk
    sensor op, and its gradients still flow to the sensor projection's k, q rows."""
    torch.manual_seed(0)
    layer = KLALayer(512, KLAConfig(d_state=16, backend="hip")).to(cuda)
    x = torch.randn(2, 64, 512, device=cuda)
    calls = []
    orig = sensors.qk_project_hip
    monkeypatch.setattr(sensors, "qk_project_hip", lambda *a, **k: calls.append(1) or orig(*a, **k))
    layer(x).square().mean().backward()
    g = layer.sensor_proj.weight.grad
    assert g is not None and g[-32:].abs().sum().item() > 0
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        layer(x)
    assert not calls
