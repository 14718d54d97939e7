"""The kla package on the CPU: the torch backend, the dispatcher and its rules,
the numeric guards, and the layer / model API (no GPU needed).

Parity anchors are the float64 oracle (oracle.kla: sequential information form,
pinned against the covariance-form filter in test_oracle_pins.py). The cases
follow the reference's tests/test_ops.py, tests/test_backends.py (guards,
dispatch coverage) and tests/test_kla_layer.py (flags, decode parity, chunked
prefill).
"""

import math

import numpy as np
import pytest
import torch

from kla import KLAConfig, KLALayer, ModelConfig, SequenceModel
from kla.ops import (
    KLAState,
    backend_names,
    init_state,
    kla_scan,
    kla_scan_reference,
    kla_scan_torch,
    kla_step,
    resolve_backend,
)
from oracle import kla as okla


def make_inputs(B=2, L=64, M=16, S=8, dtype=torch.float32, requires_grad=False, seed=0):
    """Reference tests/test_backends.py:136-150: well-conditioned seeded inputs."""
    g = torch.Generator().manual_seed(seed)
    out = (
        torch.randn(B, L, M, generator=g),
        torch.rand(B, L, M, generator=g) + 0.5,
        torch.randn(B, L, S, generator=g) * 0.3,
        torch.randn(B, L, S, generator=g) * 0.3,
        torch.rand(M, S, generator=g) * 0.5 + 0.4,
        torch.rand(M, S, generator=g) * 0.05 + 0.01,
    )
    return tuple(t.to(dtype).requires_grad_(requires_grad) for t in out)


def oracle(inputs, state=None, decode_from_prior=False):
    np_in = [t.detach().double().numpy() for t in inputs]
    lam0 = None if state is None else state.lam.detach().double().numpy()
    eta0 = None if state is None else state.eta.detach().double().numpy()
    return okla.kla_scan_sequential(*np_in, lam0, eta0, decode_from_prior=decode_from_prior)


def close(got, want, rtol, atol):
    np.testing.assert_allclose(got.detach().double().numpy(), want, rtol=rtol, atol=atol)


# -------------------------------------------------------------- torch path


@pytest.mark.parametrize("scan_impl", ["doubling", "associative", "sequential"])
@pytest.mark.parametrize("mobius_impl", ["linear", "log"])
def test_torch_path_matches_oracle(scan_impl, mobius_impl):
    inputs = make_inputs()
    y, y_var, st = kla_scan_torch(*inputs, scan_impl=scan_impl, mobius_impl=mobius_impl)
    wy, wv, wl, we = oracle(inputs)
    close(y, wy, 1e-4, 2e-5)
    close(y_var, wv, 1e-4, 2e-5)
    close(st.lam, wl, 1e-4, 1e-4)
    close(st.eta, we, 1e-4, 1e-4)


@pytest.mark.parametrize("decode_from_prior", [False, True])
def test_float64_torch_path_is_the_filter(decode_from_prior):
    """In float64 the parallel torch path and the sequential filter agree to ~1e-12."""
    inputs = make_inputs(dtype=torch.float64, L=40)
    st0 = KLAState(lam=torch.full((2, 16, 8), 1.5, dtype=torch.float64),
                   eta=torch.randn(2, 16, 8, dtype=torch.float64))
    y, y_var, st = kla_scan_torch(*inputs, initial_state=st0, scan_impl="doubling",
                                  decode_from_prior=decode_from_prior)
    want = oracle(inputs, st0, decode_from_prior)
    for got, w in zip((y, y_var, st.lam, st.eta), want):
        close(got, w, 1e-10, 1e-12)
    assert y.dtype == torch.float64 and st.lam.dtype == torch.float64


@pytest.mark.parametrize("decode_from_prior", [False, True])
def test_step_matches_scan(decode_from_prior):
    """Reference tests/test_ops.py:38-60."""
    v, lv, k, q, a, p = make_inputs(L=16)
    y_ref, v_ref, _ = kla_scan_torch(v, lv, k, q, a, p, decode_from_prior=decode_from_prior)
    state = init_state(2, 16, 8)
    ys, vs = [], []
    for t in range(16):
        y_t, v_t, state = kla_step(v[:, t], lv[:, t], k[:, t], q[:, t], a, p, state,
                                   decode_from_prior=decode_from_prior)
        ys.append(y_t)
        vs.append(v_t)
    torch.testing.assert_close(torch.stack(ys, 1), y_ref, atol=2e-4, rtol=1e-4)
    torch.testing.assert_close(torch.stack(vs, 1), v_ref, atol=2e-4, rtol=1e-4)


def test_chunked_scan_with_state():
    """Reference tests/test_ops.py:63-75."""
    v, lv, k, q, a, p = make_inputs()
    y_full, v_full, _ = kla_scan_torch(v, lv, k, q, a, p)
    y1, v1, s = kla_scan_torch(v[:, :32], lv[:, :32], k[:, :32], q[:, :32], a, p)
    y2, v2, _ = kla_scan_torch(v[:, 32:], lv[:, 32:], k[:, 32:], q[:, 32:], a, p, initial_state=s)
    torch.testing.assert_close(torch.cat([y1, y2], 1), y_full, atol=2e-4, rtol=1e-4)
    torch.testing.assert_close(torch.cat([v1, v2], 1), v_full, atol=2e-4, rtol=1e-4)


def test_gradients_match_sequential_reference():
    """Reference tests/test_ops.py:78-86."""
    ins_p = make_inputs(L=32, requires_grad=True)
    ins_r = tuple(t.detach().clone().requires_grad_(True) for t in ins_p)
    y_p, v_p, _ = kla_scan_torch(*ins_p, scan_impl="doubling")
    y_r, v_r, _ = kla_scan_reference(*ins_r)
    (y_p.square().sum() + v_p.sum()).backward()
    (y_r.square().sum() + v_r.sum()).backward()
    for gp, gr in zip(ins_p, ins_r):
        torch.testing.assert_close(gp.grad, gr.grad, atol=2e-3, rtol=1e-3)


@pytest.mark.slow
def test_gradcheck_package_torch_path():
    """float64 central differences through the package's own torch path
    (reference tests/test_gradcheck.py:60-109)."""
    ins = make_inputs(B=1, L=8, M=3, S=2, dtype=torch.float64, requires_grad=True)

    def f(*a):
        y, y_var, _ = kla_scan_torch(*a, scan_impl="doubling")
        return y, y_var

    assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-5, rtol=1e-3)


def test_dtype_policy():
    """bf16/fp16 widen to float32, float64 is preserved (reference kla_ops.py:126-137)."""
    ins = make_inputs(L=8)
    y, _, _ = kla_scan_torch(*(t.bfloat16() if t.dim() == 3 else t for t in ins))
    assert y.dtype == torch.float32
    y, _, _ = kla_scan_torch(*(t.double() for t in ins))
    assert y.dtype == torch.float64


# ---------------------------------------------------------------- guards


@pytest.mark.parametrize("bad_p", [0.0, -0.05])
def test_non_positive_process_noise_stays_finite(bad_p):
    """Reference tests/test_backends.py:421-438."""
    v, lv, k, q, a, p = make_inputs()
    y, y_var, _ = kla_scan(v, lv, k, q, a, torch.full_like(p, bad_p), backend="torch")
    assert torch.isfinite(y).all() and torch.isfinite(y_var).all()


def test_near_zero_decay_stays_finite():
    """Reference tests/test_backends.py:441-493: a^2 floored at EPS."""
    v, lv, k, q, a, p = make_inputs()
    y, y_var, _ = kla_scan(v, lv, k, q, torch.full_like(a, 1e-10), p, backend="torch")
    assert torch.isfinite(y).all() and torch.isfinite(y_var).all()


def test_high_information_tokens_are_not_clipped():
    """Reference tests/test_backends.py:496-564: phi up to ~1e4 is not capped."""
    v, lv, k, q, a, p = make_inputs()
    lv = lv * 1e4
    assert (lv.unsqueeze(-1) * (k * k).unsqueeze(-2)).max() > 1e3
    y, y_var, _ = kla_scan(v, lv, k, q, a, p, backend="torch")
    wy, wv, _, _ = oracle((v, lv, k, q, a, p))
    rel = lambda g, w: float(np.abs(g.double().numpy() - w).max() / (np.abs(w).max() + 1.0))  # noqa: E731
    assert rel(y, wy) < 5e-3 and rel(y_var, wv) < 5e-3


def test_gradient_descent_reduces_loss():
    """Reference tests/test_backends.py:374-418 (projected Adam, 10 steps)."""
    inputs = make_inputs(requires_grad=True)
    _, lv, _, _, a, p = inputs
    target = torch.randn(2, 64, 16, generator=torch.Generator().manual_seed(1))
    opt = torch.optim.Adam(inputs, lr=1e-2)
    losses = []
    for _ in range(10):
        opt.zero_grad()
        y, _, _ = kla_scan(*inputs, backend="torch")
        loss = (y - target).pow(2).mean()
        loss.backward()
        opt.step()
        with torch.no_grad():
            lv.clamp_(min=1e-3)
            p.clamp_(min=1e-6)
            a.clamp_(min=1e-3, max=0.999)
        losses.append(loss.item())
    assert all(math.isfinite(x) for x in losses) and losses[-1] < losses[0]


# ------------------------------------------------------------- dispatcher


def test_dispatcher_rules():
    ins = make_inputs(L=8)
    y, _, st = kla_scan(*ins, backend="auto")
    assert y.shape == (2, 8, 16) and st.lam.shape == (2, 16, 8)
    assert resolve_backend("cpu") == "torch"
    with pytest.raises(ValueError, match="Unknown backend"):
        kla_scan(*ins, backend="nope")
    # The MI355X kernels refuse CPU tensors and name a backend that works.
    for name in ("hip", "hip_fused", "hip_composed"):
        with pytest.raises(NotImplementedError, match="torch"):
            kla_scan(*ins, backend=name)
    # Families whose kernels are not part of this build say so.
    for name in ("cuda", "triton", "mps_fused"):
        with pytest.raises(NotImplementedError, match="hip"):
            kla_scan(*ins, backend=name)
    with pytest.raises(ValueError, match="mobius_impl"):
        kla_scan_torch(*ins, mobius_impl="tracenorm")
    with pytest.raises(ValueError, match="scan_impl"):
        kla_scan(*ins, backend="torch", scan_impl="bogus")


# Every registry entry is parity-tested somewhere (reference
# tests/test_backends.py:972-998): where, or why it need not be.
COVERAGE = {
    "torch": "this file and test_oracle_pins.py",
    "hip": "tests/test_gpu_backend.py (GPU)",
    "hip_fused": "tests/test_gpu_backend.py (GPU); the default path of 'hip'",
    "hip_composed": "tests/test_gpu_backend.py (GPU)",
    "triton": "not in this build: raises NotImplementedError (test_dispatcher_rules)",
    "triton_fused": "not in this build: raises NotImplementedError",
    "triton_composed": "not in this build: raises NotImplementedError",
    "cuda": "not in this build: raises NotImplementedError (test_dispatcher_rules)",
    "cuda_v2_2": "not in this build: raises NotImplementedError",
    "cuda_v2_1": "not in this build: raises NotImplementedError",
    "mps": "not in this build: raises NotImplementedError",
    "mps_fused": "not in this build: raises NotImplementedError (test_dispatcher_rules)",
    "mps_tiled": "not in this build: raises NotImplementedError",
    "mps_composed": "not in this build: raises NotImplementedError",
}


def test_every_backend_is_covered():
    unaccounted = [n for n in backend_names() if n not in COVERAGE]
    assert not unaccounted, f"backend(s) {unaccounted} have no parity coverage"
    ins = make_inputs(L=4)
    for name, why in COVERAGE.items():
        if why.startswith("not in this build"):
            with pytest.raises(NotImplementedError):
                kla_scan(*ins, backend=name)


# ---------------------------------------------------------- layer / model


def _decode_parity(layer, x):
    layer.eval()
    with torch.no_grad():
        full = layer(x)
        full = full[0] if isinstance(full, tuple) else full
        state = layer.init_state(x.shape[0])
        outs = []
        for t in range(x.shape[1]):
            out, state = layer(x[:, t:t + 1], state=state)
            outs.append(out[0] if isinstance(out, tuple) else out)
    return (full - torch.cat(outs, 1)).abs().max().item()


@pytest.mark.parametrize(
    "kwargs",
    [
        dict(),
        dict(discretization="zoh"),
        dict(use_conv=False),
        dict(use_gating=False),
        dict(use_lambda_skip=False),
        dict(lambda_skip_mode="vector"),
        dict(qk_norm=False),
        dict(zero_process_noise=True),
        dict(learnable_process_noise=False),
        dict(clip_value=5.0),
        dict(obs_var_max=10.0),
        dict(decode_from_prior=True),
        dict(checkpoint_ssm=True),
        dict(scan_impl="doubling"),
        dict(scan_impl="sequential"),
        dict(expand=1.5),
        dict(bias=True),
        dict(value_rank="conv", var_rank="dt"),
        dict(value_rank=16, var_rank=4),
    ],
)
def test_layer_flag_space(kwargs):
    """Reference tests/test_kla_layer.py:26-76: train step finite, decode parity."""
    torch.manual_seed(0)
    layer = KLALayer(32, KLAConfig(d_state=4, **kwargs))
    x = torch.randn(2, 12, 32)
    y = layer(x)
    y = y[0] if isinstance(y, tuple) else y
    assert y.shape == x.shape and torch.isfinite(y).all()
    y.sum().backward()
    assert all(p.grad is None or torch.isfinite(p.grad).all() for p in layer.parameters())
    assert _decode_parity(layer, x) < 1e-4


def test_layer_return_variance_and_chunked_prefill():
    torch.manual_seed(0)
    layer = KLALayer(32, KLAConfig(d_state=4, return_variance=True))
    x = torch.randn(2, 24, 32)
    y, y_var = layer(x)
    assert y.shape == y_var.shape == x.shape and (y_var >= 0).all()
    layer = KLALayer(32, KLAConfig(d_state=4)).eval()
    with torch.no_grad():
        full = layer(x)
        state = layer.init_state(2)
        y1, state = layer(x[:, :10], state=state)
        y2, state = layer(x[:, 10:], state=state)
    torch.testing.assert_close(torch.cat([y1, y2], 1), full, atol=1e-4, rtol=1e-4)


def test_sequence_model_prefill_and_decode():
    """Stateful prefill + O(1) decode through SequenceModel (config C5 in miniature)."""
    torch.manual_seed(0)
    model = SequenceModel(ModelConfig(vocab_size=97, d_model=32, n_layers=2), KLAConfig(d_state=4)).eval()
    ids = torch.randint(0, 97, (2, 10))
    with torch.no_grad():
        logits_full = model(ids)
        logits_full = logits_full[0] if isinstance(logits_full, tuple) else logits_full
        assert logits_full.shape == (2, 10, 97)
        out = model.generate(ids[:, :6], max_new_tokens=4)
    assert out.shape[0] == 2 and out.shape[1] >= 6 + 4 - 1
