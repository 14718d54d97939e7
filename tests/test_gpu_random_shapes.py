"""Randomly drawn problems through the public kla_scan on both hip paths (the
fused kernels, and the composed HIP scans with torch glue).

Each seed draws a shape (batch, a ragged sequence length, channels, and a state
width from 1 to past 256, where the state runs as consecutive groups), whether an
initial state is given, the prior read-out, whether the loss uses y_var (without
it the kernels skip the variance read-out and its adjoint), and a forced time
split of 1, 2 or 4 chunks (the fused path's chunk maps, their adjoints and both
walks; the composed path has no split). The outputs, the final state and the
gradients of every input and of the initial state are checked against float64
autograd of the reference's torch algorithm (oracle.torch_ref, reference
kla_ops.py:188-290) at the scan's bars.
"""

import random

import pytest
import torch

from kla.ops import KLAState, kla_scan
from oracle import torch_ref
from test_gpu_backend import check_scan, make_inputs, random_state

pytestmark = pytest.mark.gpu

STATE_WIDTHS = [1, 2, 3, 5, 8, 13, 16, 17, 31, 33, 64, 65, 100, 130, 256, 300]


def _draw(seed):
    r = random.Random(seed)
    S = r.choice(STATE_WIDTHS)
    B = r.randint(1, 3)
    split = r.choice([1, 1, 2, 4])
    L = r.randint(1, 160)
    if split > 1:   # chunks of whole 16-step checkpoint blocks
        L = max(16 * split, -(-L // (16 * split)) * 16 * split)
    M = r.randint(1, 24)
    while B * L * M * S > 400_000 and M > 1:
        M //= 2
    return dict(B=B, L=L, M=M, S=S, split=split, prior=r.random() < 0.4, with_var=r.random() < 0.5,
                with_state=r.random() < 0.6)


@pytest.mark.parametrize("backend", ["hip_fused", "hip_composed"])
@pytest.mark.parametrize("seed", range(24))
def test_random_problem_matches_float64_autograd(cuda, monkeypatch, seed, backend):
    from kla.ops.hip import fused

    d = _draw(seed)
    B, L, M, S = d["B"], d["L"], d["M"], d["S"]
    print(f"[random scan] {backend} seed={seed} {d}", flush=True)
    monkeypatch.setattr(fused, "train_chunks", lambda *a: d["split"])
    monkeypatch.setattr(fused, "time_chunks", lambda *a: d["split"])
    v, lv, k, q, a, p = make_inputs(B, L, M, S, seed=1000 + seed)
    st = random_state(B, M, S, seed=2000 + seed) if d["with_state"] else None
    g = torch.Generator().manual_seed(3000 + seed)
    w = [torch.randn(B, L, M, generator=g), torch.randn(B, L, M, generator=g),
         torch.randn(B, M, S, generator=g), torch.randn(B, M, S, generator=g)]

    def loss(y, y_var, lam, eta):
        ww = [t.to(device=y.device, dtype=y.dtype) for t in w]
        total = (ww[0] * y).sum() + (ww[2] * lam).sum() + (ww[3] * eta).sum()
        return total + (ww[1] * y_var).sum() if d["with_var"] else total

    leaves = [v, lv, k, q, a, p] + ([st.lam, st.eta] if st is not None else [])
    xs = [t.double().requires_grad_(True) for t in leaves]
    ref = torch_ref.kla_scan_torch(*xs[:6], *xs[6:], decode_from_prior=d["prior"])
    loss(*ref).backward()

    gs = [t.to(cuda).requires_grad_(True) for t in leaves]
    init = KLAState(lam=gs[6], eta=gs[7]) if st is not None else None
    y, y_var, state = kla_scan(*gs[:6], initial_state=init, backend=backend, decode_from_prior=d["prior"])
    out = (y, y_var, state.lam, state.eta)
    for name, got, want in zip(("y", "y_var", "lam", "eta"), out, ref):
        check_scan(name, got, want.detach().numpy())
    loss(*out).backward()
    names = ["v", "lambda_v", "k", "q", "a", "p", "lam0", "eta0"]
    for name, got, want in zip(names, gs, xs):
        check_scan("d" + name, got.grad, want.grad.numpy())
