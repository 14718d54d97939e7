"""bench.py's host logic on the CPU: it refuses more than one GPU with a message
(this build runs the path on one GPU) and says so when no GPU is visible; the
synthetic inputs follow the draw recipes of the BASELINE configs."""

import pytest
import torch

import bench


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "--gpus 2 is not supported" in capsys.readouterr().err


@pytest.mark.skipif(torch.cuda.is_available(), reason="a GPU is visible")
def test_no_gpu_is_reported(capsys):
    assert bench.main([]) == 1
    assert "no GPU visible" in capsys.readouterr().err


def test_synthetic_inputs_follow_the_recipes():
    A, B, C, lam0, dlam = bench.mobius_inputs(2, 5, 7, seed=0)
    assert A.shape == B.shape == C.shape == dlam.shape == (2, 5, 7) and lam0.shape == (2, 7)
    # A = exp(-softplus(z)) in (0, 1); B, C, lam0 = softplus(z) > 0.
    assert bool(((A > 0) & (A < 1)).all()) and bool((B > 0).all() and (C > 0).all() and (lam0 > 0).all())
    g, u, dh = bench.affine_inputs(2, 5, 7, seed=1)
    assert bool(((g > 0) & (g < 1)).all()) and g.shape == u.shape == dh.shape == (2, 5, 7)
    # Seeded on the CPU: the same draw twice.
    assert torch.equal(bench.mobius_inputs(2, 5, 7, seed=0)[0], A)
