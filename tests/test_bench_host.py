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


def test_config_rooflines_price_the_documented_work():
    """The configs' roofline numerators: the projections' multiply-add flops per
    token (2 in out of every nn.Linear: C1's KLALayer(512) has in_proj 512 -> 2048,
    sensor_proj 1024 -> 2080, out_proj 1024 -> 512), and the bytes the fused scan
    kernels of C4 must move (514 MiB forward, 898 MiB backward with bf16 sensors)."""
    from kla import KLAConfig, KLALayer

    layer = KLALayer(512, KLAConfig(d_state=16))
    assert bench.linear_flops_per_token(layer) == 2 * (512 * 2048 + 1024 * 2080 + 1024 * 512)
    b = bench._fused_kernel_bytes(4, 4096, 2048, 16, sensor_bytes=2)
    assert b == {"fused_fwd": 514 * 2**20, "fused_bwd": 898 * 2**20}
    assert bench.VALU_ISSUE_PEAK_G == 614.4


def test_unknown_config_is_refused(capsys):
    with pytest.raises(SystemExit):
        bench.main(["--configs", "c9"])
    assert "unknown config" in capsys.readouterr().err
