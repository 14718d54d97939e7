"""kla_mobius_scan_fwd_noalloc (the allocation-free entry point) against
kla_mobius_scan_fwd on the GPU, both called through the C ABI.

The no-alloc variant keeps its look-back records in the library's static
per-GPU scratch array; its results must be bit-identical to the workspace
variant's (the same kernel, the same deterministic look-back), on two calls in
a row where the second is smaller (the scratch keeps the first call's records,
which the epoch tags must invalidate), with and without D and lam0, and up to
the headline shape (8, 4096, 2048), the largest the scratch holds; the static
scratch's look-back failure count (kla_workspace_failures with a NULL
workspace) stays 0. A shape beyond the scratch is refused before any launch
(tests/test_abi.py::test_mobius_fwd_noalloc_validation, on the CPU).
"""

import pytest
import torch

from bench import mobius_inputs
from kla.ops.hip import _lib

pytestmark = pytest.mark.gpu


def _workspace_fwd(A, B, C, D, lam0, cuda):
    lib = _lib.lib()
    Bn, T, N = A.shape
    nbytes = int(lib.kla_scan_workspace_bytes(_lib.KLA_SCAN_MOBIUS_FWD, Bn, T, N))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=cuda)
    lam = torch.empty_like(A)
    pt = _lib.ptr
    _lib.check("kla_mobius_scan_fwd", lib.kla_mobius_scan_fwd(
        pt(A), pt(B), pt(C), pt(D), pt(lam0), pt(lam), Bn, T, N, pt(ws), nbytes,
        torch.cuda.current_stream(cuda).cuda_stream))
    return lam


def _noalloc_fwd(A, B, C, D, lam0, cuda):
    lib = _lib.lib()
    Bn, T, N = A.shape
    lam = torch.full_like(A, float("nan"))
    pt = _lib.ptr
    _lib.check("kla_mobius_scan_fwd_noalloc", lib.kla_mobius_scan_fwd_noalloc(
        pt(A), pt(B), pt(C), pt(D), pt(lam0), pt(lam), Bn, T, N, torch.cuda.current_stream(cuda).cuda_stream))
    return lam


@pytest.mark.parametrize("with_d", [False, True])
def test_noalloc_equals_workspace_variant(cuda, with_d):
    for shape, seed in (((8, 4096, 2048), 0), ((2, 1000, 130), 1), ((3, 7, 5), 2)):
        print(f"[noalloc] shape={shape} D={with_d}", flush=True)
        A, B, C, lam0, _ = (t.to(cuda) for t in mobius_inputs(*shape, seed=seed))
        D = (torch.rand(shape, generator=torch.Generator().manual_seed(seed)) + 0.5).to(cuda) if with_d else None
        l0 = lam0 if seed != 1 else None
        want = _workspace_fwd(A, B, C, D, l0, cuda)
        got = _noalloc_fwd(A, B, C, D, l0, cuda)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), shape
        assert _lib.noalloc_failures(cuda) == 0
        del A, B, C, D, lam0, want, got
