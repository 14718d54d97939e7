"""GPU parity of the standalone Moebius and affine scans against the CPU oracle.

Every case draws its inputs on the CPU (torch.Generator), runs the HIP kernels
through the public ops (:func:`kla.ops.hip.mobius_scan`, :func:`affine_scan`)
and compares with oracle.scans in float64 at the path's tolerance:
rtol 1e-5, atol 1e-6 for fp32 (outputs, final states and every gradient), and
rtol 2e-2 (atol 1e-5) for bf16 I/O. Shapes cover a single step, ragged lane tiles (lanes not
a multiple of 64), ragged chunks (steps not a multiple of the 64-step chunk),
long sequences (many look-back hops) and the full headline shape (every element).
"""

import sys

import numpy as np
import pytest
import torch

from bench import affine_inputs, mobius_inputs
from oracle import scans as ref

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-6
SHAPES = [
    (1, 1, 1),
    (2, 7, 3),
    (1, 64, 64),
    (2, 65, 63),
    (3, 130, 65),
    (2, 257, 130),
    (1, 1000, 64),
    (2, 4096, 96),
    (1, 3001, 1),
]


def _close(name, got, want, rtol=RTOL, atol=ATOL):
    got = got.detach().double().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    want = np.asarray(want, dtype=np.float64).reshape(got.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    ratio = np.abs(got - want) / (atol + rtol * np.abs(want))
    worst = float(ratio.max()) if ratio.size else 0.0
    print(f"  {name:8s} worst |d|/(atol+rtol|ref|) = {worst:.3f}", flush=True)
    assert worst <= 1.0, f"{name}: outside rtol={rtol} atol={atol} (worst ratio {worst:.3f})"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("with_lam0", [True, False])
def test_mobius_fwd_bwd_matches_oracle(cuda, shape, with_lam0):
    from kla.ops.hip import mobius_scan

    B, T, N = shape
    _log(f"[mobius] shape={shape} lam0={with_lam0}")
    A, Bm, C, lam0, dlam = mobius_inputs(B, T, N, seed=3)
    if not with_lam0:
        lam0 = None
    leaves = [t.to(cuda).requires_grad_(True) for t in (A, Bm, C)]
    l0 = lam0.to(cuda).requires_grad_(True) if lam0 is not None else None
    lam = mobius_scan(*leaves, None, l0)
    torch.autograd.backward(lam, dlam.to(cuda))

    want = ref.mobius_scan_fwd(A, Bm, C, None, lam0)
    _close("lam", lam, want)
    dA, dB, dC, _, dl0 = ref.mobius_scan_bwd(dlam, A, Bm, C, None, lam0, want)
    _close("dA", leaves[0].grad, dA)
    _close("dB", leaves[1].grad, dB)
    _close("dC", leaves[2].grad, dC)
    if l0 is not None:
        _close("dlam0", l0.grad, dl0)


@pytest.mark.parametrize("seed", range(16))
def test_random_shapes_match_oracle(cuda, seed):
    """Randomly drawn (B, T, lanes) -- T up to 5000, so several chunks of every
    kernel's tile, lanes from 1 to 300, ragged against the 64-lane tiles -- with or
    without the initial states and an explicit D: the Moebius and affine scans,
    forward and backward, against the float64 oracle at rtol 1e-5 / atol 1e-6."""
    import random

    from kla.ops.hip import affine_scan, mobius_scan

    r = random.Random(seed)
    B, T, N = r.randint(1, 3), r.randint(1, 5000), r.randint(1, 300)
    with_init, with_D = r.random() < 0.6, r.random() < 0.3
    _log(f"[random scans] seed={seed} shape={(B, T, N)} init={with_init} D={with_D}")
    A, Bm, C, lam0, dlam = mobius_inputs(B, T, N, seed=100 + seed)
    D = (torch.rand(B, T, N, generator=torch.Generator().manual_seed(200 + seed)) + 0.5) if with_D else None
    lam0 = lam0 if with_init else None
    leaves = [t.to(cuda).requires_grad_(True) for t in (A, Bm, C) + ((D,) if with_D else ())]
    l0 = lam0.to(cuda).requires_grad_(True) if lam0 is not None else None
    lam = mobius_scan(*leaves[:3], leaves[3] if with_D else None, l0)
    torch.autograd.backward(lam, dlam.to(cuda))
    want = ref.mobius_scan_fwd(A, Bm, C, D, lam0)
    _close("lam", lam, want)
    grads = ref.mobius_scan_bwd(dlam, A, Bm, C, D, lam0, want)
    for name, got, w in zip(("dA", "dB", "dC"), leaves, grads[:3]):
        _close(name, got.grad, w)
    if with_D:
        _close("dD", leaves[3].grad, grads[3])
    if l0 is not None:
        _close("dlam0", l0.grad, grads[4])

    g, u, dh = affine_inputs(B, T, N, seed=300 + seed)
    h0 = torch.randn(B, N, generator=torch.Generator().manual_seed(400 + seed)) if with_init else None
    gg, uu = g.to(cuda).requires_grad_(True), u.to(cuda).requires_grad_(True)
    hh0 = h0.to(cuda).requires_grad_(True) if h0 is not None else None
    h = affine_scan(gg, uu, hh0)
    torch.autograd.backward(h, dh.to(cuda))
    want = ref.affine_scan_fwd(g, u, h0)
    _close("h", h, want)
    dg, du, dh0 = ref.affine_scan_bwd(dh, g, want, h0)
    _close("dg", gg.grad, dg)
    _close("du", uu.grad, du)
    if hh0 is not None:
        _close("dh0", hh0.grad, dh0)


@pytest.mark.parametrize("shape", [(2, 130, 65), (1, 300, 128)])
def test_mobius_explicit_D(cuda, shape):
    """A general D tensor (the reference passes ones_like(phi)) and its gradient dD."""
    from kla.ops.hip import mobius_scan

    B, T, N = shape
    A, Bm, C, lam0, dlam = mobius_inputs(B, T, N, seed=4)
    D = torch.rand(B, T, N, generator=torch.Generator().manual_seed(9)) + 0.5
    xs = [t.to(cuda).requires_grad_(True) for t in (A, Bm, C, D, lam0)]
    lam = mobius_scan(*xs)
    torch.autograd.backward(lam, dlam.to(cuda))
    want = ref.mobius_scan_fwd(A, Bm, C, D, lam0)
    _close("lam", lam, want)
    grads = ref.mobius_scan_bwd(dlam, A, Bm, C, D, lam0, want)
    for name, got, w in zip(("dA", "dB", "dC", "dD", "dlam0"), xs, grads):
        _close(name, got.grad, w)


@pytest.mark.parametrize("shape", [(2, 1000, 130), (1, 4096, 64), (1, 17, 3)])
@pytest.mark.parametrize("with_D", [False, True])
def test_mobius_bwd_recomputes_lam_bitwise(cuda, shape, with_D):
    """The backward reads the saved lam only where a thread's steps begin and
    recomputes the rest with the forward's own step, so the recomputed values
    are the stored ones bit for bit: poisoning every other row of lam (with NaN)
    leaves every gradient bitwise unchanged. Threads hold MOBIUS_BWD_STEPS (24)
    consecutive steps in reverse time, so the rows read are t = T-1-24m, m >= 1."""
    from bench import MOBIUS_BWD_STEPS
    from kla.ops.hip import scans as hs

    B, T, N = shape
    A, Bm, C, lam0, dlam = (t.to(cuda) for t in mobius_inputs(B, T, N, seed=21))
    D = (torch.rand(B, T, N, generator=torch.Generator().manual_seed(22)) + 0.5).to(cuda) if with_D else None
    lam = hs._mobius_scan_op(A, Bm, C, D, lam0)
    ref_grads = hs._mobius_scan_bwd_op(dlam, A, Bm, C, D, lam0, lam)
    t = torch.arange(T, device=cuda)
    keep = ((T - 1 - t) % MOBIUS_BWD_STEPS == 0) & (t != T - 1)
    poisoned = torch.where(keep[None, :, None], lam, torch.full_like(lam, float("nan")))
    got = hs._mobius_scan_bwd_op(dlam, A, Bm, C, D, lam0, poisoned)
    names = ("dA", "dB", "dC", "dD", "dlam0")
    for name, a, b in zip(names, ref_grads, got):  # dD is empty without D
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), f"{name}: the backward read a poisoned row of lam"


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("with_h0", [True, False])
def test_affine_fwd_bwd_matches_oracle(cuda, shape, with_h0):
    from kla.ops.hip import affine_scan

    B, T, N = shape
    _log(f"[affine] shape={shape} h0={with_h0}")
    g, u, dh = affine_inputs(B, T, N, seed=5)
    h0 = torch.randn(B, N, generator=torch.Generator().manual_seed(6)) if with_h0 else None
    gg, uu = g.to(cuda).requires_grad_(True), u.to(cuda).requires_grad_(True)
    hh0 = h0.to(cuda).requires_grad_(True) if h0 is not None else None
    h = affine_scan(gg, uu, hh0)
    torch.autograd.backward(h, dh.to(cuda))
    want = ref.affine_scan_fwd(g, u, h0)
    _close("h", h, want)
    dg, du, dh0 = ref.affine_scan_bwd(dh, g, want, h0)
    _close("dg", gg.grad, dg)
    _close("du", uu.grad, du)
    if hh0 is not None:
        _close("dh0", hh0.grad, dh0)


@pytest.mark.parametrize("with_h0", [False, True])
@pytest.mark.parametrize("shape", [(2, 65, 63), (2, 1000, 130), (1, 4096, 64), (2, 1000, 128), (1, 4096, 256),
                                   (3, 300, 2048)])
def test_affine_bf16_io(cuda, shape, with_h0):
    """bf16 sequence I/O, fp32 accumulation: within rtol 2e-2 of the fp64 oracle run
    on the same (bf16-exact) inputs (atol 1e-5 for values that cancel to near
    zero); outputs come back in bf16. With an fp32 initial state h0 the backward's
    step at time 0 takes h_{-1} = h0 unrounded (dg_0 = mu_0 h0) and dh0 comes back
    fp32. Lanes that are a multiple of 4 run the 4-lanes-per-thread tile (time 0 in
    a partial chunk at T = 300 and 1000, in a whole one at T = 4096), the others
    the 1-lane tile."""
    from kla.ops.hip import affine_scan

    B, T, N = shape
    _log(f"[affine bf16] shape={shape} h0={with_h0}")
    g, u, dh = affine_inputs(B, T, N, seed=7, dtype=torch.bfloat16)
    h0 = torch.randn(B, N, generator=torch.Generator().manual_seed(8)) if with_h0 else None
    gg, uu = g.to(cuda).requires_grad_(True), u.to(cuda).requires_grad_(True)
    hh0 = h0.to(cuda).requires_grad_(True) if with_h0 else None
    h = affine_scan(gg, uu, hh0)
    assert h.dtype == torch.bfloat16
    torch.autograd.backward(h, dh.to(cuda))
    assert gg.grad.dtype == torch.bfloat16 and uu.grad.dtype == torch.bfloat16
    want = ref.affine_scan_fwd(g.float(), u.float(), h0)
    _close("h", h, want, rtol=2e-2, atol=1e-5)
    dg, du, dh0 = ref.affine_scan_bwd(dh.float(), g.float(), want, h0)
    _close("dg", gg.grad, dg, rtol=2e-2, atol=1e-5)
    _close("du", uu.grad, du, rtol=2e-2, atol=1e-5)
    if with_h0:
        assert hh0.grad.dtype == torch.float32
        _close("dh0", hh0.grad, dh0, rtol=2e-2, atol=1e-5)
        # The step at time 0 multiplies by h0 itself: dg_0 / mu_0 = h0 to bf16 rounding.
        _close("dg_0", gg.grad[:, 0], (uu.grad[:, 0].double().cpu() * h0.double()).numpy(), rtol=1e-2, atol=1e-5)


def test_affine_bf16_streaming_forward_equals_cached(cuda):
    """The affine forward stores a bf16 output of up to 256 MiB with cache-allocating
    stores (the backward reads it next) and a larger one nontemporally; the
    arithmetic is the same. At (9, 8192, 2048) bf16 (288 MiB) the streaming run's
    first four batch rows equal the cached run of those rows alone bit for bit,
    and sampled lanes of the first and last rows match the float64 oracle."""
    from kla.ops.hip import affine_scan

    B, T, N = 9, 8192, 2048
    gen = torch.Generator(device=cuda).manual_seed(31)
    g = torch.sigmoid(torch.randn(B, T, N, device=cuda, generator=gen) + 2.0).to(torch.bfloat16)
    u = torch.randn(B, T, N, device=cuda, generator=gen).to(torch.bfloat16)
    with torch.no_grad():
        h = affine_scan(g, u)
        h4 = affine_scan(g[:4].contiguous(), u[:4].contiguous())
    assert torch.equal(h[:4], h4)
    lanes = torch.cat([torch.arange(0, 128), torch.arange(1000, 1128), torch.arange(N - 128, N)])
    for b in (0, B - 1):
        gs, us = g[b:b + 1, :, lanes].float().cpu(), u[b:b + 1, :, lanes].float().cpu()
        _close(f"h[{b}]", h[b:b + 1, :, lanes], ref.affine_scan_fwd(gs, us), rtol=2e-2, atol=1e-5)


@pytest.mark.parametrize("lanes", [64, 130, 2048])
def test_affine_bf16_outputs_round_to_nearest_even(cuda, lanes):
    """The kernels' fp32 -> bf16 stores round exactly as torch does (to nearest, ties
    to even), bit for bit. One step with g = 1, u = -0 stores h = round(h0) of an fp32
    h0 (1 * h0 + (-0) = h0 exactly); h0 holds random values over all binades, exact
    ties on even and odd bf16 mantissas, values one fp32 ulp either side of a tie,
    signed zeros, fp32 subnormals and the largest finite value."""
    from kla.ops.hip import affine_scan

    gen = torch.Generator().manual_seed(11)
    B = 4
    n = B * lanes
    mant = torch.randint(0, 1 << 23, (n,), generator=gen, dtype=torch.int64)
    expo = torch.randint(1, 255, (n,), generator=gen, dtype=torch.int64)
    sign = torch.randint(0, 2, (n,), generator=gen, dtype=torch.int64)
    bits = (sign << 31) | (expo << 23) | mant
    # Every 4th value an exact tie (low 16 bits 0x8000), every 4th + 1 one ulp
    # either side of it, the first few special.
    bits[0::4] = (bits[0::4] & ~0xFFFF) | 0x8000
    bits[1::4] = (bits[1::4] & ~0xFFFF) | 0x7FFF
    bits[2::4] = (bits[2::4] & ~0xFFFF) | 0x8001
    special = torch.tensor([0x00000000, 0x80000000, 0x00000001, 0x007FFFFF, 0x00408000, 0x80018000,
                            0x7F7FFFFF, 0x3F808000, 0x3F818000], dtype=torch.int64)
    bits[:len(special)] = special
    h0 = bits.to(torch.int32).view(torch.float32).reshape(B, lanes)
    g = torch.ones(B, 1, lanes, dtype=torch.bfloat16)
    u = torch.full((B, 1, lanes), -0.0, dtype=torch.bfloat16)   # x + (-0) = x, signed zeros included
    h = affine_scan(g.to(cuda), u.to(cuda), h0.to(cuda))
    want = h0.to(torch.bfloat16).reshape(B, 1, lanes)
    got = h.cpu()
    mismatch = (got.view(torch.int16) != want.view(torch.int16)).nonzero()
    assert mismatch.numel() == 0, (
        f"{mismatch.shape[0]} values rounded differently, e.g. h0 bits "
        f"{int(bits.reshape(B, 1, lanes)[tuple(mismatch[0])]) & 0xFFFFFFFF:#010x}")


def test_empty_and_zero_length(cuda):
    from kla.ops.hip import affine_scan, mobius_scan

    for shape in [(0, 5, 4), (2, 0, 4), (2, 5, 0)]:
        A = torch.rand(*shape, device=cuda) + 0.1
        lam = mobius_scan(A, A, A)
        assert lam.shape == shape
        h = affine_scan(A, A)
        assert h.shape == shape
    # Zero steps with a state: the state gradient is exactly zero.
    A = (torch.rand(2, 0, 4, device=cuda) + 0.1).requires_grad_(True)
    l0 = torch.rand(2, 4, device=cuda).requires_grad_(True)
    lam = mobius_scan(A, A, A, None, l0)
    lam.sum().backward()
    assert torch.equal(l0.grad, torch.zeros_like(l0))


def test_deterministic_bitwise(cuda):
    """The look-back composes carries in a fixed order, so repeated runs agree bit for bit."""
    from kla.ops.hip import affine_scan, mobius_scan

    A, Bm, C, lam0, dlam = (t.to(cuda) for t in mobius_inputs(4, 2048, 512, seed=11))
    runs = []
    for _ in range(3):
        xs = [t.clone().requires_grad_(True) for t in (A, Bm, C, lam0)]
        lam = mobius_scan(xs[0], xs[1], xs[2], None, xs[3])
        lam.backward(dlam)
        runs.append([lam.detach()] + [x.grad for x in xs])
    for other in runs[1:]:
        for a, b in zip(runs[0], other):
            assert torch.equal(a, b)
    g, u, dh = (t.to(cuda) for t in affine_inputs(4, 2048, 512, seed=12))
    hs = [affine_scan(g, u) for _ in range(3)]
    assert torch.equal(hs[0], hs[1]) and torch.equal(hs[0], hs[2])
    # A fresh (zero-filled) workspace after reset_workspaces gives the same bits.
    from kla.ops.hip import _lib

    _lib.reset_workspaces()
    assert torch.equal(affine_scan(g, u), hs[0])
    assert torch.equal(mobius_scan(A, Bm, C, None, lam0), runs[0][0])


def test_headline_shape_whole_tensors(cuda):
    """Full (8, 4096, 2048) Moebius and affine fwd + bwd: every element of every
    output and gradient against the float64 oracle at rtol 1e-5 / atol 1e-6 (as the
    reference's tests/test_backends.py:220-249 compares whole tensors), one batch
    row at a time to bound host memory; no look-back wait gave up."""
    from kla.ops.hip import _lib, affine_scan, mobius_scan

    B, T, N = 8, 4096, 2048
    _log("[headline] generating inputs")
    A, Bm, C, lam0, dlam = mobius_inputs(B, T, N, seed=0)
    xs = [t.to(cuda).requires_grad_(True) for t in (A, Bm, C, lam0)]
    lam = mobius_scan(xs[0], xs[1], xs[2], None, xs[3])
    lam.backward(dlam.to(cuda))
    g, u, dh = affine_inputs(B, T, N, seed=1)
    gg, uu = g.to(cuda).requires_grad_(True), u.to(cuda).requires_grad_(True)
    h = affine_scan(gg, uu)
    h.backward(dh.to(cuda))
    torch.cuda.synchronize()
    assert _lib.workspace_failures(cuda) == 0
    got = {name: t.detach().cpu() for name, t in (("lam", lam), ("dA", xs[0].grad), ("dB", xs[1].grad),
                                                  ("dC", xs[2].grad), ("dlam0", xs[3].grad), ("h", h),
                                                  ("dg", gg.grad), ("du", uu.grad))}
    del xs, lam, gg, uu, h
    worst = {}

    def close(name, got_, want):
        ratio = np.abs(got_.double().numpy() - want) / (ATOL + RTOL * np.abs(want))
        assert np.isfinite(got_.numpy()).all(), name
        worst[name] = max(worst.get(name, 0.0), float(ratio.max()))

    for b in range(B):
        _log(f"[headline] oracle, batch row {b}")
        r = slice(b, b + 1)
        want = ref.mobius_scan_fwd(A[r], Bm[r], C[r], None, lam0[r])
        close("lam", got["lam"][r], want)
        dA, dBm, dC, _, dl0 = ref.mobius_scan_bwd(dlam[r], A[r], Bm[r], C[r], None, lam0[r], want)
        close("dA", got["dA"][r], dA)
        close("dB", got["dB"][r], dBm)
        close("dC", got["dC"][r], dC)
        close("dlam0", got["dlam0"][r], dl0)
        del want, dA, dBm, dC
        hw = ref.affine_scan_fwd(g[r], u[r])
        close("h", got["h"][r], hw)
        dgw, duw, _ = ref.affine_scan_bwd(dh[r], g[r], hw)
        close("dg", got["dg"][r], dgw)
        close("du", got["du"][r], duw)
    for name, w in worst.items():
        print(f"  {name:8s} worst |d|/(atol+rtol|ref|) = {w:.3f}", flush=True)
    assert all(w <= 1.0 for w in worst.values()), worst


def test_carry_only_launches_match_aggregate_launches_bitwise(cuda):
    """At (8, 4096, 2048) every look-back scan publishes carries only (one chunk
    of all tiles moves >= 8 MiB); one batch row's first 1024 lanes alone (16x
    fewer tiles) publish chunk aggregates too. The carry chain is the same float32
    computation either way, so every output and gradient of the whole launch
    equals those launches bit for bit: fp32 Moebius and affine, and bf16 affine
    I/O."""
    from kla.ops.hip import _lib
    from kla.ops.hip import scans as hs

    B, T, N = 8, 4096, 2048
    _log("[carry-only] Moebius")
    A, Bm, C, lam0, dlam = (t.to(cuda) for t in mobius_inputs(B, T, N, seed=3))
    whole = [hs._mobius_scan_op(A, Bm, C, None, lam0)]
    whole += [t for t in hs._mobius_scan_bwd_op(dlam, A, Bm, C, None, lam0, whole[0]) if t is not None]
    half = N // 2

    def part(t, b):  # batch row b, lanes [0, half), contiguous
        return t[b:b + 1, ..., :half].contiguous()

    def whole_part(t, b):  # unrequested gradients come back as empty tensors
        return t[b:b + 1, ..., :half] if t.numel() else t

    for b in range(B):
        lam = hs._mobius_scan_op(part(A, b), part(Bm, b), part(C, b), None, part(lam0, b))
        rows = [lam] + [t for t in hs._mobius_scan_bwd_op(part(dlam, b), part(A, b), part(Bm, b), part(C, b), None,
                                                          part(lam0, b), lam) if t is not None]
        for i, (w, g_) in enumerate(zip(whole, rows)):
            assert torch.equal(whole_part(w, b), g_), f"Moebius output {i}, batch row {b}"
    del A, Bm, C, lam0, dlam, whole
    for dtype in (torch.float32, torch.bfloat16):
        _log(f"[carry-only] affine {dtype}")
        g, u, dh = (t.to(cuda, dtype) for t in affine_inputs(B, T, N, seed=4))
        h = hs._affine_scan_op(g, u, None)
        whole = [h] + [t for t in hs._affine_scan_bwd_op(dh, g, h, None) if t is not None]
        for b in range(B):
            hr = hs._affine_scan_op(part(g, b), part(u, b), None)
            rows = [hr] + [t for t in hs._affine_scan_bwd_op(part(dh, b), part(g, b), hr, None) if t is not None]
            for i, (w, g_) in enumerate(zip(whole, rows)):
                assert torch.equal(whole_part(w, b), g_), f"affine {dtype} output {i}, batch row {b}"
        del g, u, dh, h, whole
    torch.cuda.synchronize()
    assert _lib.workspace_failures(cuda) == 0


def test_scans_past_2_31_elements(cuda):
    """Element indices past 2^31 need 64-bit offsets: (4, 65536, 8193) is 2^31 +
    262144 elements (8.6 GB per fp32 tensor; MI355X holds the whole Moebius fwd +
    bwd and a bf16 affine fwd + bwd). Inputs are drawn on the GPU from the bench's
    families; five lanes of every batch -- tile edges and the ragged last lane,
    whose elements in the last batch lie past 2^31 -- are checked against the
    float64 oracle, and no look-back wait gave up."""
    import torch.nn.functional as F

    from kla.ops.hip import _lib
    from kla.ops.hip import scans as hs

    B, T, N = 4, 65536, 8193
    assert B * T * N > 2 ** 31 and (B - 1) * T * N + (T - 1) * N + (N - 1) >= 2 ** 31
    lanes = torch.tensor([0, 63, 64, 8191, 8192])
    gen = torch.Generator(device=cuda).manual_seed(5)

    def draw(fn):
        return fn(torch.randn(B, T, N, device=cuda, generator=gen))

    sub = lambda t: t[..., lanes.to(cuda)].float().cpu()  # noqa: E731
    _log("[2^31] Moebius inputs")
    A = draw(lambda z: torch.exp(-F.softplus(z)))
    Bm = draw(F.softplus)
    C = draw(F.softplus)
    lam0 = F.softplus(torch.randn(B, N, device=cuda, generator=gen))
    lam = hs._mobius_scan_op(A, Bm, C, None, lam0)
    dlam = draw(lambda z: z)
    dA, dB, dC, _, dl0 = hs._mobius_scan_bwd_op(dlam, A, Bm, C, None, lam0, lam)
    torch.cuda.synchronize()
    assert _lib.workspace_failures(cuda) == 0
    for t in (lam, dA, dB, dC, dl0):
        assert torch.isfinite(t).all()
    sA, sB, sC, sl0, sdl = sub(A), sub(Bm), sub(C), lam0[:, lanes.to(cuda)].cpu(), sub(dlam)
    got = [sub(t) for t in (lam, dA, dB, dC)] + [dl0[:, lanes.to(cuda)].cpu()]
    del A, Bm, C, lam, dlam, dA, dB, dC
    torch.cuda.empty_cache()
    _log("[2^31] Moebius oracle")
    want = ref.mobius_scan_fwd(sA, sB, sC, None, sl0)
    _close("lam", got[0], want)
    wA, wB, wC, _, wl0 = ref.mobius_scan_bwd(sdl, sA, sB, sC, None, sl0, want)
    for name, g_, w in (("dA", got[1], wA), ("dB", got[2], wB), ("dC", got[3], wC), ("dlam0", got[4], wl0)):
        _close(name, g_, w)

    _log("[2^31] affine bf16 inputs")
    g = draw(torch.sigmoid).to(torch.bfloat16)
    u = draw(lambda z: z).to(torch.bfloat16)
    h = hs._affine_scan_op(g, u, None)
    dh = draw(lambda z: z).to(torch.bfloat16)
    dg, du, _ = hs._affine_scan_bwd_op(dh, g, h, None)
    torch.cuda.synchronize()
    assert _lib.workspace_failures(cuda) == 0
    sg, su, sdh = sub(g), sub(u), sub(dh)
    got = [sub(t) for t in (h, dg, du)]
    del g, u, h, dh, dg, du
    torch.cuda.empty_cache()
    _log("[2^31] affine oracle")
    hw = ref.affine_scan_fwd(sg, su)
    _close("h", got[0], hw, rtol=2e-2, atol=1e-5)
    dgw, duw, _ = ref.affine_scan_bwd(sdh, sg, hw)
    _close("dg", got[1], dgw, rtol=2e-2, atol=1e-5)
    _close("du", got[2], duw, rtol=2e-2, atol=1e-5)
