"""The C ABI of libkla_hip.so, exercised on the CPU (no GPU needed).

* the library loads, reports the ABI version the Python binding expects, and
  exports every function include/kla_hip.h declares (and the binding binds);
* every argument check returns its documented status and message before any
  HIP call: NULL operands, negative or oversized shapes, unknown dtype or scan
  kind, operands not aligned to their element, a missing / misaligned / short
  workspace. Calls here use fake device addresses that the library rejects
  before dereferencing or launching anything;
* empty problems succeed without launching;
* the last-error message is per thread.

Mirrors the reference binding's TORCH_CHECK validation
(src/kla/ops/kernels/cuda/v2_2/kla_matmul_scan.cu:35-59).
"""

import ctypes
import os
import re
import threading

import pytest
import torch

from kla.ops.hip import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "kla_hip.h")

# Fake, never-dereferenced device addresses: aligned (ALIGNED) and not (ODD).
ALIGNED = 0x7F0000000000
ODD = ALIGNED + 2
WS = 0x7F0000100000  # 256-byte aligned


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kla_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


def err(lib):
    return lib.kla_hip_last_error().decode()


def test_library_loads_and_reports_abi(lib):
    assert lib.kla_hip_abi_version() == _lib.ABI_VERSION


def test_every_declared_function_is_exported_and_bound(lib):
    declared = header_functions()
    assert len(declared) >= 8
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in kla_hip.h but not exported"
    assert sorted(_lib._SIGNATURES) == declared, "ctypes binding and header disagree"


GUIDE = os.path.join(REPO, "INTEGRATION.md")   # the maintainers' integration guide


def test_every_declared_function_has_a_row_in_integration():
    """The integration guide's ABI table names every entry point of kla_hip.h,
    with the reference code it replaces (or why it has none)."""
    text = open(GUIDE).read()
    missing = [name for name in header_functions() if f"`{name}`" not in text]
    assert not missing, f"entry points without a row in the integration guide: {missing}"


def test_workspace_bytes(lib):
    for kind in range(4):
        n = lib.kla_scan_workspace_bytes(kind, 8, 4096, 2048)
        assert n > 256 and n % 8 == 0
        # Grows with the problem, never shrinks.
        assert lib.kla_scan_workspace_bytes(kind, 8, 8192, 2048) >= n
        assert lib.kla_scan_workspace_bytes(kind, 1, 1, 1) > 0
    assert lib.kla_scan_workspace_bytes(9, 8, 4096, 2048) == 0
    assert "unknown scan kind 9" in err(lib)
    assert lib.kla_scan_workspace_bytes(0, -1, 4, 4) == 0
    assert "negative size" in err(lib)


def _mobius_fwd(lib, A=ALIGNED, B=ALIGNED, C=ALIGNED, D=None, lam0=None, lam=ALIGNED, shape=(2, 3, 4),
                ws=WS, ws_bytes=1 << 40):
    return lib.kla_mobius_scan_fwd(A, B, C, D, lam0, lam, *shape, ws, ws_bytes, None)


def test_mobius_fwd_validation(lib):
    assert _mobius_fwd(lib, A=None) == _lib.KLA_ERR_INVALID_ARG
    assert "must not be NULL" in err(lib)
    assert _mobius_fwd(lib, shape=(2, -3, 4)) == _lib.KLA_ERR_INVALID_ARG
    assert "negative size" in err(lib)
    assert _mobius_fwd(lib, shape=(2, 3, (1 << 31) + 1)) == _lib.KLA_ERR_INVALID_ARG
    assert "above 2^31" in err(lib)
    assert _mobius_fwd(lib, C=ODD) == _lib.KLA_ERR_ALIGN
    assert _mobius_fwd(lib, D=ODD) == _lib.KLA_ERR_ALIGN
    assert _mobius_fwd(lib, lam0=ODD) == _lib.KLA_ERR_ALIGN
    assert _mobius_fwd(lib, ws=None) == _lib.KLA_ERR_WORKSPACE
    assert "workspace is NULL" in err(lib)
    assert _mobius_fwd(lib, ws=WS + 8) == _lib.KLA_ERR_WORKSPACE
    assert "256-byte aligned" in err(lib)
    assert _mobius_fwd(lib, ws_bytes=64) == _lib.KLA_ERR_WORKSPACE
    assert "needed" in err(lib)
    # Empty problems succeed without touching any operand.
    for shape in [(0, 3, 4), (2, 0, 4), (2, 3, 0)]:
        assert _mobius_fwd(lib, A=None, B=None, C=None, lam=None, ws=None, shape=shape) == _lib.KLA_OK


def test_mobius_bwd_validation(lib):
    def call(**kw):
        a = dict(dlam=ALIGNED, A=ALIGNED, B=ALIGNED, C=ALIGNED, D=None, lam0=None, lam=ALIGNED, dA=ALIGNED,
                 dB=ALIGNED, dC=ALIGNED, dD=None, dlam0=None, shape=(2, 3, 4), ws=WS, ws_bytes=1 << 40)
        a.update(kw)
        return lib.kla_mobius_scan_bwd(a["dlam"], a["A"], a["B"], a["C"], a["D"], a["lam0"], a["lam"], a["dA"],
                                       a["dB"], a["dC"], a["dD"], a["dlam0"], *a["shape"], a["ws"], a["ws_bytes"],
                                       None)

    assert call(lam=None) == _lib.KLA_ERR_INVALID_ARG
    assert call(dlam=None) == _lib.KLA_ERR_INVALID_ARG
    assert call(dB=ODD) == _lib.KLA_ERR_ALIGN
    assert call(dlam0=ODD) == _lib.KLA_ERR_ALIGN
    assert call(ws=None) == _lib.KLA_ERR_WORKSPACE
    assert call(ws_bytes=8) == _lib.KLA_ERR_WORKSPACE
    # Zero steps and no state gradient asked for: nothing to do.
    assert call(shape=(2, 0, 4), dlam=None, A=None, B=None, C=None, lam=None) == _lib.KLA_OK
    assert call(shape=(0, 5, 4)) == _lib.KLA_OK


def test_affine_validation(lib):
    def fwd(dtype=_lib.KLA_DTYPE_F32, g=ALIGNED, u=ALIGNED, h0=None, h=ALIGNED, shape=(2, 3, 4), ws=WS,
            ws_bytes=1 << 40):
        return lib.kla_affine_scan_fwd(dtype, g, u, h0, h, *shape, ws, ws_bytes, None)

    assert fwd(dtype=7) == _lib.KLA_ERR_DTYPE
    assert "unsupported dtype code 7" in err(lib)
    assert fwd(u=None) == _lib.KLA_ERR_INVALID_ARG
    assert fwd(g=ODD) == _lib.KLA_ERR_ALIGN
    # bf16 operands need 2-byte alignment only.
    assert fwd(dtype=_lib.KLA_DTYPE_BF16, g=ALIGNED + 1) == _lib.KLA_ERR_ALIGN
    assert fwd(dtype=_lib.KLA_DTYPE_BF16, g=ODD, ws=None) == _lib.KLA_ERR_WORKSPACE
    assert fwd(h0=ODD) == _lib.KLA_ERR_ALIGN
    assert fwd(ws_bytes=0) == _lib.KLA_ERR_WORKSPACE

    def bwd(dtype=_lib.KLA_DTYPE_F32, dh=ALIGNED, g=ALIGNED, h=ALIGNED, h0=None, dg=ALIGNED, du=ALIGNED,
            dh0=None, shape=(2, 3, 4), ws=WS, ws_bytes=1 << 40):
        return lib.kla_affine_scan_bwd(dtype, dh, g, h, h0, dg, du, dh0, *shape, ws, ws_bytes, None)

    assert bwd(dtype=-1) == _lib.KLA_ERR_DTYPE
    assert bwd(h=None) == _lib.KLA_ERR_INVALID_ARG
    assert bwd(du=ODD) == _lib.KLA_ERR_ALIGN
    assert bwd(ws=WS + 64) == _lib.KLA_ERR_WORKSPACE
    assert bwd(shape=(2, 0, 4), dh=None, g=None, h=None) == _lib.KLA_OK


def test_workspace_failures_validation(lib):
    out = ctypes.c_uint32(7)
    assert lib.kla_workspace_failures(WS, None, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_workspace_failures(None, None, None) == _lib.KLA_ERR_INVALID_ARG
    # NULL workspace: the current device's static scratch (the allocation-free
    # entry point's). Without a GPU there is no current device: a HIP error, and
    # nothing is written; with one (and no allocation-free call yet) the count is 0.
    rc = lib.kla_workspace_failures(None, None, ctypes.byref(out))
    if torch.cuda.is_available():
        assert rc == _lib.KLA_OK and out.value in (0, 7)
    else:
        assert rc == _lib.KLA_ERR_HIP and out.value == 7
        assert "kla_workspace_failures" in err(lib)


def test_set_kernel_events_validation(lib):
    E = ctypes.c_void_p(0x1000)
    assert lib.kla_set_kernel_events(2, None, None) == _lib.KLA_ERR_INVALID_ARG
    assert "unknown kernel 2" in err(lib)
    assert lib.kla_set_kernel_events(_lib.KLA_KERNEL_FUSED_BWD, E, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_set_kernel_events(_lib.KLA_KERNEL_FUSED_FWD, None, E) == _lib.KLA_ERR_INVALID_ARG
    for kernel in (_lib.KLA_KERNEL_FUSED_FWD, _lib.KLA_KERNEL_FUSED_BWD):
        assert lib.kla_set_kernel_events(kernel, None, None) == _lib.KLA_OK


def test_last_error_is_per_thread(lib):
    assert _mobius_fwd(lib, A=None) == _lib.KLA_ERR_INVALID_ARG
    seen = {}

    def other():
        seen["before"] = err(lib)
        lib.kla_affine_scan_fwd(5, None, None, None, None, 1, 1, 1, None, 0, None)
        seen["after"] = err(lib)

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == ""
    assert "unsupported dtype code 5" in seen["after"]
    assert "must not be NULL" in err(lib)


def test_python_errors_carry_the_message():
    e = _lib.KLAHipError("kla_x", 1, "boom")
    assert "kla_x failed with status 1: boom" in str(e)
    with pytest.raises(_lib.KLAHipError, match="must not be NULL"):
        _mobius_fwd(_lib.lib(), A=None)
        _lib.check("kla_mobius_scan_fwd", _lib.KLA_ERR_INVALID_ARG)


def test_fused_and_step_validation(lib):
    p = [ALIGNED] * 14
    shape = (2, 5, 6, 16)
    assert lib.kla_fused_scan_fwd(*p[:12], None, None, 0, 2, 5, 6, 257, None) == _lib.KLA_ERR_INVALID_ARG
    assert "above 256" in err(lib)
    assert lib.kla_fused_scan_fwd(*p[:12], ALIGNED, None, 0, *shape, None) == _lib.KLA_ERR_INVALID_ARG
    assert "both checkpoint buffers" in err(lib)
    assert lib.kla_fused_scan_fwd(None, *p[1:12], None, None, 0, *shape, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_fused_scan_fwd(ODD, *p[1:12], None, None, 0, *shape, None) == _lib.KLA_ERR_ALIGN
    assert lib.kla_fused_scan_fwd(*p[:12], None, None, 0, 0, 5, 6, 16, None) == _lib.KLA_OK
    assert lib.kla_fused_checkpoints(33) == 3 and lib.kla_fused_checkpoints(0) == 0
    n = lib.kla_fused_workspace_bytes(*shape)
    assert n >= 4 * (2 * 2 * 5 * 16 + 2 * 2 * 6 * 16)
    q = [ALIGNED] * 20
    assert lib.kla_fused_scan_bwd(*q, 0, *shape, None, n, None) == _lib.KLA_ERR_WORKSPACE
    assert lib.kla_fused_scan_bwd(*q, 0, *shape, WS, n - 4, None) == _lib.KLA_ERR_WORKSPACE
    assert lib.kla_fused_scan_bwd(*q[:4], None, *q[5:], 0, *shape, WS, n, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_step_fwd(*[ALIGNED] * 11, None, 0, 2, 6, 16, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_step_fwd(*[ALIGNED] * 11, ODD, 0, 2, 6, 16, None) == _lib.KLA_ERR_ALIGN
    assert lib.kla_step_fwd(*[ALIGNED] * 12, 0, 2, 6, 257, None) == _lib.KLA_ERR_INVALID_ARG


def test_decode_and_conv_step_validation(lib):
    cfg = _lib.DecodeConfig(discretization=0, obs_var_min=1e-4, obs_var_max=float("inf"), gate_activation=1)
    P = ALIGNED

    def dec(v=P, ld_v=8, lv=P, ld_lv=8, k=P, q=P, ld_kq=4, z=None, ld_z=0, skip=None, gate=None, ld_g=0,
            delta=P, ll=P, pn=P, lam=P, eta=P, lo=P, eo=P, y=P, yv=P, c=cfg, shape=(2, 8, 4)):
        return lib.kla_decode_step_fwd(v, ld_v, lv, ld_lv, k, q, ld_kq, z, ld_z, skip, gate, ld_g, delta, ll, pn,
                                       lam, eta, lo, eo, y, yv, ctypes.byref(c) if c is not None else None,
                                       *shape, None)

    assert dec(c=None) == _lib.KLA_ERR_INVALID_ARG
    assert "cfg must not be NULL" in err(lib)
    assert dec(shape=(2, 8, 257)) == _lib.KLA_ERR_INVALID_ARG
    assert dec(v=None) == _lib.KLA_ERR_INVALID_ARG
    assert dec(z=P, ld_z=8) == _lib.KLA_ERR_INVALID_ARG
    assert "residual and lambda_skip" in err(lib)
    assert dec(ld_v=7) == _lib.KLA_ERR_INVALID_ARG
    assert "row stride" in err(lib)
    bad = _lib.DecodeConfig(discretization=2)
    assert dec(c=bad) == _lib.KLA_ERR_INVALID_ARG
    bad = _lib.DecodeConfig(gate_activation=7)
    assert dec(c=bad, gate=P, ld_g=8) == _lib.KLA_ERR_INVALID_ARG
    assert dec(k=ODD) == _lib.KLA_ERR_ALIGN
    assert dec(shape=(0, 8, 4), v=None) == _lib.KLA_OK

    def conv(x=P, ld_x=8, st=P, so=P, w=P, b=None, act=1, y=P, shape=(2, 8, 4)):
        return lib.kla_conv_step_fwd(x, ld_x, st, so, w, b, act, y, *shape, None)

    assert conv(shape=(2, 8, 0)) == _lib.KLA_ERR_INVALID_ARG
    assert conv(act=5) == _lib.KLA_ERR_INVALID_ARG
    assert conv(ld_x=4) == _lib.KLA_ERR_INVALID_ARG
    assert conv(st=None) == _lib.KLA_ERR_INVALID_ARG
    assert conv(w=ODD) == _lib.KLA_ERR_ALIGN
    assert conv(shape=(0, 8, 4), x=None) == _lib.KLA_OK


def test_fused_sensors_validation(lib):
    P = ALIGNED
    shape = (2, 5, 6, 16)

    def sensors(**kw):
        a = dict(v=P, ld_v=10, obs=P, ld_obs=10, dtype=_lib.KLA_DTYPE_BF16, log_var=1, obs_var_min=1e-4,
                 obs_var_max=float("inf"))
        a.update(kw)
        return _lib.Sensors(**a)

    def fwd(sn, k=P, shape=shape):
        return lib.kla_fused_scan_sensors_fwd(ctypes.byref(sn) if sn is not None else None, k, P, P, P, None, None,
                                              P, P, P, P, None, None, 0, *shape, None)

    assert fwd(None) == _lib.KLA_ERR_INVALID_ARG
    assert "sensors is NULL" in err(lib)
    assert fwd(sensors(dtype=7)) == _lib.KLA_ERR_DTYPE
    assert fwd(sensors(ld_v=5)) == _lib.KLA_ERR_INVALID_ARG
    assert "row strides" in err(lib)
    assert fwd(sensors(obs_var_max=0.0)) == _lib.KLA_ERR_INVALID_ARG
    assert fwd(sensors(v=P + 1)) == _lib.KLA_ERR_ALIGN
    assert fwd(sensors(v=ODD, dtype=_lib.KLA_DTYPE_F32)) == _lib.KLA_ERR_ALIGN
    assert fwd(sensors(v=None)) == _lib.KLA_ERR_INVALID_ARG
    assert fwd(sensors(), k=ODD) == _lib.KLA_ERR_ALIGN
    assert fwd(sensors(), shape=(2, 5, 6, 257)) == _lib.KLA_ERR_INVALID_ARG
    assert fwd(sensors(), shape=(0, 5, 6, 16)) == _lib.KLA_OK

    n = lib.kla_fused_workspace_bytes(*shape)

    def bwd(sn, dv=P, ws=WS, nbytes=n):
        return lib.kla_fused_scan_sensors_bwd(P, P, None, None, ctypes.byref(sn) if sn is not None else None,
                                              P, P, P, P, P, P, dv, P, P, P, P, P, None, None, 0, *shape, ws,
                                              nbytes, None)

    assert bwd(None) == _lib.KLA_ERR_INVALID_ARG
    assert bwd(sensors(), dv=P + 1) == _lib.KLA_ERR_ALIGN
    assert "sensor gradient" in err(lib)
    assert bwd(sensors(dtype=_lib.KLA_DTYPE_F32), dv=ODD) == _lib.KLA_ERR_ALIGN
    assert bwd(sensors(), dv=None) == _lib.KLA_ERR_INVALID_ARG
    assert bwd(sensors(), ws=None) == _lib.KLA_ERR_WORKSPACE
    assert bwd(sensors(), nbytes=n - 4) == _lib.KLA_ERR_WORKSPACE


def test_time_split_validation(lib):
    """kla_fused_chunk_maps and kla_chunk_starts (the time-split forward's two
    extra passes) check shape, sensors, NULL and alignment before launching."""
    P = ALIGNED
    P16 = ALIGNED + 16

    def sensors(**kw):
        a = dict(v=P, ld_v=6, obs=P, ld_obs=6, dtype=_lib.KLA_DTYPE_F32, log_var=0, obs_var_min=0.0,
                 obs_var_max=float("inf"))
        a.update(kw)
        return _lib.Sensors(**a)

    def maps(k=P, out=P, shape=(2, 5, 6, 16), s=None):
        s = sensors() if s is None else s
        return lib.kla_fused_chunk_maps(ctypes.byref(s), k, P, P, out, *shape, None)

    assert maps(shape=(2, 5, 6, 257)) == _lib.KLA_ERR_INVALID_ARG
    assert maps(shape=(2, -1, 6, 16)) == _lib.KLA_ERR_INVALID_ARG
    assert maps(shape=(0, 5, 6, 16)) == _lib.KLA_OK
    assert maps(out=None) == _lib.KLA_ERR_INVALID_ARG
    assert "maps must not be NULL" in err(lib)
    assert maps(k=None) == _lib.KLA_ERR_INVALID_ARG
    assert maps(s=sensors(v=None)) == _lib.KLA_ERR_INVALID_ARG
    assert maps(s=sensors(dtype=9)) == _lib.KLA_ERR_DTYPE
    assert maps(k=ODD) == _lib.KLA_ERR_ALIGN
    assert maps(out=P + 4) == _lib.KLA_ERR_ALIGN
    assert "16-byte" in err(lib)
    assert lib.kla_fused_chunk_maps(None, P, P, P, P, 2, 5, 6, 16, None) == _lib.KLA_ERR_INVALID_ARG

    def starts(m=P16, lam0=None, eta0=None, ls=P, es=P, le=None, ee=None, shape=(2, 4, 6, 16)):
        return lib.kla_chunk_starts(m, lam0, eta0, ls, es, le, ee, *shape, None)

    assert starts(shape=(-2, 4, 6, 16)) == _lib.KLA_ERR_INVALID_ARG
    assert starts(shape=(0, 4, 6, 16)) == _lib.KLA_OK
    assert starts(shape=(2, 0, 6, 16)) == _lib.KLA_OK
    assert starts(m=None) == _lib.KLA_ERR_INVALID_ARG
    assert starts(es=None) == _lib.KLA_ERR_INVALID_ARG
    assert starts(lam0=ODD) == _lib.KLA_ERR_ALIGN
    assert starts(m=P + 8) == _lib.KLA_ERR_ALIGN
    assert starts(le=P) == _lib.KLA_ERR_INVALID_ARG
    assert "go together" in err(lib)
    assert starts(le=P, ee=ODD) == _lib.KLA_ERR_ALIGN
    assert starts(shape=(2**31, 2**31, 2**31, 16)) == _lib.KLA_ERR_INVALID_ARG


def test_time_split_backward_validation(lib):
    """kla_fused_adjoint_maps and kla_adjoint_ends (the time-split backward's two
    extra passes) check shape, sensors, NULL and alignment before launching."""
    P = ALIGNED
    P16 = ALIGNED + 16

    def sensors(**kw):
        a = dict(v=P, ld_v=6, obs=P, ld_obs=6, dtype=_lib.KLA_DTYPE_F32, log_var=0, obs_var_min=0.0,
                 obs_var_max=float("inf"))
        a.update(kw)
        return _lib.Sensors(**a)

    def maps(dy=P, dyv=None, k=P, q=P, ck=P, out=P, shape=(2, 32, 6, 16), s=None):
        s = sensors() if s is None else s
        return lib.kla_fused_adjoint_maps(dy, dyv, ctypes.byref(s), k, q, P, P, ck, ck, out, 0, *shape, None)

    assert maps(shape=(2, 32, 6, 257)) == _lib.KLA_ERR_INVALID_ARG
    assert maps(shape=(2, -1, 6, 16)) == _lib.KLA_ERR_INVALID_ARG
    assert maps(shape=(0, 32, 6, 16)) == _lib.KLA_OK
    assert maps(out=None) == _lib.KLA_ERR_INVALID_ARG
    assert "maps must not be NULL" in err(lib)
    assert maps(dy=None) == _lib.KLA_ERR_INVALID_ARG
    assert maps(ck=None) == _lib.KLA_ERR_INVALID_ARG
    assert "checkpoints" in err(lib)
    assert maps(s=sensors(obs=None)) == _lib.KLA_ERR_INVALID_ARG
    assert maps(s=sensors(dtype=9)) == _lib.KLA_ERR_DTYPE
    assert maps(dyv=ODD) == _lib.KLA_ERR_ALIGN
    assert maps(out=P + 4) == _lib.KLA_ERR_ALIGN
    assert "16-byte" in err(lib)
    assert lib.kla_fused_adjoint_maps(P, None, None, P, P, P, P, P, P, P, 0, 2, 32, 6, 16,
                                      None) == _lib.KLA_ERR_INVALID_ARG

    def ends(m=P16, dl=None, de=None, gl=P, ge=P, shape=(2, 4, 6, 16)):
        return lib.kla_adjoint_ends(m, dl, de, gl, ge, *shape, None)

    assert ends(shape=(-2, 4, 6, 16)) == _lib.KLA_ERR_INVALID_ARG
    assert ends(shape=(0, 4, 6, 16)) == _lib.KLA_OK
    assert ends(shape=(2, 0, 6, 16)) == _lib.KLA_OK
    assert ends(m=None) == _lib.KLA_ERR_INVALID_ARG
    assert ends(ge=None) == _lib.KLA_ERR_INVALID_ARG
    assert ends(dl=ODD) == _lib.KLA_ERR_ALIGN
    assert ends(m=P + 8) == _lib.KLA_ERR_ALIGN
    assert ends(shape=(2**31, 2**31, 2**31, 16)) == _lib.KLA_ERR_INVALID_ARG


def test_train_chunks_plan():
    """The time-split training pair cuts grids below one workgroup per CU, doubling
    the chunk count while the grid stays below two per CU, with chunks that divide
    L into whole 16-step checkpoint blocks and last at least MIN_CHUNK steps."""
    from kla.ops.hip.fused import MIN_CHUNK, train_chunks

    assert train_chunks(4, 4096, 1024 * 2, 16, 256) == 1   # C4: 512 workgroups
    assert train_chunks(4, 1024, 1024, 16, 256) == 1       # one workgroup per CU
    assert train_chunks(2, 1024, 1024, 16, 256) == 4       # C1's shape with gradients: 128 -> 512
    assert train_chunks(1, 2048, 1024, 16, 256) == 8       # 64 -> 512
    assert train_chunks(2, 2048, 512, 64, 256) == 1        # 256 workgroups of 4 channels
    assert train_chunks(1, 2048, 512, 64, 256) == 4        # 128 -> 512
    assert train_chunks(1, 4096, 128, 256, 256) == 4       # 128 single-channel workgroups -> 512
    assert train_chunks(1, 256, 64, 16, 256) == 2          # 128-step chunks at least
    assert train_chunks(1, 100, 64, 16, 256) == 1          # not whole 16-step blocks
    assert train_chunks(1, 2 * MIN_CHUNK + 16, 8, 16, 256) == 1
    for B, L, M, S in [(1, 4096, 64, 64), (3, 1024, 200, 32), (1, 65536, 1, 1), (2, 8192, 4096, 16)]:
        nc = train_chunks(B, L, M, S, 256)
        assert nc >= 1 and L % (16 * nc) == 0 and (nc == 1 or L // nc >= MIN_CHUNK)


def test_time_chunks_plan():
    """The time-split forward cuts only small grids (below one workgroup per CU up
    to d_state 64, two above), into up to eight workgroups per CU, with chunks
    that divide L and last at least MIN_CHUNK steps."""
    from kla.ops.hip.fused import MIN_CHUNK, time_chunks

    assert MIN_CHUNK == 128
    assert time_chunks(4, 4096, 2048, 16, 256) == 1       # C4: 512 workgroups already
    assert time_chunks(16, 2048, 1024, 16, 256) == 1      # C5 prefill
    assert time_chunks(2, 2048, 512, 128, 256) == 1       # 512 workgroups of 2 channels
    assert time_chunks(4, 1024, 1024, 16, 256) == 1       # one workgroup per CU at d_state 16
    assert time_chunks(1, 2048, 1024, 64, 256) == 1       # and at d_state 64
    assert time_chunks(1, 2048, 512, 64, 256) == 16       # half a workgroup per CU: split
    assert time_chunks(1, 4096, 512, 128, 256) == 8       # one per CU at d_state 128: split
    assert time_chunks(2, 1024, 512, 16, 256) == 8        # C1: 64 workgroups, 128-step chunks
    assert time_chunks(1, 2048, 1024, 16, 256) == 16
    assert time_chunks(1, 4096, 2048, 16, 256) == 16      # 128 -> 2048 workgroups
    assert time_chunks(1, 100, 1024, 16, 256) == 1
    assert time_chunks(1, 255, 8, 16, 256) == 1           # odd
    assert time_chunks(1, 2 * MIN_CHUNK, 8, 16, 256) == 2
    assert time_chunks(1, 2500, 8, 16, 256) == 4          # 2500 = 4 * 625
    assert time_chunks(1, 4096, 256, 256, 256) == 8       # 256 single-channel workgroups
    for B, L, M, S in [(1, 4096, 64, 64), (3, 1000, 200, 32), (1, 65536, 1, 1), (2, 8192, 4096, 16)]:
        nc = time_chunks(B, L, M, S, 256)
        assert L % nc == 0 and (nc == 1 or L // nc >= MIN_CHUNK)


def test_state_groups_plan():
    """d_state above 256 runs as groups of 256 state lanes with the remainder last;
    each group's checkpoints are one contiguous block of the [B, n_ck, M, S] buffer,
    in group order, so the blocks tile the buffer exactly."""
    import torch

    from kla.ops.hip.fused import MAX_STATE, _ck_group, state_groups, time_chunks, train_chunks

    assert MAX_STATE == 256
    for plan in (train_chunks, time_chunks):   # the planners plan one launch
        with pytest.raises(ValueError, match="state_groups"):
            plan(1, 1024, 4, 300, 256)
    assert state_groups(16) == [(0, 16)]
    assert state_groups(256) == [(0, 256)]
    assert state_groups(257) == [(0, 256), (256, 1)]
    assert state_groups(300) == [(0, 256), (256, 44)]
    assert state_groups(520) == [(0, 256), (256, 256), (512, 8)]
    B, n_ck, M, S = 2, 3, 5, 300
    ck = torch.arange(B * n_ck * M * S, dtype=torch.float32).view(B, n_ck, M, S)
    blocks = [_ck_group(ck, B, n_ck, M, s0, n) for s0, n in state_groups(S)]
    assert [tuple(b.shape) for b in blocks] == [(B, n_ck, M, 256), (B, n_ck, M, 44)]
    assert all(b.is_contiguous() and b.data_ptr() >= ck.data_ptr() for b in blocks)
    assert torch.equal(torch.cat([b.reshape(-1) for b in blocks]), ck.view(-1))


def test_sensor_row_layouts():
    """Which [B, L, M] views the fused-sensor kernels read in place: rows of one
    stride ld >= M with element (b, t, m) at (b * L + t) * ld + m."""
    import torch

    from kla.ops.hip.fused import _sensor_rows

    proj = torch.zeros(3, 7, 20)
    assert _sensor_rows(proj[..., :6]) == 20
    assert _sensor_rows(proj[..., 7:13]) == 20
    assert _sensor_rows(torch.zeros(3, 7, 6)) == 6
    assert _sensor_rows(proj[:, :1, :6]) == 140          # one step: the batch stride is the row stride
    assert _sensor_rows(proj[:1, :, :6]) == 20
    assert _sensor_rows(proj[:1, :1, :6]) == 6
    assert _sensor_rows(proj[:, :5, :6]) is None          # batch stride 140 != 5 * 20
    assert _sensor_rows(proj[..., :6].transpose(0, 1).contiguous().transpose(0, 1)) is None
    assert _sensor_rows(proj.transpose(1, 2)[..., :6]) is None


def test_gate_skip_validation(lib):
    P = ALIGNED

    def fwd(dtype=_lib.KLA_DTYPE_BF16, odt=_lib.KLA_DTYPE_F32, y=P, res=P, ld_res=8, gate=P, ld_gate=16, lam=P,
            vec=0, act=1, out=P, shape=(5, 8)):
        return lib.kla_gate_skip_fwd(dtype, odt, y, res, ld_res, gate, ld_gate, lam, vec, act, out, *shape, None)

    assert fwd(dtype=9) == _lib.KLA_ERR_DTYPE
    assert fwd(odt=9) == _lib.KLA_ERR_DTYPE
    assert fwd(odt=_lib.KLA_DTYPE_BF16, out=P + 1) == _lib.KLA_ERR_ALIGN
    assert fwd(act=4) == _lib.KLA_ERR_INVALID_ARG
    assert fwd(lam=None) == _lib.KLA_ERR_INVALID_ARG
    assert "needs lambda_skip" in err(lib)
    assert fwd(ld_gate=7) == _lib.KLA_ERR_INVALID_ARG
    assert fwd(res=P + 1) == _lib.KLA_ERR_ALIGN
    assert fwd(out=None) == _lib.KLA_ERR_INVALID_ARG
    assert fwd(y=ODD) == _lib.KLA_ERR_ALIGN
    assert fwd(shape=(0, 8), y=None) == _lib.KLA_OK
    n = lib.kla_gate_skip_workspace_bytes(5, 8)
    assert n >= 4 * (1 * 8 + 8 + 1)

    def bwd(dl=P, ws=WS, nbytes=n, dres=P, dy=P, dout=P):
        return lib.kla_gate_skip_bwd(_lib.KLA_DTYPE_BF16, _lib.KLA_DTYPE_BF16, dout, P, P, 8, P, 16, P, 0, 1, dy,
                                     dres, P, dl, 5, 8, ws, nbytes, None)

    assert bwd(dl=None) == _lib.KLA_ERR_INVALID_ARG
    assert bwd(ws=None) == _lib.KLA_ERR_WORKSPACE
    assert bwd(nbytes=n - 4) == _lib.KLA_ERR_WORKSPACE
    assert bwd(dres=P + 1) == _lib.KLA_ERR_ALIGN
    assert bwd(dy=None) == _lib.KLA_ERR_INVALID_ARG
    assert bwd(dout=P + 1) == _lib.KLA_ERR_ALIGN


def test_model_kernels_validation(lib):
    P = ALIGNED
    assert lib.kla_rms_norm_fwd(5, P, P, 1e-5, P, 4, 8, None) == _lib.KLA_ERR_DTYPE
    assert lib.kla_rms_norm_fwd(_lib.KLA_DTYPE_F32, None, P, 1e-5, P, 4, 8, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_rms_norm_fwd(_lib.KLA_DTYPE_F32, ODD, P, 1e-5, P, 4, 8, None) == _lib.KLA_ERR_ALIGN
    assert lib.kla_rms_norm_fwd(_lib.KLA_DTYPE_F32, None, None, 1e-5, None, 0, 8, None) == _lib.KLA_OK
    assert lib.kla_swiglu_fwd(_lib.KLA_DTYPE_BF16, P, 7, P, 4, 4, None) == _lib.KLA_ERR_INVALID_ARG
    assert "row stride" in err(lib)
    assert lib.kla_swiglu_fwd(_lib.KLA_DTYPE_BF16, P + 1, 8, P, 4, 4, None) == _lib.KLA_ERR_ALIGN
    assert lib.kla_swiglu_fwd(_lib.KLA_DTYPE_BF16, None, 8, None, 0, 4, None) == _lib.KLA_OK


def test_sum_parts_validation(lib):
    P = ALIGNED
    assert lib.kla_sum_parts(5, P, 4, 16, P, None) == _lib.KLA_ERR_DTYPE
    assert lib.kla_sum_parts(_lib.KLA_DTYPE_BF16, P, 0, 16, P, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_sum_parts(_lib.KLA_DTYPE_BF16, P, 4, -1, P, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_sum_parts(_lib.KLA_DTYPE_BF16, None, 4, 16, P, None) == _lib.KLA_ERR_INVALID_ARG
    assert lib.kla_sum_parts(_lib.KLA_DTYPE_F32, P + 2, 4, 16, P, None) == _lib.KLA_ERR_ALIGN
    assert lib.kla_sum_parts(_lib.KLA_DTYPE_F32, P, 4, 16, P + 2, None) == _lib.KLA_ERR_ALIGN
    assert lib.kla_sum_parts(_lib.KLA_DTYPE_F32, None, 4, 0, None, None) == _lib.KLA_OK


def test_mobius_fwd_noalloc_validation(lib):
    """The allocation-free Moebius forward checks its arguments like
    kla_mobius_scan_fwd and refuses problems whose look-back records exceed its
    static 32 MiB scratch, all before touching the GPU."""
    f = lib.kla_mobius_scan_fwd_noalloc
    assert f(ALIGNED, ALIGNED, ALIGNED, None, None, ALIGNED, 0, 5, 4, None) == _lib.KLA_OK
    assert f(None, ALIGNED, ALIGNED, None, None, ALIGNED, 2, 3, 4, None) == _lib.KLA_ERR_INVALID_ARG
    assert "kla_mobius_scan_fwd_noalloc" in err(lib) and "must not be NULL" in err(lib)
    assert f(ODD, ALIGNED, ALIGNED, None, None, ALIGNED, 2, 3, 4, None) == _lib.KLA_ERR_ALIGN
    assert f(ALIGNED, ALIGNED, ALIGNED, None, None, ALIGNED, -1, 3, 4, None) == _lib.KLA_ERR_INVALID_ARG
    need = lib.kla_scan_workspace_bytes(_lib.KLA_SCAN_MOBIUS_FWD, 16, 4096, 2048)
    assert need > 32 << 20
    assert f(ALIGNED, ALIGNED, ALIGNED, None, None, ALIGNED, 16, 4096, 2048, None) == _lib.KLA_ERR_WORKSPACE
    assert "static scratch holds 33554432" in err(lib)
    assert lib.kla_scan_workspace_bytes(_lib.KLA_SCAN_MOBIUS_FWD, 8, 4096, 2048) <= 32 << 20
