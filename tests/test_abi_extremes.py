"""Host-side size arithmetic of the C ABI at extreme shapes (no GPU needed).

Every workspace size is a product of caller-given counts. With dimensions up to
2^63 - 1 these products must neither overflow (undefined behaviour in C++)
nor wrap to a small size that a caller would then allocate: the queries return
0 ("too large") or a size below 2^62, and the entry points reject such calls
before anything is launched. Every call here is one the library must refuse
(workspace NULL or 0 bytes): fake device addresses are never dereferenced.

The same file runs against the host-sanitised build of the library in
tests/test_abi_sanitized.py, where AddressSanitizer and UndefinedBehaviorSanitizer
watch the arithmetic.
"""

import itertools

import pytest

from kla.ops.hip import _lib

ALIGNED = 0x7F0000000000
WS = 0x7F0000100000
EXTREME = [0, 1, 2**31 - 1, 2**31, 2**40, 2**62, 2**63 - 1]
LIMIT = 2**62


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


def _shapes(n):
    return itertools.product(EXTREME, repeat=n)


def test_workspace_queries_saturate(lib):
    for kind in range(4):
        for b, t, l in _shapes(3):
            n = lib.kla_scan_workspace_bytes(kind, b, t, l)
            assert n < LIMIT, (kind, b, t, l, n)
    for b, t, m in _shapes(3):
        for s in (1, 16, 256):
            assert lib.kla_fused_workspace_bytes(b, t, m, s) < LIMIT
    for b, t, c in _shapes(3):
        assert lib.kla_causal_conv_workspace_bytes(b, t, c, 4) < LIMIT
    for r, m in _shapes(2):
        assert lib.kla_gate_skip_workspace_bytes(r, m) < LIMIT
        assert lib.kla_argmax_workspace_bytes(r, m) < LIMIT
    # A saturated size reads as "too large", not as a small number.
    assert lib.kla_scan_workspace_bytes(0, 2**31, 2**31, 2**31) == 0
    assert "too large" in lib.kla_hip_last_error().decode()
    assert lib.kla_fused_workspace_bytes(2**31, 2**31, 2**31, 256) == 0
    assert lib.kla_gate_skip_workspace_bytes(2**62, 2**62) == 0


def test_scan_entry_points_reject_extreme_shapes(lib):
    refuse = {_lib.KLA_ERR_INVALID_ARG, _lib.KLA_ERR_WORKSPACE}
    P = ALIGNED
    for b, t, l in _shapes(3):
        if 0 in (b, t, l):
            continue
        assert lib.kla_mobius_scan_fwd(P, P, P, None, None, P, b, t, l, None, 0, None) in refuse
        assert lib.kla_mobius_scan_bwd(P, P, P, P, None, None, P, P, P, P, None, None, b, t, l, None, 0,
                                       None) in refuse
        assert lib.kla_affine_scan_fwd(0, P, P, None, P, b, t, l, None, 0, None) in refuse
        assert lib.kla_affine_scan_bwd(1, P, P, P, None, P, P, None, b, t, l, None, 0, None) in refuse
        if max(b, t, l) >= 2**31 - 1:
            # Records for 2^31 elements or more: far beyond the static scratch, refused on the host.
            assert lib.kla_mobius_scan_fwd_noalloc(P, P, P, None, None, P, b, t, l, None) in refuse


def test_fused_backward_rejects_extreme_shapes(lib):
    refuse = {_lib.KLA_ERR_INVALID_ARG, _lib.KLA_ERR_WORKSPACE}
    q = [ALIGNED] * 20
    for b, t, m in _shapes(3):
        if 0 in (b, t, m):
            continue
        for s in (16, 200):
            # A 256-byte aligned workspace of 0 bytes: rejected by its size, after the size is formed.
            assert lib.kla_fused_scan_bwd(*q, 0, b, t, m, s, WS, 0, None) in refuse


def test_conv_backward_rejects_extreme_shapes(lib):
    refuse = {_lib.KLA_ERR_INVALID_ARG, _lib.KLA_ERR_WORKSPACE}
    P = ALIGNED
    for b, t, c in _shapes(3):
        if 0 in (b, t, c):
            continue
        rc = lib.kla_causal_conv_bwd(0, P, P, c, t * c if t * c < 2**63 else 2**63 - 1, None, P, None, 1, None, P,
                                     None, P, None, b, t, c, 4, None, 0, None)
        assert rc in refuse
