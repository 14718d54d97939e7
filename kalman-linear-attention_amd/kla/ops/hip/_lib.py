"""ctypes binding of libkla_hip.so (the C ABI declared in include/kla_hip.h).

The library is loaded after torch, so it binds to the HIP runtime torch already
brought into the process (both name it libamdhip64.so.7), and streams and device
pointers from torch are valid on its side. A missing or stale library is an
error here, never a silent fallback.
"""

from __future__ import annotations

import ctypes
import functools
import os
import threading

import torch

# KLA_HIP_LIB names another build of the same library (e.g. the host-sanitised
# one the ABI tests run against); by default the in-tree libkla_hip.so.
LIB_PATH = os.environ.get("KLA_HIP_LIB") or os.path.join(
    os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))), "lib", "libkla_hip.so")
ABI_VERSION = 17

KLA_OK = 0
KLA_ERR_INVALID_ARG = 1
KLA_ERR_WORKSPACE = 2
KLA_ERR_DTYPE = 3
KLA_ERR_ALIGN = 4
KLA_ERR_HIP = 5

KLA_DTYPE_F32 = 0
KLA_DTYPE_BF16 = 1

KLA_ROWS_PLAIN = 0
KLA_ROWS_RESIDUAL = 1
KLA_ROWS_SWIGLU = 2

KLA_SCAN_MOBIUS_FWD = 0
KLA_SCAN_MOBIUS_BWD = 1
KLA_SCAN_AFFINE_FWD = 2
KLA_SCAN_AFFINE_BWD = 3

KLA_KERNEL_FUSED_FWD = 0
KLA_KERNEL_FUSED_BWD = 1

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_SIGNATURES = {
    "kla_hip_abi_version": (ctypes.c_int, []),
    "kla_hip_last_error": (ctypes.c_char_p, []),
    "kla_scan_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, _i64, _i64, _i64]),
    "kla_workspace_failures": (ctypes.c_int, [_p, _p, ctypes.POINTER(ctypes.c_uint32)]),
    "kla_set_kernel_events": (ctypes.c_int, [ctypes.c_int, _p, _p]),
    "kla_mobius_scan_fwd": (ctypes.c_int, [_p] * 6 + [_i64] * 3 + [_p, ctypes.c_size_t, _p]),
    "kla_mobius_scan_fwd_noalloc": (ctypes.c_int, [_p] * 6 + [_i64] * 3 + [_p]),
    "kla_mobius_scan_bwd": (ctypes.c_int, [_p] * 12 + [_i64] * 3 + [_p, ctypes.c_size_t, _p]),
    "kla_affine_scan_fwd": (ctypes.c_int, [ctypes.c_int] + [_p] * 4 + [_i64] * 3 + [_p, ctypes.c_size_t, _p]),
    "kla_affine_scan_bwd": (ctypes.c_int, [ctypes.c_int] + [_p] * 7 + [_i64] * 3 + [_p, ctypes.c_size_t, _p]),
    "kla_fused_checkpoints": (_i64, [_i64]),
    "kla_fused_workspace_bytes": (ctypes.c_size_t, [_i64] * 4),
    "kla_fused_scan_fwd": (ctypes.c_int, [_p] * 14 + [ctypes.c_int] + [_i64] * 4 + [_p]),
    "kla_fused_scan_bwd": (ctypes.c_int, [_p] * 20 + [ctypes.c_int] + [_i64] * 4 + [_p, ctypes.c_size_t, _p]),
    "kla_fused_scan_sensors_fwd": (ctypes.c_int, [_p] * 13 + [ctypes.c_int] + [_i64] * 4 + [_p]),
    "kla_fused_scan_sensors_bwd": (ctypes.c_int, [_p] * 19 + [ctypes.c_int] + [_i64] * 4
                                   + [_p, ctypes.c_size_t, _p]),
    "kla_fused_chunk_maps": (ctypes.c_int, [_p] * 5 + [_i64] * 4 + [_p]),
    "kla_chunk_starts": (ctypes.c_int, [_p] * 7 + [_i64] * 4 + [_p]),
    "kla_fused_adjoint_maps": (ctypes.c_int, [_p] * 10 + [ctypes.c_int] + [_i64] * 4 + [_p]),
    "kla_adjoint_ends": (ctypes.c_int, [_p] * 5 + [_i64] * 4 + [_p]),
    "kla_step_fwd": (ctypes.c_int, [_p] * 12 + [ctypes.c_int] + [_i64] * 3 + [_p]),
    "kla_decode_step_fwd": (ctypes.c_int, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _p, _p, _i64] + [_p] * 10
                            + [_i64] * 3 + [_p]),
    "kla_conv_step_fwd": (ctypes.c_int, [_p, _i64, _p, _p, _p, _p, ctypes.c_int, _p] + [_i64] * 3 + [_p]),
    "kla_causal_conv_fwd": (ctypes.c_int, [ctypes.c_int, _p, _i64, _i64, _p, _p, _p, ctypes.c_int, _p, _p]
                            + [_i64] * 4 + [_p]),
    "kla_causal_conv_workspace_bytes": (ctypes.c_size_t, [_i64] * 4),
    "kla_gate_skip_fwd": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _p, _p, _i64, _p, _i64, _p, ctypes.c_int,
                                         ctypes.c_int, _p] + [_i64] * 2 + [_p]),
    "kla_gate_skip_workspace_bytes": (ctypes.c_size_t, [_i64] * 2),
    "kla_rms_norm_fwd": (ctypes.c_int, [ctypes.c_int, _p, _p, ctypes.c_float, _p, _i64, _i64, _p]),
    "kla_swiglu_fwd": (ctypes.c_int, [ctypes.c_int, _p, _i64, _p, _i64, _i64, _p]),
    "kla_rows_linear_qk_fwd": (ctypes.c_int, [_p, _i64, _p, _i64, _p, _p, _p, _i64, _i64, _i64, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_float, _p]),
    "kla_rows_linear_conv_fwd": (ctypes.c_int, [_p, _i64, _p, _i64, _p, _p, ctypes.c_float, _p, _i64, _i64, _i64,
                                                _i64, _p, _p, _p, _p, _i64, ctypes.c_int, ctypes.c_int, _p]),
    "kla_discretize_fwd": (ctypes.c_int, [_p] * 3 + [_i64] + [ctypes.c_int] * 3 + [ctypes.c_float] + [_p] * 3),
    "kla_discretize_bwd": (ctypes.c_int, [_p] * 3 + [_i64] + [ctypes.c_int] * 3 + [ctypes.c_float] + [_p] * 6),
    "kla_qk_sensors_fwd": (ctypes.c_int, [ctypes.c_int, _p, _i64, _p, _i64, _p, _p, _i64, _i64, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_float, _p]),
    "kla_qk_sensors_bwd": (ctypes.c_int, [ctypes.c_int, _p, _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_float, _p]),
    "kla_cat_cols": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _p, _p, _p, _p, _i64, _p]),
    "kla_sum_parts": (ctypes.c_int, [ctypes.c_int, _p, _i64, _i64, _p, _p]),
    "kla_gather_rows": (ctypes.c_int, [ctypes.c_int, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p]),
    "kla_argmax_rows": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _i64, _p, ctypes.c_size_t, _p]),
    "kla_argmax_workspace_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "kla_rows_linear_fwd": (ctypes.c_int, [ctypes.c_int, _p, _i64, _p, _i64, _p, _p, ctypes.c_float, _p, _i64, _p,
                                           _i64, _i64, _i64, _i64, _i64, _p]),
    "kla_gate_skip_bwd": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _p, _p, _p, _i64, _p, _i64, _p, ctypes.c_int,
                                         ctypes.c_int] + [_p] * 4 + [_i64] * 2 + [_p, ctypes.c_size_t, _p]),
    "kla_causal_conv_bwd": (ctypes.c_int, [ctypes.c_int, _p, _p, _i64, _i64, _p, _p, _p, ctypes.c_int, _p, _p, _p,
                                           _p, _p] + [_i64] * 4 + [_p, ctypes.c_size_t, _p]),
}


class DecodeConfig(ctypes.Structure):
    """kla_decode_config of include/kla_hip.h."""

    _fields_ = [
        ("discretization", ctypes.c_int),
        ("zero_process_noise", ctypes.c_int),
        ("qk_norm", ctypes.c_int),
        ("has_clip", ctypes.c_int),
        ("clip_value", ctypes.c_float),
        ("obs_var_min", ctypes.c_float),
        ("obs_var_max", ctypes.c_float),
        ("decode_from_prior", ctypes.c_int),
        ("gate_activation", ctypes.c_int),
        ("skip_vector", ctypes.c_int),
    ]


class Sensors(ctypes.Structure):
    """kla_sensors of include/kla_hip.h."""

    _fields_ = [
        ("v", ctypes.c_void_p),
        ("ld_v", ctypes.c_int64),
        ("obs", ctypes.c_void_p),
        ("ld_obs", ctypes.c_int64),
        ("dtype", ctypes.c_int),
        ("log_var", ctypes.c_int),
        ("obs_var_min", ctypes.c_float),
        ("obs_var_max", ctypes.c_float),
    ]


class KLAHipError(RuntimeError):
    """A libkla_hip.so entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


@functools.cache
def lib() -> ctypes.CDLL:
    """Load libkla_hip.so (once). Raises RuntimeError if it is missing or stale."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} not found: build the MI355X kernels with "
            "`python kalman-linear-attention_amd/csrc/build.py` (or __graft_entry__.build())."
        )
    handle = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    got = handle.kla_hip_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI version {got}, this package expects {ABI_VERSION}; rebuild it")
    return handle


def last_error() -> str:
    return lib().kla_hip_last_error().decode(errors="replace")


def check(fn: str, status: int) -> None:
    if status != KLA_OK:
        raise KLAHipError(fn, status, last_error())


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    """Handle of the current HIP stream of ``device``: the value of
    ``torch.cuda.current_stream(device).cuda_stream`` (the capture stream under
    graph capture) without building the Stream object, ~0.1 us of host time a call
    against ~2 us."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


# ------------------------------------------------------------ op dispatch
#
# Each kernel entry point is a torch.library custom op (autograd, fake tensors
# for torch.compile). Going through the dispatcher costs ~13 us of host time a
# call against ~2 us for a plain Python call, more than several of these kernels
# take on the GPU, so calls that need none of what it adds run the op's function
# directly.


def hip_op(name: str):
    """Decorator: ``torch.library.custom_op(name, mutates_args=())`` that keeps the
    undecorated function as ``op.direct``."""
    def wrap(fn):
        op = torch.library.custom_op(name, mutates_args=())(fn)
        op.direct = fn
        return op
    return wrap


_PLAIN = (torch.Tensor, torch.nn.Parameter)


def call(op, *args):
    """``op(*args)``, run without the dispatcher where it adds nothing: outside
    torch.compile / export tracing, every tensor argument a plain tensor or
    parameter (no fake or other subclass), and no autograd to record (grad mode
    off, or no tensor argument requires grad). The same function runs either way."""
    if torch.compiler.is_compiling():
        return op(*args)
    grad = torch.is_grad_enabled()
    for a in args:
        if isinstance(a, torch.Tensor) and (type(a) not in _PLAIN or (grad and a.requires_grad)):
            return op(*args)
    return op.direct(*args)


# ----------------------------------------------------------------- workspace
#
# One zero-filled workspace per (device, stream): the kernels keep it valid from
# call to call, and calls on one stream are ordered, so reuse needs no reset.

_WORKSPACES: dict = {}
_WS_LOCK = threading.Lock()


def workspace(kind: int, batch: int, steps: int, lanes: int, device: torch.device) -> tuple[torch.Tensor, int]:
    """(workspace tensor, stream handle) for a scan on the current stream of ``device``."""
    need = int(lib().kla_scan_workspace_bytes(kind, batch, steps, lanes))
    if need == 0:
        raise ValueError(f"kla_scan_workspace_bytes: {last_error()}")
    handle = stream(device)
    key = (device.index, handle)
    with _WS_LOCK:
        ws = _WORKSPACES.get(key)
        if ws is None or ws.numel() < need:
            size = max(need, 2 * ws.numel() if ws is not None else 0)
            with torch.cuda.stream(torch.cuda.current_stream(device)):
                ws = torch.zeros(size, dtype=torch.uint8, device=device)
            if ws.data_ptr() % 256:
                raise RuntimeError("workspace allocation is not 256-byte aligned")
            _WORKSPACES[key] = ws
    return ws, handle


_SCRATCH: dict = {}


def scratch(nbytes: int, device: torch.device) -> tuple[torch.Tensor, int]:
    """(uninitialised buffer of at least ``nbytes``, stream handle) for the current
    stream of ``device``: scratch whose contents no call relies on between calls
    (the fused backward's partial sums). Reused while large enough."""
    handle = stream(device)
    key = (device.index, handle)
    with _WS_LOCK:
        buf = _SCRATCH.get(key)
        if buf is None or buf.numel() < nbytes:
            with torch.cuda.stream(torch.cuda.current_stream(device)):
                buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            _SCRATCH[key] = buf
    return buf, handle


def workspace_failures(device: torch.device) -> int:
    """Look-back waits that gave up on the current stream's workspace (0 when healthy)."""
    stream = torch.cuda.current_stream(device)
    ws = _WORKSPACES.get((device.index, stream.cuda_stream))
    if ws is None:
        return 0
    out = ctypes.c_uint32(0)
    check("kla_workspace_failures", lib().kla_workspace_failures(ws.data_ptr(), stream.cuda_stream, ctypes.byref(out)))
    return int(out.value)


class KernelTimer:
    """Brackets launches of one fused kernel with HIP events (kla_set_kernel_events,
    process-wide, so the backward that torch's autograd launches from its own
    thread is seen too) while the context is open: ``arm()`` before each step
    hands the library a fresh event pair, and ``times_ms()`` are the durations
    of the last launch in each armed step, in order."""

    def __init__(self, kernel: int, device: torch.device):
        self.kernel, self.device = kernel, device
        self.pairs = []

    def arm(self):
        """Hand the library a fresh event pair for the next launch."""
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        stream = torch.cuda.current_stream(self.device)
        s.record(stream)   # creates the events; the library records them again at the launch
        e.record(stream)
        self.pairs.append((s, e))
        check("kla_set_kernel_events", lib().kla_set_kernel_events(self.kernel, s.cuda_event, e.cuda_event))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        check("kla_set_kernel_events", lib().kla_set_kernel_events(self.kernel, None, None))

    def times_ms(self) -> list:
        torch.cuda.synchronize(self.device)
        return [s.elapsed_time(e) for s, e in self.pairs]


def noalloc_failures(device: torch.device) -> int:
    """Look-back waits that gave up in the static scratch of kla_mobius_scan_fwd_noalloc
    on ``device`` (kla_workspace_failures with a NULL workspace; 0 if never used)."""
    stream = torch.cuda.current_stream(device)
    out = ctypes.c_uint32(0)
    with torch.cuda.device(device):
        check("kla_workspace_failures", lib().kla_workspace_failures(None, stream.cuda_stream, ctypes.byref(out)))
    return int(out.value)


def workspace_failures_all(device: torch.device) -> int:
    """Look-back waits that gave up on every stream's workspace of ``device``."""
    total = 0
    for (index, stream_handle), ws in list(_WORKSPACES.items()):
        if index != device.index:
            continue
        out = ctypes.c_uint32(0)
        check("kla_workspace_failures", lib().kla_workspace_failures(ws.data_ptr(), stream_handle, ctypes.byref(out)))
        total += int(out.value)
    return total


def reset_workspaces() -> None:
    """Drop every cached workspace (the next call allocates a fresh zero-filled one)."""
    with _WS_LOCK:
        _WORKSPACES.clear()
        _SCRATCH.clear()
