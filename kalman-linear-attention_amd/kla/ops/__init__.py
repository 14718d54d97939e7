from kla.ops.kla_ops import (
    KLAState,
    backend_names,
    default_device,
    init_state,
    kla_scan,
    kla_scan_reference,
    kla_scan_torch,
    kla_step,
    resolve_backend,
)

__all__ = [
    "KLAState",
    "backend_names",
    "default_device",
    "init_state",
    "kla_scan",
    "kla_scan_reference",
    "kla_scan_torch",
    "kla_step",
    "resolve_backend",
]
