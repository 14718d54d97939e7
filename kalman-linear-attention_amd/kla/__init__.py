"""Kalman Linear Attention (KLA) with MI355X-native scan kernels.

Drop-in for the reference package ``kla`` (vaisakh-shaj/kalman-linear-attention):
same public API (KLAConfig, KLALayer, SequenceModel, kla_scan, kla_step, ...),
plus the ``"hip"`` backend, which ``backend="auto"`` selects on a ROCm GPU::

    import torch
    from kla import KLAConfig, KLALayer

    layer = KLALayer(d_model=512, config=KLAConfig(d_state=16)).cuda()
    y = layer(torch.randn(2, 1024, 512, device="cuda"))
"""

from kla.configs import KLAConfig, ModelConfig
from kla.layers import KLALayer, KLALayerState
from kla.models import SequenceModel, build_mixer, register_mixer
from kla.ops import KLAState, backend_names, kla_scan, kla_scan_reference, kla_step, resolve_backend

__version__ = "0.1.0"

__all__ = [
    "KLAConfig",
    "KLALayer",
    "KLALayerState",
    "KLAState",
    "ModelConfig",
    "SequenceModel",
    "backend_names",
    "build_mixer",
    "kla_scan",
    "kla_scan_reference",
    "kla_step",
    "register_mixer",
    "resolve_backend",
    "__version__",
]
