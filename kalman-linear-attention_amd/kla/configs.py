"""Configuration dataclasses of the KLA layer and sequence model.

Field names, defaults and meanings are those of the reference's
``kla.configs`` (src/kla/configs.py:45-240), so a config written for the
reference loads here unchanged. The one addition is the ``"hip"`` backend
family (MI355X kernels), which ``"auto"`` selects on ROCm devices.
"""

from __future__ import annotations

import dataclasses
from typing import Literal, Optional, Union

# Backend names accepted by kla_scan (reference configs.py:16-29, plus "hip").
# "auto" reads the device; every other value pins one implementation. The bare
# family name is that family's default implementation.
Backend = Literal[
    "auto",
    "torch",
    "hip",
    "hip_fused",
    "hip_composed",
    "triton",
    "triton_fused",
    "triton_composed",
    "cuda",
    "cuda_v2_2",
    "cuda_v2_1",
    "mps",
    "mps_fused",
    "mps_tiled",
    "mps_composed",
]
ScanImpl = Literal["auto", "associative", "doubling", "sequential"]
MobiusImpl = Literal["linear", "log"]

# Width of a d_inner-wide sensor signal produced from the post-conv stream z:
# "full" = one M x M map, "dt" = low rank ceil(d_model/8) (or dt_rank), an int =
# that rank, and for the value only, "conv" = v is z itself.
Rank = Union[int, Literal["full", "dt"]]
ValueRank = Union[int, Literal["full", "dt", "conv"]]


@dataclasses.dataclass
class KLAConfig:
    """Configuration of one :class:`~kla.layers.KLALayer` (reference configs.py:45-222)."""

    # dimensions
    d_state: int = 16
    expand: float = 2.0

    # discretisation of the static learned step Delta [d_inner, d_state]
    dt_min: float = 0.001
    dt_max: float = 0.1
    dt_init_floor: float = 1e-4
    discretization: Literal["ou", "zoh"] = "ou"

    # process / observation noise
    process_noise_scale: float = 0.01
    learnable_process_noise: bool = True
    zero_process_noise: bool = False
    obs_var_min: float = 1e-4
    obs_var_max: Optional[float] = None

    # sensor path shape ("plain" block: full/full, "mamba" block: conv/dt)
    value_rank: ValueRank = "full"
    var_rank: Rank = "full"

    # projections / normalisation
    qk_norm: bool = True
    bias: bool = False

    # short causal conv
    use_conv: bool = True
    conv_kernel_size: int = 4
    conv_activation: Literal["silu", "relu", "gelu"] = "silu"

    # gating / skip
    use_gating: bool = True
    gating_activation: Literal["silu", "gelu", "relu"] = "silu"
    use_lambda_skip: bool = True
    lambda_skip_mode: Literal["scalar", "vector"] = "scalar"
    lambda_skip_init: float = -1.0

    # probabilistic outputs
    return_variance: bool = False
    decode_from_prior: bool = False
    dt_rank: Optional[int] = None

    # numerics
    clip_value: Optional[float] = None

    # kernels
    backend: Backend = "auto"
    """Scan backend. "auto" picks "hip" for tensors on a ROCm GPU when the MI355X
    kernels are built, otherwise "torch"."""
    scan_impl: ScanImpl = "auto"
    """Parallel-scan form of the torch backend (ignored by kernel backends)."""
    mobius_impl: MobiusImpl = "linear"
    """Representation of the Moebius map in the torch backend ("linear" trace-
    normalised 2x2 products, or "log" logaddexp). Kernel backends are linear."""
    checkpoint_ssm: bool = False
    """Recompute the scan in backward (activation checkpointing)."""

    def d_inner(self, d_model: int) -> int:
        return int(self.expand * d_model)


@dataclasses.dataclass
class ModelConfig:
    """Embedding + N blocks (mixer [+ MLP]) + LM head (reference configs.py:224-240)."""

    vocab_size: int = 50304
    d_model: int = 512
    n_layers: int = 6
    mlp: Literal["none", "swiglu", "gelu"] = "swiglu"
    mlp_ratio: float = 4.0
    norm_eps: float = 1e-5
    tie_embeddings: bool = False
    logit_softcap: Optional[float] = None
