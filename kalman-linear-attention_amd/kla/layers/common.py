"""Building blocks around the KLA filter: activations, l2 norm, Delta init,
RMSNorm, the depthwise causal conv with carried state, and the channel MLP.

Behaviour (including parameter shapes, init distributions and the order in
which they draw from the torch RNG) matches the reference's
src/kla/layers/common.py, so seeded layers initialise identically.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

_ACTIVATIONS = {"silu": F.silu, "gelu": F.gelu, "relu": F.relu}


def get_activation(name: str):
    """Activation function by name ("silu", "gelu", "relu")."""
    if name not in _ACTIVATIONS:
        raise ValueError(f"Unknown activation {name!r}; expected one of {sorted(_ACTIVATIONS)}")
    return _ACTIVATIONS[name]


def l2_norm(x: torch.Tensor, eps: float = 1e-12) -> torch.Tensor:
    """x / max(||x||_2, eps) over the last dimension."""
    return x / x.norm(dim=-1, keepdim=True).clamp_min(eps)


def inv_softplus_dt_init(shape, dt_min: float, dt_max: float, dt_init_floor: float) -> torch.Tensor:
    """Delta drawn log-uniformly in [dt_min, dt_max] (floored), returned pre-softplus.

    softplus(dt + log(1 - exp(-dt))) = dt, so the stored value maps back to dt.
    """
    lo, hi = math.log(dt_min), math.log(dt_max)
    dt = torch.exp(torch.rand(*shape) * (hi - lo) + lo).clamp_min(dt_init_floor)
    return dt + torch.log(-torch.expm1(-dt))


def _hip_inference(backend: str, *tensors: torch.Tensor) -> bool:
    """Whether a module with kla backend ``backend`` runs its inference kernel on
    the MI355X: a hip-family backend on a ROCm GPU and no gradient to carry."""
    if backend == "torch" or not tensors[0].is_cuda:
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return False
    from kla.ops.kla_ops import _step_on_hip

    return _step_on_hip(backend, tensors[0])


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight, computed in float32.

    ``backend`` is the kla backend of the model it sits in (set by the model);
    on a hip-family backend, inference (no gradient) uses one HIP kernel."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))
        self.backend = "torch"

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype in (torch.float32, torch.bfloat16) and _hip_inference(self.backend, x, self.weight):
            from kla.ops.hip.model_ops import rms_norm_hip

            return rms_norm_hip(x, self.weight, self.eps)
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return (xf * self.weight.float()).to(x.dtype)


class CausalConv1d(nn.Module):
    """Depthwise causal conv over time on [B, L, D], with its state carried explicitly.

    The state is the last ``kernel_size - 1`` pre-conv inputs, [B, D, kernel_size - 1].
    """

    def __init__(self, dim: int, kernel_size: int, activation: str = "silu", bias: bool = True):
        super().__init__()
        self.dim = dim
        self.kernel_size = kernel_size
        self.activation = activation
        self.act = get_activation(activation)
        self.weight = nn.Parameter(torch.empty(dim, 1, kernel_size))
        self.bias = nn.Parameter(torch.empty(dim)) if bias else None
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self):
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            nn.init.zeros_(self.bias)

    def init_state(self, batch: int, device=None, dtype=None) -> torch.Tensor:
        return torch.zeros(batch, self.dim, self.kernel_size - 1, device=device, dtype=dtype)

    def forward(self, x: torch.Tensor, conv_state: torch.Tensor | None = None, hip: bool = False):
        """Returns (y [B, L, D], new_state [B, D, kernel_size - 1]).

        ``hip``: run the MI355X kernels (kla.ops.hip.conv; x on a ROCm GPU, fp32 or
        bf16), which stream over x once instead of concatenating and calling a
        library conv."""
        if hip:
            from kla.ops.hip.conv import causal_conv_hip

            return causal_conv_hip(x, conv_state, self.weight[:, 0, :], self.bias, self.activation)
        xt = x.transpose(1, 2)
        if conv_state is None:
            conv_state = self.init_state(x.shape[0], device=x.device, dtype=xt.dtype)
        padded = torch.cat((conv_state.to(xt.dtype), xt), dim=-1)
        if xt.shape[-1] == 1:
            # One decode token: the depthwise conv is a kernel_size-tap weighted sum
            # per channel (no convolution library call, so it replays in a HIP graph).
            y = (padded * self.weight[:, 0, :].to(padded.dtype)).sum(-1, keepdim=True)
            if self.bias is not None:
                y = y + self.bias.to(y.dtype).unsqueeze(-1)
        else:
            y = F.conv1d(padded, self.weight, self.bias, groups=self.dim)
        keep = self.kernel_size - 1
        new_state = padded[..., padded.shape[-1] - keep:]
        return self.act(y).transpose(1, 2), new_state


class MLP(nn.Module):
    """Channel mixer: SwiGLU (hidden = 2/3 of dim*ratio) or a GELU MLP."""

    def __init__(self, dim: int, ratio: float = 4.0, kind: str = "swiglu", bias: bool = False):
        super().__init__()
        hidden = int(dim * ratio)
        self.kind = kind
        self.backend = "torch"   # the model's kla backend (see RMSNorm)
        if kind == "swiglu":
            hidden = int(2 * hidden / 3)
            self.w12 = nn.Linear(dim, 2 * hidden, bias=bias)
            self.w3 = nn.Linear(hidden, dim, bias=bias)
        elif kind == "gelu":
            self.w1 = nn.Linear(dim, hidden, bias=bias)
            self.w2 = nn.Linear(hidden, dim, bias=bias)
        else:
            raise ValueError(f"Unknown MLP kind {kind!r}")

    def block_decode_ok(self, x: torch.Tensor, norm: "RMSNorm") -> bool:
        """Whether :meth:`block_decode_hip` serves ``x + self(norm(x))`` here: a SwiGLU
        MLP in inference on a hip backend, fp32 throughout, at most 64 rows."""
        if self.kind != "swiglu" or x.dtype != torch.float32 or x.numel() // max(x.shape[-1], 1) > 64:
            return False
        if any(p.dtype != torch.float32 for p in (self.w12.weight, self.w3.weight, norm.weight)):
            return False
        return _hip_inference(self.backend, x, self.w12.weight, self.w3.weight, norm.weight)

    def block_decode_hip(self, x: torch.Tensor, norm: "RMSNorm") -> torch.Tensor:
        """``x + self(norm(x))`` as two row kernels (kla.ops.hip.model_ops.rows_linear_hip):
        norm + w12 + SwiGLU, then w3 + the residual add. The values are those of the
        torch lines (reference src/kla/layers/common.py:45-55, :116-123 and the
        block's residual, src/kla/models/sequence_model.py:77) up to the order of
        the fp32 sums."""
        from kla.ops.hip.model_ops import rows_linear_hip

        x2 = x.reshape(-1, x.shape[-1])
        h = rows_linear_hip(x2, self.w12.weight, self.w12.bias, norm_weight=norm.weight, eps=norm.eps, swiglu=True)
        return rows_linear_hip(h, self.w3.weight, self.w3.bias, residual=x2).reshape(x.shape)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.kind == "swiglu":
            h = self.w12(x)
            if h.dtype in (torch.float32, torch.bfloat16) and _hip_inference(self.backend, h):
                from kla.ops.hip.model_ops import swiglu_hip

                return self.w3(swiglu_hip(h))
            gate, up = h.chunk(2, dim=-1)
            return self.w3(F.silu(gate) * up)
        return self.w2(F.gelu(self.w1(x)))
