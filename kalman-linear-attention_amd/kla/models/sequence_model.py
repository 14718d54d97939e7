"""Decoder-only sequence model: embedding, N pre-norm blocks, LM head
(reference src/kla/models/sequence_model.py:1-233).

Each block is ``x += mixer(norm(x))`` then, unless ``mlp="none"``,
``x += mlp(norm(x))``. Mixers come from a registry keyed by config type
(KLAConfig -> KLALayer); every mixer takes ``forward(x, state=None,
return_state=False)`` and ``init_state(batch)``, which is what makes stateful
prefill and O(1) decode work through :meth:`SequenceModel.generate`.
"""

from __future__ import annotations

from typing import Any, Callable, Optional, Sequence

import torch
import torch.nn as nn

from kla.configs import KLAConfig, ModelConfig
from kla.layers.common import MLP, RMSNorm
from kla.layers.kla_layer import KLALayer
from kla.models.readout import MarginalReadout

MixerBuilder = Callable[[int, Any], nn.Module]
_MIXER_REGISTRY: dict[type, MixerBuilder] = {}


def register_mixer(config_type: type, builder: MixerBuilder) -> None:
    """Register ``builder(d_model, config) -> nn.Module`` for a config dataclass type."""
    _MIXER_REGISTRY[config_type] = builder


def build_mixer(d_model: int, config: Any) -> nn.Module:
    builder = _MIXER_REGISTRY.get(type(config))
    if builder is None:
        raise TypeError(f"No mixer registered for config type {type(config).__name__}; "
                        "call kla.models.register_mixer first.")
    return builder(d_model, config)


register_mixer(KLAConfig, KLALayer)


class Block(nn.Module):
    def __init__(self, d_model: int, mixer_config: Any, model_config: ModelConfig):
        super().__init__()
        self.mixer_norm = RMSNorm(d_model, model_config.norm_eps)
        self.mixer = build_mixer(d_model, mixer_config)
        if model_config.mlp != "none":
            self.mlp_norm = RMSNorm(d_model, model_config.norm_eps)
            self.mlp = MLP(d_model, model_config.mlp_ratio, model_config.mlp)
        else:
            self.mlp_norm = None
            self.mlp = None
        # The norms and the MLP follow the mixer's kla backend for their inference kernels.
        backend = getattr(mixer_config, "backend", "torch")
        for m in (self.mixer_norm, self.mlp_norm, self.mlp):
            if m is not None:
                m.backend = backend

    def mix(self, x: torch.Tensor):
        """Sequence-mixing half: (x + mixer(norm(x)), variance or None). Stateless."""
        mixed = self.mixer(self.mixer_norm(x))
        mixed, var = mixed if isinstance(mixed, tuple) else (mixed, None)
        return x + mixed, var

    def channel(self, x: torch.Tensor) -> torch.Tensor:
        """Channel-mixing half: x + mlp(norm(x)) (identity when there is no MLP)."""
        return x if self.mlp is None else x + self.mlp(self.mlp_norm(x))

    def forward(self, x: torch.Tensor, state=None, return_state: bool = False):
        emit_state = return_state or state is not None
        if (state is not None and isinstance(self.mixer, KLALayer)
                and self.mixer.block_decode_ok(x, state) and self.mixer_norm.weight.dtype == torch.float32):
            # One-token step on the MI355X row kernels: norm + in_proj, the conv and
            # SSM steps, out_proj + residual; then norm + w12 + SwiGLU, w3 + residual.
            x, new_state = self.mixer.block_decode_hip(x, self.mixer_norm.weight, self.mixer_norm.eps, state)
            if self.mlp is not None and self.mlp.block_decode_ok(x, self.mlp_norm):
                x = self.mlp.block_decode_hip(x, self.mlp_norm)
            else:
                x = self.channel(x)
            return x, new_state
        if emit_state:
            mixed, new_state = self.mixer(self.mixer_norm(x), state=state, return_state=True)
            if isinstance(mixed, tuple):
                mixed = mixed[0]
            x = x + mixed
        else:
            x, _ = self.mix(x)
            new_state = None
        x = self.channel(x)
        return (x, new_state) if emit_state else x


class SequenceModel(MarginalReadout, nn.Module):
    """Decoder-only model over token ids with a unified mixer interface."""

    def __init__(self, config: ModelConfig, mixer: Any | Sequence[Any] | None = None):
        super().__init__()
        self.config = config
        if mixer is None:
            mixer = KLAConfig()
        mixers = list(mixer) if isinstance(mixer, (list, tuple)) else [mixer] * config.n_layers
        if len(mixers) != config.n_layers:
            raise ValueError(f"Got {len(mixers)} mixer configs for {config.n_layers} layers")
        self.embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.blocks = nn.ModuleList(Block(config.d_model, m, config) for m in mixers)
        self.norm_f = RMSNorm(config.d_model, config.norm_eps)
        self.norm_f.backend = getattr(mixers[-1], "backend", "torch") if mixers else "torch"
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        if config.tie_embeddings:
            self.lm_head.weight = self.embedding.weight
        self.apply(self._init_weights)

    def _init_weights(self, module: nn.Module):
        if isinstance(module, nn.Linear):
            if not getattr(module.weight, "_no_reinit", False):
                nn.init.normal_(module.weight, std=0.02)
            if module.bias is not None and not getattr(module.bias, "_no_reinit", False):
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, std=0.02)

    @property
    def device(self) -> torch.device:
        return self.embedding.weight.device

    def init_state(self, batch: int, device=None, dtype=None) -> list:
        device = device or self.device
        return [blk.mixer.init_state(batch, device=device, dtype=dtype) for blk in self.blocks]

    def _logits(self, x: torch.Tensor) -> torch.Tensor:
        if self._head_on_rows(x):
            # One-token step: final norm + LM head as one row kernel.
            from kla.ops.hip.model_ops import rows_linear_hip

            logits = rows_linear_hip(x.reshape(-1, x.shape[-1]), self.lm_head.weight, self.lm_head.bias,
                                     norm_weight=self.norm_f.weight, eps=self.norm_f.eps)
            logits = logits.reshape(*x.shape[:-1], logits.shape[-1])
        else:
            logits = self.lm_head(self.norm_f(x))
        cap = self.config.logit_softcap
        return logits if cap is None else cap * torch.tanh(logits / cap)

    def _embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Token embeddings; in inference on a hip backend one gather kernel
        (kla.ops.hip.model_ops.gather_rows_hip) instead of torch's index kernel."""
        w = self.embedding.weight
        if w.dtype in (torch.float32, torch.bfloat16) and input_ids.dtype == torch.int64:
            from kla.layers.common import _hip_inference

            if _hip_inference(self.norm_f.backend, w):
                from kla.ops.hip.model_ops import gather_rows_hip

                return gather_rows_hip(w, input_ids)
        return self.embedding(input_ids)

    def _head_on_rows(self, x: torch.Tensor) -> bool:
        """Whether the final norm + LM head of a one-token step runs as one row kernel."""
        if x.dim() != 3 or x.shape[1] != 1 or x.shape[0] > 64 or x.dtype != torch.float32:
            return False
        if self.lm_head.weight.dtype != torch.float32 or self.norm_f.weight.dtype != torch.float32:
            return False
        from kla.layers.common import _hip_inference

        return _hip_inference(self.norm_f.backend, x, self.lm_head.weight, self.norm_f.weight)

    def forward(self, input_ids: torch.Tensor, state: Optional[list] = None, return_state: bool = False):
        """input_ids [B, L] -> logits [B, L, vocab]; per-layer state in/out for prefill and decode."""
        emit_state = return_state or state is not None
        x = self._embed(input_ids)
        new_states = []
        for i, blk in enumerate(self.blocks):
            if emit_state:
                x, s = blk(x, state=state[i] if state is not None else None, return_state=True)
                new_states.append(s)
            else:
                x = blk(x)
        logits = self._logits(x)
        return (logits, new_states) if emit_state else logits

    def _trunk(self, input_ids: torch.Tensor):
        """ids -> (mu, var) just after the last block's sequence mixer."""
        x = self.embedding(input_ids)
        for blk in self.blocks[:-1]:
            x = blk(x)
        last = self.blocks[-1]
        mu, var = last.mix(x)
        self._last_block = last
        return mu, var

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        """Last channel mixer + final norm + LM head + softcap, as log-probabilities."""
        x = self._last_block.channel(x)
        logits = self.lm_head(self.norm_f(x)).float()
        cap = self.config.logit_softcap
        if cap is not None:
            logits = cap * torch.tanh(logits / cap)
        return torch.log_softmax(logits, dim=-1)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, temperature: float = 1.0,
                 top_k: Optional[int] = None, cuda_graph: bool = False) -> torch.Tensor:
        """Sample with recurrent state: one prefill, then O(1) work per new token.

        ``cuda_graph`` replays the one-token step as a HIP graph
        (:class:`kla.models.decode_graph.DecodeGraph`); same tokens, fewer launches.
        """
        self.eval()
        state = self.init_state(input_ids.shape[0])
        logits, state = self.forward(input_ids, state=state)
        out = [input_ids]
        token = self._sample(logits[:, -1], temperature, top_k)
        graph = None
        if cuda_graph and max_new_tokens > 1:
            from kla.models.decode_graph import DecodeGraph

            graph = DecodeGraph(self, state)
        for _ in range(max_new_tokens - 1):
            out.append(token)
            if graph is not None:
                logits = graph.step(token)
            else:
                logits, state = self.forward(token, state=state)
            token = self._sample(logits[:, -1], temperature, top_k)
        out.append(token)
        return torch.cat(out, dim=1)

    def _sample(self, logits: torch.Tensor, temperature: float, top_k: Optional[int]) -> torch.Tensor:
        if temperature <= 0:
            from kla.layers.common import _hip_inference

            if logits.dtype == torch.float32 and logits.shape[-1] > 0 and _hip_inference(self.norm_f.backend, logits):
                # Greedy choice as one kernel (torch.argmax's order: NaN first, ties to the lower id).
                from kla.ops.hip.model_ops import argmax_rows_hip

                return argmax_rows_hip(logits)
            return logits.argmax(dim=-1, keepdim=True)
        logits = logits / temperature
        if top_k is not None:
            kth = torch.topk(logits, top_k, dim=-1).values[..., -1, None]
            logits = logits.masked_fill(logits < kth, float("-inf"))
        return torch.multinomial(torch.softmax(logits.float(), dim=-1), num_samples=1)
