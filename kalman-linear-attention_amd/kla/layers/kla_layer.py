"""The KLA sequence-mixing layer (reference src/kla/layers/kla_layer.py:49-349).

    x [B, L, D] -> in_proj -> (z, gate) [B, L, d_inner]
    z -> causal conv -> sensor_proj -> v, log sigma^2_v [B, L, M], k, q [B, L, S]
    static Delta, a, p -> discrete (a_bar, p_bar) [M, S]
    -> kla_scan (information-form Kalman filter) -> y [B, L, M]
    -> lambda-skip, gate -> out_proj -> [B, L, D]

Everything is driven by :class:`kla.configs.KLAConfig`; the scan itself is
:func:`kla.ops.kla_scan` (or :func:`kla.ops.kla_step` for one-token decode),
dispatched on ``config.backend``. Modules are created and initialised in the
reference's order, so a seeded layer draws the same parameters.
"""

from __future__ import annotations

import math
from typing import NamedTuple, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from kla.configs import KLAConfig
from kla.layers.common import CausalConv1d, get_activation, inv_softplus_dt_init, l2_norm
from kla.ops import KLAState, init_state, kla_scan, kla_step
from kla.ops.kla_ops import _resolve_auto, _step_on_hip


class KLALayerState(NamedTuple):
    """Recurrent state of one layer: the conv window and the filter state."""

    conv: Optional[torch.Tensor]  # [B, d_inner, K - 1]
    ssm: KLAState  # (lam, eta), each [B, d_inner, d_state]


class KLALayer(nn.Module):
    def __init__(self, d_model: int, config: KLAConfig | None = None):
        super().__init__()
        cfg = config if config is not None else KLAConfig()
        self.config = cfg
        self.d_model = d_model
        self.d_inner = cfg.d_inner(d_model)
        self.d_state = cfg.d_state
        M, S = self.d_inner, self.d_state

        self.in_proj = nn.Linear(d_model, 2 * M if cfg.use_gating else M, bias=cfg.bias)
        self.conv = CausalConv1d(M, cfg.conv_kernel_size, cfg.conv_activation) if cfg.use_conv else None

        # One projection emits v (unless v = z), log sigma^2_v (full width or a
        # low-rank code), k and q.
        rank = cfg.dt_rank or math.ceil(d_model / 8)
        self._value_rank = rank if cfg.value_rank == "dt" else cfg.value_rank
        self._var_rank = rank if cfg.var_rank == "dt" else cfg.var_rank
        if self._value_rank == "conv":
            self._w_value = 0
        elif self._value_rank == "full":
            self._w_value = M
        else:
            self._w_value = int(self._value_rank)
        self._w_var = M if self._var_rank == "full" else int(self._var_rank)
        self.sensor_proj = nn.Linear(M, self._w_value + self._w_var + 2 * S, bias=cfg.bias)
        low_rank_value = self._value_rank not in ("full", "conv")
        self.value_expand = nn.Linear(int(self._value_rank), M, bias=cfg.bias) if low_rank_value else None
        self.var_expand = nn.Linear(int(self._var_rank), M, bias=cfg.bias) if self._var_rank != "full" else None

        # Static, time-invariant dynamics: step Delta, continuous rate a = -exp(lambda_log), noise p.
        self.delta = nn.Parameter(torch.empty(M, S))
        self.delta._no_weight_decay = True
        self.lambda_log = nn.Parameter(torch.empty(M, S))
        self.lambda_log._no_weight_decay = True
        if cfg.learnable_process_noise and not cfg.zero_process_noise:
            self.process_noise = nn.Parameter(torch.empty(M, S))
        else:
            self.register_buffer("process_noise", torch.empty(M, S))

        if cfg.use_lambda_skip:
            shape = (M,) if cfg.lambda_skip_mode == "vector" else ()
            self.lambda_skip = nn.Parameter(torch.empty(shape))
        else:
            self.lambda_skip = None

        self.gate_act = get_activation(cfg.gating_activation) if cfg.use_gating else None
        # One-token hip decode writes the new state over the state it was given
        # (set by a decode graph that owns its state buffers); otherwise new tensors.
        self._decode_in_place = False
        self.out_proj = nn.Linear(M, d_model, bias=cfg.bias)
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self):
        """(Re-)initialise every parameter (safe after meta-device construction)."""
        cfg = self.config
        for mod in self.modules():
            if isinstance(mod, (nn.Linear, CausalConv1d)):
                mod.reset_parameters()
        self.delta.copy_(inv_softplus_dt_init((self.d_inner, self.d_state), cfg.dt_min, cfg.dt_max,
                                              cfg.dt_init_floor))
        self.lambda_log.zero_()
        self.process_noise.fill_(0.0 if cfg.zero_process_noise else cfg.process_noise_scale)
        if self.lambda_skip is not None:
            self.lambda_skip.fill_(cfg.lambda_skip_init)

    # ------------------------------------------------------------------ state

    def init_state(self, batch: int, device=None, dtype=None) -> KLALayerState:
        conv = self.conv.init_state(batch, device=device, dtype=dtype) if self.conv is not None else None
        return KLALayerState(conv=conv, ssm=init_state(batch, self.d_inner, self.d_state, device=device))

    # ------------------------------------------------------------- dynamics

    def _continuous_params(self):
        """Continuous transition a (< 0) and process noise p, each [M, S]."""
        cfg = self.config
        a = -torch.exp(self.lambda_log.float())
        p = self.process_noise.float()
        if cfg.zero_process_noise:
            p = p + 1e-12
        else:
            p = p.clamp_min(1e-7)
            if cfg.clip_value is not None:
                p = p.clamp_max(cfg.clip_value)
        return a, p

    def _discretize(self, delta: torch.Tensor, a: torch.Tensor, p: torch.Tensor):
        """Delta -> a_bar = exp(Delta a) and p_bar (Ornstein-Uhlenbeck or zero-order hold)."""
        a_bar = torch.exp(delta * a)
        if self.config.discretization == "ou":
            rate = a.abs().clamp_min(1e-8)
            p_bar = (p / (2.0 * rate)) * (-torch.expm1(-2.0 * rate * delta))
        else:
            p_bar = p * delta
        return a_bar, p_bar

    def _compute_aq(self):
        """Discrete (a_bar, p_bar), each [M, S]."""
        if self._aq_on_hip():
            # One HIP kernel each way for the ~40 small torch kernels below.
            from kla.ops.hip.dynamics import discretize_hip

            cfg = self.config
            return discretize_hip(self.delta, self.lambda_log, self.process_noise,
                                  discretization=cfg.discretization, zero_process_noise=cfg.zero_process_noise,
                                  clip_value=cfg.clip_value)
        a, p = self._continuous_params()
        delta = F.softplus(self.delta.float()) + 1e-7
        return self._discretize(delta, a, p)

    # ----------------------------------------------------------- projections

    def _project_sensors_raw(self, z: torch.Tensor):
        """z [B, L, M] -> (v, log sigma^2 [B, L, M] in the projection's dtype, k, q
        [B, L, S] float32 after the norm and the clip)."""
        cfg = self.config
        S = self.d_state
        if self._qk_project_on_hip(z):
            # Inference at few tokens: value and variance columns as one hipBLASLt
            # product, k and q with their norm and clip as one HIP kernel (a 2S-row
            # tail would otherwise set hipBLASLt's tile for the whole product).
            from kla.ops.hip.sensors import qk_project_hip

            w, b = self.sensor_proj.weight, self.sensor_proj.bias
            n1 = self._w_value + self._w_var
            B, L, _ = z.shape
            k, q = qk_project_hip(z.reshape(B * L, z.shape[-1]), w[n1:], None if b is None else b[n1:], S,
                                  norm=cfg.qk_norm, clip=cfg.clip_value)
            v, log_var = torch.split(F.linear(z, w[:n1], None if b is None else b[:n1]),
                                     [self._w_value, self._w_var], dim=-1)
            if self._value_rank == "conv":
                v = z
            elif self.value_expand is not None:
                v = self.value_expand(v)
            if self.var_expand is not None:
                log_var = self.var_expand(log_var)
            return v, log_var, k.view(B, L, S), q.view(B, L, S)
        v, log_var, k, q = self._linear_split(self.sensor_proj, z, [self._w_value, self._w_var, S, S])
        if self._value_rank == "conv":
            v = z
        elif self.value_expand is not None:
            v = self.value_expand(v)
        if self.var_expand is not None:
            log_var = self.var_expand(log_var)
        if self._qk_on_hip(k):
            # Norm, clip and .float() of both as one HIP kernel each way (same values).
            from kla.ops.hip.sensors import qk_sensors_hip

            k, q = qk_sensors_hip(k, q, norm=cfg.qk_norm, clip=cfg.clip_value)
            return v, log_var, k, q
        if cfg.qk_norm:
            k, q = l2_norm(k), l2_norm(q)
        if cfg.clip_value is not None:
            k = k.clamp(-cfg.clip_value, cfg.clip_value)
            q = q.clamp(-cfg.clip_value, cfg.clip_value)
        return v, log_var, k.float(), q.float()

    def _project_sensors(self, z: torch.Tensor):
        """z [B, L, M] -> (v, lambda_v [B, L, M], k, q [B, L, S]), all float32."""
        cfg = self.config
        v, log_var, k, q = self._project_sensors_raw(z)
        obs_var = F.softplus(log_var.float()) + cfg.obs_var_min
        if cfg.obs_var_max is not None:
            obs_var = obs_var.clamp_max(cfg.obs_var_max)
        return v.float(), 1.0 / obs_var, k, q

    # ---------------------------------------------------------------- compute

    def _run_ssm(self, z: torch.Tensor, ssm_state: KLAState | None):
        cfg = self.config
        a_bar, p_bar = self._compute_aq()
        if self._sensors_on_hip(z):
            # The fused hip scan reads v and log sigma^2 straight from the projection
            # and forms lambda_v itself (the values _project_sensors would give).
            from kla.ops.hip.fused import kla_scan_fused_sensors

            v, obs, k, q = self._project_sensors_raw(z)

            def scan(v, log_var, k, q, lam0, eta0):
                y, y_var, lam, eta = kla_scan_fused_sensors(
                    v, log_var, k, q, a_bar, p_bar, lam0, eta0, log_var=True, obs_var_min=cfg.obs_var_min,
                    obs_var_max=cfg.obs_var_max, decode_from_prior=cfg.decode_from_prior,
                    with_var=cfg.return_variance)
                return y, y_var, KLAState(lam=lam, eta=eta)
        else:
            v, obs, k, q = self._project_sensors(z)

            def scan(v, lambda_v, k, q, lam0, eta0):
                state = None if lam0 is None else KLAState(lam=lam0, eta=eta0)
                return kla_scan(v, lambda_v, k, q, a_bar, p_bar, initial_state=state, backend=cfg.backend,
                                scan_impl=cfg.scan_impl, mobius_impl=cfg.mobius_impl,
                                decode_from_prior=cfg.decode_from_prior)

        lam0 = ssm_state.lam if ssm_state is not None else None
        eta0 = ssm_state.eta if ssm_state is not None else None
        with torch.autocast(device_type=z.device.type, enabled=False):
            if cfg.checkpoint_ssm and torch.is_grad_enabled() and self.training:
                return torch.utils.checkpoint.checkpoint(scan, v, obs, k, q, lam0, eta0, use_reentrant=False)
            return scan(v, obs, k, q, lam0, eta0)

    def _run_ssm_step(self, z: torch.Tensor, ssm_state: KLAState):
        """One-token decode, z [B, 1, M]."""
        cfg = self.config
        v, lambda_v, k, q = self._project_sensors(z)
        a_bar, p_bar = self._compute_aq()
        with torch.autocast(device_type=z.device.type, enabled=False):
            y, y_var, new_state = kla_step(v[:, 0], lambda_v[:, 0], k[:, 0], q[:, 0], a_bar, p_bar, ssm_state,
                                           decode_from_prior=cfg.decode_from_prior, backend=cfg.backend)
        return y.unsqueeze(1), y_var.unsqueeze(1), new_state

    def _split(self, t: torch.Tensor, sizes: list[int]):
        """torch.split(t, sizes, dim=-1); on a hip-family backend with a gradient to
        carry, the split whose backward concatenates on the MI355X."""
        if t.requires_grad and torch.is_grad_enabled() and _step_on_hip(self.config.backend, t):
            from kla.ops.hip.split import split_last

            return split_last(t, sizes)
        return torch.split(t, sizes, dim=-1)

    def _linear(self, mod: nn.Linear, x: torch.Tensor) -> torch.Tensor:
        """mod(x); on a hip-family backend with a gradient to carry, the projection
        whose weight gradient is split over the tokens (kla.ops.hip.linear)."""
        if torch.is_grad_enabled() and _step_on_hip(self.config.backend, x):
            from kla.ops.hip.linear import linear

            return linear(mod, x)
        return mod(x)

    def _linear_split(self, mod: nn.Linear, x: torch.Tensor, sizes: list[int]):
        """self._split(mod(x), sizes); on a hip-family backend with a gradient to
        carry, the projection and the split as one (kla.ops.hip.linear), and
        otherwise the product in row blocks where the pieces allow it
        (kla.ops.hip.linear.split_blocks)."""
        if _step_on_hip(self.config.backend, x):
            from kla.ops.hip.linear import linear_split, split_blocks

            pieces = linear_split(mod, x, sizes) if torch.is_grad_enabled() else None
            if pieces is None and not (torch.is_grad_enabled() and x.requires_grad):
                pieces = split_blocks(mod, x, sizes)
            if pieces is not None:
                return pieces
        return self._split(mod(x), sizes)

    def _qk_project_on_hip(self, z: torch.Tensor) -> bool:
        """Whether the k, q columns of the sensor projection, their norm and clip run
        as one HIP kernel (kla.ops.hip.sensors.qk_project_hip): inference (no
        gradient, no autocast), fp32 dense z on a ROCm GPU with a hip-family
        backend, d_state a power of two <= 16, value or variance columns beside
        them, and fewer than QK_PROJECT_MAX_TOKENS tokens."""
        from kla.ops.hip.sensors import QK_PROJECT_MAX_TOKENS

        S = self.d_state
        return (not torch.is_grad_enabled() and z.dtype == torch.float32 and z.dim() == 3 and z.is_cuda
                and self.sensor_proj.weight.dtype == torch.float32
                and S <= 16 and S & (S - 1) == 0 and self._w_value + self._w_var > 0
                and 0 < z.shape[0] * z.shape[1] < QK_PROJECT_MAX_TOKENS and z.is_contiguous()
                and not torch.is_autocast_enabled(z.device.type) and _step_on_hip(self.config.backend, z))

    def _qk_on_hip(self, k: torch.Tensor) -> bool:
        """Whether the k, q sensors come from the MI355X kernels: a hip-family backend
        on a ROCm GPU, fp32 or bf16 projection, d_state <= 64, and a norm or a clip
        to apply."""
        cfg = self.config
        return ((cfg.qk_norm or cfg.clip_value is not None) and k.dtype in (torch.float32, torch.bfloat16)
                and self.d_state <= 64 and k.dim() == 3 and _step_on_hip(cfg.backend, k))

    def _aq_on_hip(self) -> bool:
        """Whether (a_bar, p_bar) come from the MI355X kernels: fp32 parameters on a
        ROCm GPU and a hip-family backend."""
        params = (self.delta, self.lambda_log, self.process_noise)
        return (all(t.dtype == torch.float32 for t in params)
                and _step_on_hip(self.config.backend, self.delta))

    def _sensors_on_hip(self, z: torch.Tensor) -> bool:
        """Whether the sequence scan runs on the fused hip kernel with the sensor
        read-out inside it: a backend that picks the fused scan ("hip", "hip_fused"
        or "auto" on a ROCm GPU), d_state <= 256, a ROCm GPU."""
        from kla.ops.hip.fused import MAX_STATE

        backend = self.config.backend
        if backend == "auto":
            backend = _resolve_auto(z)
        return (backend in ("hip", "hip_fused") and self.d_state <= MAX_STATE and z.dtype != torch.float64
                and _step_on_hip(backend, z))

    def _tail_on_hip(self, y: torch.Tensor, residual: torch.Tensor, gate: torch.Tensor | None) -> bool:
        """Whether the skip + gate after the scan run on the MI355X kernels: a
        hip-family backend on a ROCm GPU, fp32 y, residual and gate of one dtype
        (fp32 or bf16), and a skip or a gate to apply. Not with return_variance
        and a gate: act(gate) then also scales y_var, and torch adds the two
        bf16 gradients of act(gate) before the activation's backward."""
        skip = self.lambda_skip is not None
        if not (skip or gate is not None) or y.dtype != torch.float32:
            return False
        if self.config.return_variance and gate is not None:
            return False
        dtypes = {t.dtype for t in ((residual,) if skip else ()) + ((gate,) if gate is not None else ())}
        return (len(dtypes) == 1 and dtypes <= {torch.float32, torch.bfloat16} and y.dim() == 3
                and _step_on_hip(self.config.backend, y))

    def _decode_on_hip(self, projected: torch.Tensor) -> bool:
        """Whether a one-token step runs on the MI355X decode kernels: inference
        (no gradient), fp32 activations on a ROCm GPU, a hip-family backend,
        d_state <= 256."""
        from kla.ops.hip.fused import MAX_STATE
        return (not torch.is_grad_enabled() and projected.dtype == torch.float32 and self.d_state <= MAX_STATE
                and _step_on_hip(self.config.backend, projected))

    def _conv_on_hip(self, z: torch.Tensor) -> bool:
        """Whether the causal conv runs on the MI355X kernels (with autograd)."""
        return (z.dtype in (torch.float32, torch.bfloat16) and self.conv.kernel_size <= 8
                and _step_on_hip(self.config.backend, z))

    def _decode_step_hip(self, z, gate, residual, ssm_state, rows_linear: bool = False):
        """The one-token SSM step with the lambda skip and the gate, as one HIP kernel
        (kla.ops.hip.decode); the same values as _run_ssm_step plus the tail of forward.
        ``rows_linear``: the sensor projection runs on kla.ops.hip.model_ops.rows_linear_hip."""
        from kla.ops.hip.decode import decode_step_hip

        cfg = self.config
        S = self.d_state
        if rows_linear:
            from kla.ops.hip.model_ops import rows_linear_hip

            proj = rows_linear_hip(z[:, 0], self.sensor_proj.weight, self.sensor_proj.bias)
        else:
            proj = self.sensor_proj(z)[:, 0]
        v, log_var, k, q = torch.split(proj, [self._w_value, self._w_var, S, S], dim=-1)
        if self._value_rank == "conv":
            v = z[:, 0]
        elif self.value_expand is not None:
            v = self.value_expand(v)
        if self.var_expand is not None:
            log_var = self.var_expand(log_var)
        skip = self.lambda_skip.float() if self.lambda_skip is not None else None
        lam, eta = ssm_state.lam.contiguous(), ssm_state.eta.contiguous()
        in_place = self._decode_in_place and lam is ssm_state.lam and eta is ssm_state.eta
        y, y_var, lam, eta = decode_step_hip(
            v, log_var, k, q, self.delta.float(), self.lambda_log.float(), self.process_noise.float(), lam, eta,
            residual=residual[:, 0] if skip is not None else None, lambda_skip=skip,
            gate=gate[:, 0] if gate is not None else None, gate_activation=cfg.gating_activation,
            discretization=cfg.discretization, zero_process_noise=cfg.zero_process_noise, qk_norm=cfg.qk_norm,
            clip_value=cfg.clip_value, obs_var_min=cfg.obs_var_min, obs_var_max=cfg.obs_var_max,
            decode_from_prior=cfg.decode_from_prior, in_place=in_place)
        return y.unsqueeze(1), y_var.unsqueeze(1), KLAState(lam=lam, eta=eta)

    def _one_token_hip(self, z, gate, state, rows_linear: bool = False):
        """Conv step and SSM step (with skip and gate) of one token on the HIP decode
        kernels (kla.ops.hip.decode): (y, y_var, conv_state, ssm_state)."""
        cfg = self.config
        conv_state = state.conv
        if self.conv is not None:
            from kla.ops.hip.decode import conv_step_hip

            # A torch prefill leaves the window as a view of its padded input.
            window = conv_state.to(z.dtype).contiguous()
            zc, conv_state = conv_step_hip(z[:, 0], window, self.conv.weight[:, 0, :], self.conv.bias,
                                           cfg.conv_activation,
                                           in_place=self._decode_in_place and window is state.conv)
            z = zc.unsqueeze(1)
        y, y_var, ssm_state = self._decode_step_hip(z, gate, z, state.ssm, rows_linear=rows_linear)
        return y, y_var, conv_state, ssm_state

    def block_decode_ok(self, x: torch.Tensor, state: KLALayerState | None) -> bool:
        """Whether :meth:`block_decode_hip` serves this one-token step: the HIP decode
        kernels apply (inference, fp32, hip backend), fp32 projection weights, and a
        batch small enough for the row kernels (at most 64 rows)."""
        if state is None or x.dim() != 3 or x.shape[1] != 1 or x.shape[0] > 64 or x.dtype != torch.float32:
            return False
        if state.ssm.lam.dtype != torch.float32 or not self._decode_on_hip(x):
            return False
        if self.value_expand is not None or self.var_expand is not None:
            return False
        return all(m.weight.dtype == torch.float32 for m in (self.in_proj, self.sensor_proj, self.out_proj))

    def block_decode_hip(self, x: torch.Tensor, norm_weight: torch.Tensor, eps: float, state: KLALayerState):
        """``x + self(rms_norm(x), state)`` for one token (x [B, 1, d_model]), returning
        (that, new_state): the block's pre-norm and the conv step are fused into
        in_proj and the residual add into out_proj (kla.ops.hip.model_ops row
        kernels), the sensor projection runs on the same row kernel, and the SSM
        step is the HIP decode kernel. The values are those of the block's torch
        lines (reference src/kla/models/sequence_model.py:79-87) up to the order
        of the fp32 sums."""
        from kla.ops.hip.model_ops import rows_linear_hip

        cfg = self.config
        x2 = x[:, 0]
        window = state.conv
        if (self.conv is not None and self.conv.kernel_size <= 8 and window.dtype == torch.float32
                and window.is_contiguous()):
            # The conv step rides in in_proj's epilogue on the z columns.
            from kla.ops.hip.model_ops import rows_linear_conv_hip

            projected, conv_state = rows_linear_conv_hip(
                x2, self.in_proj.weight, self.in_proj.bias, norm_weight=norm_weight, eps=eps,
                conv_weight=self.conv.weight[:, 0, :], conv_bias=self.conv.bias, window=window,
                activation=cfg.conv_activation, in_place=self._decode_in_place)
            projected = projected.unsqueeze(1)
            z, gate = projected.chunk(2, dim=-1) if cfg.use_gating else (projected, None)
            y, _, ssm_state = self._decode_step_hip(z, gate, z, state.ssm, rows_linear=True)
        else:
            projected = rows_linear_hip(x2, self.in_proj.weight, self.in_proj.bias, norm_weight=norm_weight,
                                        eps=eps).unsqueeze(1)
            z, gate = projected.chunk(2, dim=-1) if cfg.use_gating else (projected, None)
            y, _, conv_state, ssm_state = self._one_token_hip(z, gate, state, rows_linear=True)
        out = rows_linear_hip(y[:, 0], self.out_proj.weight, self.out_proj.bias, residual=x2)
        return out.unsqueeze(1), KLALayerState(conv=conv_state, ssm=ssm_state)

    def forward(self, x: torch.Tensor, state: KLALayerState | None = None, return_state: bool = False):
        """x [B, L, d_model] -> out, or (out, new_state) when a state is passed or requested.

        ``out`` is y, or (y, y_var) when ``config.return_variance``.
        """
        cfg = self.config
        L = x.shape[1]
        emit_state = return_state or state is not None

        if cfg.use_gating:
            z, gate = self._linear_split(self.in_proj, x, [self.d_inner, self.d_inner])
            projected = z
        else:
            z = projected = self._linear(self.in_proj, x)
            gate = None
        # One-token inference step on the GPU: the conv step and the SSM step
        # (with skip and gate) run as two HIP kernels (kla.ops.hip.decode).
        hip_decode = (state is not None and L == 1 and state.ssm.lam.dtype == torch.float32
                      and self._decode_on_hip(projected))

        if hip_decode:
            y, y_var, conv_state, ssm_state = self._one_token_hip(z, gate, state)
        else:
            conv_state = state.conv if state is not None else None
            if self.conv is not None:
                z, conv_state = self.conv(z, conv_state, hip=self._conv_on_hip(z))
            residual = z
            ssm_state = state.ssm if state is not None else None
            if state is not None and L == 1:
                y, y_var, ssm_state = self._run_ssm_step(z, ssm_state)
            else:
                y, y_var, ssm_state = self._run_ssm(z, ssm_state)
            # y_var only reaches the output with return_variance; otherwise its
            # tail is skipped (the fused hip scan does not even compute it).
            y = y.to(x.dtype)
            y_var = y_var.to(x.dtype) if cfg.return_variance else None

            if self._tail_on_hip(y, residual, gate):
                # skip + gate as one HIP kernel each way (kla.ops.hip.tail); same values.
                from kla.ops.hip.tail import gate_skip_hip

                # Under bf16 autocast the output projection takes y in bf16: the
                # kernel writes it rounded (the same values), so no cast follows.
                autocast_bf16 = (torch.is_autocast_enabled(y.device.type)
                                 and torch.get_autocast_dtype(y.device.type) == torch.bfloat16)
                y = gate_skip_hip(y, residual if self.lambda_skip is not None else None, gate, self.lambda_skip,
                                  cfg.gating_activation,
                                  out_dtype=torch.bfloat16 if autocast_bf16 else torch.float32)
            else:
                if self.lambda_skip is not None:
                    y = y + self.lambda_skip * residual
                if gate is not None:
                    g = self.gate_act(gate)
                    y = y * g
                    if y_var is not None:
                        y_var = y_var * g.pow(2)

        out = self._linear(self.out_proj, y)
        result = (out, F.linear(y_var, self.out_proj.weight.pow(2))) if cfg.return_variance else out
        if emit_state:
            return result, KLALayerState(conv=conv_state, ssm=ssm_state)
        return result
