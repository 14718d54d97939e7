"""Deterministic and Monte-Carlo read-outs of a model carrying a posterior
(reference src/kla/models/readout.py:34-89).

    deterministic   log softmax(head(mu))
    Monte Carlo     log (1/S) sum_s softmax(head(mu + eps_s * std))
"""

from __future__ import annotations

import math

import torch


def marginal_logprobs(head, mu, var, mc_samples: int, generator=None, owner: str = "model"):
    """log (1/S) sum_s softmax(head(mu + eps_s std)), all S samples in one batch.

    ``head`` returns log-probabilities and broadcasts over a leading sample axis;
    the mean of the S distributions is taken in log space with logsumexp.
    """
    if var is None:
        raise ValueError(f"{owner}: mc_samples>0 needs a mixer that emits a variance -- set "
                         "return_variance=True on a KLAConfig.")
    std = var.clamp_min(1e-12).sqrt()
    eps = torch.randn((mc_samples, *mu.shape), device=mu.device, dtype=mu.dtype, generator=generator)
    log_p = head(mu + eps * std)
    return torch.logsumexp(log_p, dim=0) - math.log(mc_samples)


class MarginalReadout:
    """Mixin: :meth:`logprobs` in terms of the model's ``_trunk`` and ``_head``."""

    def logprobs(self, input_ids: torch.Tensor, mc_samples: int = 0, generator=None):
        """(deterministic, mc) log-probabilities from one trunk evaluation; mc is None if mc_samples=0."""
        mu, var = self._trunk(input_ids)
        det = self._head(mu)
        if not mc_samples:
            return det, None
        return det, marginal_logprobs(self._head, mu, var, mc_samples, generator, owner=type(self).__name__)
