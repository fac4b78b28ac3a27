"""RMSNorm (reference ``looped_blockell/layers/norms.py:8-15``), run by the HIP kernel."""

from __future__ import annotations

import torch
from torch import nn

from .. import kernels


class RMSNorm(nn.Module):
    """``x / sqrt(mean(x^2) + eps) * scale``; scale initialised to ones, eps 1e-5.

    The reference infers the width at call time; a torch module takes it at
    construction (``dim``).
    """

    def __init__(self, dim: int, eps: float = 1e-5, device=None):
        super().__init__()
        self.eps = eps
        self.scale = nn.Parameter(torch.ones(dim, device=device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Differentiable in x and scale (``titan::rmsnorm_bwd``)."""
        lead = x.shape[:-1]
        y = kernels.rmsnorm(x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous(), self.scale, self.eps)
        return y.reshape(*lead, x.shape[-1])
