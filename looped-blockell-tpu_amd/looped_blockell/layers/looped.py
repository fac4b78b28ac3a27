"""Looped pre-norm SwiGLU block with shared weights.

The MLP half of the reference's core block applied L times:
``h <- h + MLPBlock(RMSNorm(h))`` (reference ``looped_blockell/layers/transformer_block.py:83-84``,
the core loop ``looped_blockell/looping/looped_model.py:293-350`` and the MLP path of
``csrc/loop/persistent_core.cu:315-335``), one operator call
(``titan::looped_swiglu``): the weights are packed once, the carried state is
kept in fp32, and each application is a gate/up launch with the RMSNorm fused
into its input stage followed by a down launch that adds into the state.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import kernels
from .mlp import MLPBlock
from .norms import RMSNorm


class LoopedSwiGLU(nn.Module):
    def __init__(self, d_model: int, d_ff: int, L: int, tile_size: int = 16, density: float = 1.0,
                 eps: float = 1e-5, device=None):
        super().__init__()
        self.L = L
        self.norm = RMSNorm(d_model, eps=eps, device=device)
        self.mlp = MLPBlock(d_model, d_ff, use_swiglu=True, tile_size=tile_size, density=density, device=device)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        lead = h.shape[:-1]
        d = h.shape[-1]
        h2 = h.reshape(-1, d).to(torch.bfloat16).contiguous()
        out = kernels.looped_swiglu(h2, self.norm.scale, *self.mlp.swiglu_weights(), L=self.L, eps=self.norm.eps)
        return out.reshape(*lead, d)
