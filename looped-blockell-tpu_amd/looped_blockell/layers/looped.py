"""Looped pre-norm SwiGLU block with shared weights.

The MLP half of the reference's core block applied L times:
``h <- h + MLPBlock(RMSNorm(h))`` (reference ``looped_blockell/layers/transformer_block.py:83-84``,
the core loop ``looped_blockell/looping/looped_model.py:293-350`` and the MLP path of
``csrc/loop/persistent_core.cu:315-335``), one operator call
(``titan::looped_swiglu``): the weights are packed once, then a gate/up and a down launch per
application with the carried state in fp32 (``titan::looped_swiglu_persistent`` runs all L in
one launch).  With gradients required the applications
run one by one through the differentiable RMSNorm and SwiGLU instead.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import kernels
from .mlp import MLPBlock
from .norms import RMSNorm


class LoopedSwiGLU(nn.Module):
    def __init__(self, d_model: int, d_ff: int, L: int, tile_size: int = 16, density: float = 1.0,
                 eps: float = 1e-5, device=None, bias: bool = True):
        super().__init__()
        self.L = L
        self.norm = RMSNorm(d_model, eps=eps, device=device)
        self.mlp = MLPBlock(d_model, d_ff, use_swiglu=True, tile_size=tile_size, density=density, device=device,
                            bias=bias)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        lead = h.shape[:-1]
        d = h.shape[-1]
        h2 = h.reshape(-1, d).to(torch.bfloat16).contiguous()
        if torch.is_grad_enabled() and (h.requires_grad or any(p.requires_grad for p in self.parameters())):
            # training: the L applications one by one through the differentiable RMSNorm and
            # SwiGLU (titan::rmsnorm_bwd, titan::block_ell_swiglu_bwd_bias), as the reference's
            # scan is differentiated (looped_blockell/looping/looped_model.py:342-350); the
            # carried state stays in fp32 as in the operator path
            hf = h2.float()
            for _ in range(self.L):
                hf = hf + self.mlp(self.norm(hf.to(torch.bfloat16))).float()
            return hf.to(torch.bfloat16).reshape(*lead, d)
        vg, cg, vu, cu, vd, cd = self.mlp.swiglu_weights()
        bg, bu, bd = self.mlp.swiglu_biases()
        out = kernels.looped_swiglu_bias(h2, self.norm.scale, vg, cg, bg, vu, cu, bu, vd, cd, bd, L=self.L,
                                         eps=self.norm.eps)
        return out.reshape(*lead, d)
