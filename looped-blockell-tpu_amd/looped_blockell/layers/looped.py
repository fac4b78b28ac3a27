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


class LoopedCore(nn.Module):
    """The FFN path of the reference's looped core (``looped_blockell/looping/looped_model.py:293-340``,
    ``interop/pt_model.py:1441-1509``): per iteration the diagonal injection ``h = decay * h + dt * e``
    (``interop/pt_model.py:923-935``, same parameters and initial decay 0.447), ``n_core`` distinct
    pre-norm residual SwiGLU blocks, then the per-sequence depth freeze
    ``h = where(t < depths[b], h_new, h_agg)``.  ``forward(h, e, depths, L)`` takes ``h, e`` of shape
    ``[B, S, d_model]`` (or ``[N, d_model]``) and ``depths`` of shape ``[B]`` (or None: every
    sequence runs L iterations).  Without gradients it is one ``titan::looped_core`` call (fp32
    state, packed weights, masked state updates); with gradients the iterations run through the
    differentiable injection, RMSNorm and SwiGLU with ``torch.where`` for the freeze."""

    def __init__(self, d_model: int, d_ff: int, n_core: int, tile_size: int = 16, density: float = 1.0,
                 eps: float = 1e-5, device=None, bias: bool = True, init_decay: float = 0.447):
        super().__init__()
        import math
        self.n_core = n_core
        self.eps = eps
        self.norms = nn.ModuleList(RMSNorm(d_model, eps=eps, device=device) for _ in range(n_core))
        self.mlps = nn.ModuleList(MLPBlock(d_model, d_ff, use_swiglu=True, tile_size=tile_size, density=density,
                                           device=device, bias=bias) for _ in range(n_core))
        target_dt = -math.log(init_decay)
        self.log_A = nn.Parameter(torch.zeros(d_model, device=device))
        self.log_dt = nn.Parameter(torch.full((d_model,), math.log(math.exp(target_dt) - 1.0), device=device))

    def forward(self, h: torch.Tensor, e: torch.Tensor | None = None, depths: torch.Tensor | None = None,
                L: int = 1) -> torch.Tensor:
        lead = h.shape[:-1]
        d = h.shape[-1]
        seq_len = h.shape[-2] if h.dim() == 3 else 1
        h2 = h.reshape(-1, d).to(torch.bfloat16).contiguous()
        e2 = None if e is None else e.reshape(-1, d).to(torch.bfloat16).contiguous()
        if torch.is_grad_enabled() and (h.requires_grad or (e is not None and e.requires_grad)
                                        or any(p.requires_grad for p in self.parameters())):
            act = None
            if depths is not None:
                tok = torch.repeat_interleave(depths.to(h2.device, torch.int64), seq_len)[: h2.shape[0]]
            hf = h2.float()
            for t in range(L):
                h_new = hf
                if e2 is not None:
                    h_new = kernels.diagonal_injection(h_new.to(torch.bfloat16), e2, self.log_A, self.log_dt).float()
                for norm, mlp in zip(self.norms, self.mlps):
                    h_new = h_new + mlp(norm(h_new.to(torch.bfloat16))).float()
                if depths is not None:
                    act = (t < tok)[:, None]
                    hf = torch.where(act, h_new, hf)
                else:
                    hf = h_new
            return hf.to(torch.bfloat16).reshape(*lead, d)
        ws = [m.swiglu_weights() for m in self.mlps]
        bs = [m.swiglu_biases() for m in self.mlps]
        out = kernels.looped_core(
            h2, e2, self.log_A if e2 is not None else None, self.log_dt if e2 is not None else None,
            [n.scale for n in self.norms], [w[0] for w in ws], [w[1] for w in ws], [w[2] for w in ws],
            [w[3] for w in ws], [w[4] for w in ws], [w[5] for w in ws], L, biases=bs, depths=depths,
            seq_len=seq_len, eps=self.eps)
        return out.reshape(*lead, d)
