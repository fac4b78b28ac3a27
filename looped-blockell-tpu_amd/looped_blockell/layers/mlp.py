"""Block-ELL MLP layers (PyTorch), mirroring the reference's Flax module.

Reference: ``looped_blockell/layers/mlp.py``.

Weight layout per projection:
  values:      [R, K, B, B] parameter (tiles [B_in, B_out]), init N(0, 0.02)
  col_indices: [R, K] int32 buffer (topology, updated externally by pruning)
  alive_mask:  [R, K] bool buffer; dead tiles contribute nothing
  bias:        [out_features] parameter, zeros (BlockELLLinear only)

``MLPBlock(use_swiglu=True)`` runs the whole SwiGLU FFN as one fused HIP
operator (``titan::block_ell_swiglu_fwd_bias``, differentiable through
``titan::block_ell_swiglu_bwd_bias``); each projection carries a zero-initialised
trainable bias, as every ``BlockELLLinear`` of the reference's Flax module does
(``mlp.py:56-60``, ``:82``), added in fp32 in the kernels' epilogues.  ``bias=False``
gives the bias-free form of the reference's PyTorch mirror (``interop/pt_model.py:865-867``)
and CUDA operator (``csrc/block_ell/swiglu_fwd.cuh:75-84``).  The GELU form uses the tanh
approximation, ``jax.nn.gelu``'s default (``mlp.py:156``).

Forwards that need no gradient (``torch.no_grad()`` / ``torch.inference_mode()``) run from
weights prepared once per weight version: the bf16 tiles and their fragment-major packed copy
(``titan::block_ell_swiglu_prepack``, ``titan::block_ell_matmul_prepack`` for ``BlockELLLinear``)
are cached on the module and rebuilt when a value tensor,
a column-index buffer or an alive mask changes (tensor version counters), so such a forward is
the gate/up and down launches only.  Writes through ``.data`` bypass the version counter: call
``release_inference_cache()`` after them.  The cache holds about two bytes per weight element
twice (bf16 tiles, packed tiles); ``release_inference_cache()`` drops it.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import kernels
from .block_ell import BlockELLConfig, BlockELLTensor, create_random_topology


class BlockELLLinear(nn.Module):
    """Single Block-ELL linear layer (reference ``mlp.py:28-95``).

    ``K = max(1, int(C * density))``; at density 1.0 the topology is sequential,
    otherwise random and seeded from ``hash((out_features, in_features))`` so
    that layers of equal shape start with the same topology, as in the
    reference (``mlp.py:84-95``).
    """

    def __init__(self, out_features: int, in_features: int, tile_size: int = 16, density: float = 1.0,
                 dtype: torch.dtype = torch.bfloat16, bias: bool = True, device=None):
        super().__init__()
        B = tile_size
        if out_features % B or in_features % B:
            raise ValueError("features must be multiples of tile_size")
        self.out_features, self.in_features, self.tile_size = out_features, in_features, B
        self.density, self.dtype = density, dtype
        self.R, self.C = out_features // B, in_features // B
        self.K = max(1, int(self.C * density))
        self.values = nn.Parameter(torch.randn(self.R, self.K, B, B, device=device) * 0.02)
        self.bias = nn.Parameter(torch.zeros(out_features, device=device)) if bias else None
        self.register_buffer("col_indices", self._init_topology().to(device))
        self.register_buffer("alive_mask", torch.ones(self.R, self.K, dtype=torch.bool, device=device))
        self._eff_cache = None
        self._frozen = None

    def _init_topology(self) -> torch.Tensor:
        if self.density >= 1.0:
            return torch.arange(self.C, dtype=torch.int32).repeat(self.R, 1)[:, :self.K].contiguous()
        seed = hash((self.out_features, self.in_features)) % 2 ** 31
        return create_random_topology(self.R, self.C, self.K, seed)

    @property
    def config(self) -> BlockELLConfig:
        return BlockELLConfig(R=self.R, C=self.C, K=self.K, B=self.tile_size)

    def effective_col_indices(self) -> torch.Tensor:
        """col_indices with dead tiles (alive_mask False) set to the -1 sentinel (cached per version)."""
        key = (self.col_indices.data_ptr(), self.col_indices._version, self.alive_mask.data_ptr(),
               self.alive_mask._version)
        if self._eff_cache is None or self._eff_cache[0] != key:
            # an ordinary tensor even when built under inference mode: a later forward with
            # gradients saves it for the backward
            with torch.inference_mode(False):
                eff = torch.where(self.alive_mask, self.col_indices, torch.full_like(self.col_indices, -1))
                self._eff_cache = (key, eff.to(torch.int32).contiguous())
        return self._eff_cache[1]

    def kernel_values(self) -> torch.Tensor:
        return self.values.to(torch.bfloat16)

    def as_block_ell(self) -> BlockELLTensor:
        return BlockELLTensor(self.kernel_values(), self.effective_col_indices(), self.config)

    def _frozen_weight(self):
        """(bf16 tiles, effective columns, packed copy), rebuilt when the values or the topology change."""
        cols = self.effective_col_indices()
        key = (self.values.data_ptr(), self.values._version, self._eff_cache[0])
        if self._frozen is None or self._frozen[0] != key:
            with torch.inference_mode(False):
                v = self.kernel_values()
                self._frozen = (key, v, cols, kernels.block_ell_matmul_prepack(v, cols, self.in_features))
        return self._frozen[1:]

    def release_inference_cache(self) -> None:
        """Drop the cached bf16 and packed tiles of gradient-free forwards."""
        self._frozen = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        grad = torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))
        if grad:
            return kernels.block_ell_matmul(x, self.kernel_values(), self.effective_col_indices(), self.bias)
        # weights fixed across gradient-free forwards: bf16 tiles and their packed copy cached
        v, cols, packed = self._frozen_weight()
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous()
        y = kernels.block_ell_matmul_prepacked(x2, packed, v, cols, self.bias)
        return y.reshape(*lead, y.shape[-1])


class MLPBlock(nn.Module):
    """Block-ELL MLP (reference ``mlp.py:98-168``).

    SwiGLU: ``out = w_down(silu(w_gate(x)) * w_up(x))`` as one fused operator.
    GELU:   ``out = fc2(gelu(fc1(x)))`` with two Block-ELL products.
    """

    def __init__(self, d_model: int, d_ff: int, use_swiglu: bool = False, dropout: float = 0.0,
                 tile_size: int = 16, density: float = 1.0, dtype: torch.dtype = torch.bfloat16, device=None,
                 bias: bool = True):
        super().__init__()
        self.d_model, self.d_ff, self.use_swiglu, self.dropout = d_model, d_ff, use_swiglu, dropout
        kw = dict(tile_size=tile_size, density=density, dtype=dtype, device=device)
        if use_swiglu:
            self.w_gate = BlockELLLinear(d_ff, d_model, bias=bias, **kw)
            self.w_up = BlockELLLinear(d_ff, d_model, bias=bias, **kw)
            self.w_down = BlockELLLinear(d_model, d_ff, bias=bias, **kw)
        else:
            self.fc1 = BlockELLLinear(d_ff, d_model, **kw)
            self.fc2 = BlockELLLinear(d_model, d_ff, **kw)
        self._frozen = None

    def swiglu_weights(self):
        """(v_gate, ci_gate, v_up, ci_up, v_down, ci_down) in kernel form.

        When gate and up have the same topology (as initialised: both are seeded from the
        same hash, reference ``mlp.py:94``) the same index tensor is passed for both, which
        lets the kernel read each activation tile once for the two products.  The comparison
        runs once per topology version."""
        cg, cu = self.w_gate.effective_col_indices(), self.w_up.effective_col_indices()
        key = (self.w_gate._eff_cache[0], self.w_up._eff_cache[0])   # (pointer, version) of both
        if getattr(self, "_shared_key", None) != key:
            self._shared_key, self._shared = key, bool(torch.equal(cg, cu))
        if self._shared:
            cu = cg
        return (self.w_gate.kernel_values(), cg, self.w_up.kernel_values(), cu,
                self.w_down.kernel_values(), self.w_down.effective_col_indices())

    def _frozen_swiglu(self):
        """(kernel-form weights, packed copy), rebuilt when any weight's version changes."""
        lins = (self.w_gate, self.w_up, self.w_down)
        for lin in lins:
            lin.effective_col_indices()                  # refreshes each topology key
        key = tuple((lin.values.data_ptr(), lin.values._version, lin._eff_cache[0]) for lin in lins)
        if self._frozen is None or self._frozen[0] != key:
            w = self.swiglu_weights()
            self._frozen = (key, w, kernels.swiglu_prepack(*w))
        return self._frozen[1], self._frozen[2]

    def release_inference_cache(self) -> None:
        """Drop the cached bf16 and packed weights of gradient-free forwards."""
        self._frozen = None

    def swiglu_biases(self):
        """(b_gate, b_up, b_down): the projections' biases (None where a projection has none)."""
        return self.w_gate.bias, self.w_up.bias, self.w_down.bias

    def forward(self, x: torch.Tensor, deterministic: bool = True) -> torch.Tensor:
        lead = x.shape[:-1]
        if self.use_swiglu:
            x2 = x.reshape(-1, self.d_model).to(torch.bfloat16).contiguous()
            bg, bu, bd = self.swiglu_biases()
            grad = torch.is_grad_enabled() and (x2.requires_grad or any(p.requires_grad for p in self.parameters()))
            if grad:
                out = kernels.swiglu(x2, *self.swiglu_weights(), add_residual=False, b_gate=bg, b_up=bu, b_down=bd)
            else:
                w, packed = self._frozen_swiglu()
                out = kernels.swiglu_fwd_prepacked(x2, packed, *w, add_residual=False, b_gate=bg, b_up=bu, b_down=bd)
            out = out.reshape(*lead, self.d_model)
        else:
            out = self.fc2(F.gelu(self.fc1(x).float(), approximate="tanh").to(torch.bfloat16))
        if self.dropout > 0.0 and not deterministic:
            out = F.dropout(out, p=self.dropout, training=True)
        return out
