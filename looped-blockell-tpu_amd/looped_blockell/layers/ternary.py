"""Ternary Block-ELL SwiGLU FFN: {-1,0,+1} tiles with one scale per block, int8 activations.

The arithmetic follows the reference's BitLinear quantisers
(``bonsai-test/bitlinear.py:34-69``) with the scaling group set to one B x B
Block-ELL tile: weights ``t = clamp(round(w / s), -1, 1)`` with
``s = mean|w|`` per tile, activations int8 per token with absmax scaling.
Tiles are stored 2 bits per weight (format of ``include/lbk.h``).
"""

from __future__ import annotations

import torch
from torch import nn

from .. import kernels
from .block_ell import create_random_topology


class TernaryBlockELLWeight(nn.Module):
    """Packed ternary Block-ELL weight: packed [R,K,B,B/16] int32, scales [R,K] fp32, col_indices [R,K]."""

    def __init__(self, packed: torch.Tensor, scales: torch.Tensor, col_indices: torch.Tensor):
        super().__init__()
        self.register_buffer("packed", packed)
        self.register_buffer("scales", scales)
        self.register_buffer("col_indices", col_indices.to(torch.int32))

    @classmethod
    def from_latent(cls, values: torch.Tensor, col_indices: torch.Tensor) -> "TernaryBlockELLWeight":
        """Quantise latent tiles [R,K,B,B] (per-tile absmean) on the GPU and pack them."""
        packed, scales = kernels.ternary_quantize_weights(values)
        return cls(packed, scales, col_indices)

    @classmethod
    def from_codes(cls, codes: torch.Tensor, scales: torch.Tensor, col_indices: torch.Tensor):
        """Pack int8 codes in {-1,0,+1} [R,K,B,B] (tiles [B_in, B_out])."""
        return cls(kernels.pack_ternary(codes.to(torch.int8).contiguous()), scales.float().contiguous(), col_indices)

    def triple(self):
        return (self.packed, self.scales, self.col_indices)


class TernaryMLPBlock(nn.Module):
    """SwiGLU FFN with ternary gate/up/down weights; forward quantises x per token.

    The kernels' prepared form of the three weights (``titan::ternary_prepare``) is cached on the
    module and rebuilt when a packed, scales or col_indices buffer changes (tensor version
    counters; writes through ``.data`` bypass them: call ``release_prepared()`` after those)."""

    def __init__(self, gate: TernaryBlockELLWeight, up: TernaryBlockELLWeight, down: TernaryBlockELLWeight):
        super().__init__()
        self.w_gate, self.w_up, self.w_down = gate, up, down
        self._prepared = None

    def prepared(self):
        """The cached prepared weights, rebuilt when any weight buffer's version changes."""
        bufs = [t for w in (self.w_gate, self.w_up, self.w_down) for t in w.triple()]
        key = tuple((t.data_ptr(), t._version) for t in bufs)
        if self._prepared is None or self._prepared[0] != key:
            with torch.inference_mode(False):
                self._prepared = (key, kernels.ternary_prepare(self.w_gate.triple(), self.w_up.triple(),
                                                               self.w_down.triple()))
        return self._prepared[1]

    def release_prepared(self) -> None:
        """Drop the cached prepared weights."""
        self._prepared = None

    @classmethod
    def random(cls, d_model: int, d_ff: int, tile_size: int, density: float, device, seed: int = 0):
        """Latent N(0, 0.02) tiles with random topology, quantised to ternary."""
        g = torch.Generator().manual_seed(seed)
        B = tile_size

        def make(out_f, in_f):
            R, C = out_f // B, in_f // B
            K = max(1, int(C * density))
            vals = (torch.randn(R, K, B, B, generator=g) * 0.02).to(device=device, dtype=torch.bfloat16)
            cols = create_random_topology(R, C, K, g).to(device)
            return TernaryBlockELLWeight.from_latent(vals, cols)

        return cls(make(d_ff, d_model), make(d_ff, d_model), make(d_model, d_ff))

    def forward(self, x: torch.Tensor, add_residual: bool = False) -> torch.Tensor:
        lead, d = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, d).to(torch.bfloat16).contiguous()
        xq, sx = kernels.quantize_act_int8(x2)
        out = kernels.ternary_swiglu_fwd_prepared(xq, sx, self.prepared(), self.w_gate.triple(), self.w_up.triple(),
                                                  self.w_down.triple(), x2 if add_residual else None)
        return out.reshape(*lead, d)
