"""Block-ELL sparse tensor format (PyTorch), mirroring the reference's JAX module.

Reference: ``looped_blockell/layers/block_ell.py``.

Block-ELL stores a sparse weight as
  values:      [R, K, B, B]  dense tiles, tile values[r, k] is [B_in, B_out]
  col_indices: [R, K] int32  input column block of each tile (-1 = dead slot)
Layout convention: the weight is [out_features, in_features] = [R*B, C*B].

``block_ell_matmul`` and the dense conversions run on the GPU through the HIP kernels
(``titan::block_ell_matmul``, ``lbk_block_ell_topk_columns``, ``lbk_dense_to_block_ell``,
``lbk_block_ell_to_dense``); ``create_random_topology`` is torch RNG code usable on any device.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import kernels


@dataclass
class BlockELLConfig:
    """Geometry (reference ``block_ell.py:19-50``)."""

    R: int
    C: int
    K: int
    B: int = 16

    def __post_init__(self) -> None:
        if self.K > self.C:
            raise ValueError(f"K ({self.K}) cannot exceed C ({self.C})")
        if any(v < 1 for v in (self.R, self.C, self.K, self.B)):
            raise ValueError("R, C, K, B must all be >= 1")

    @property
    def out_features(self) -> int:
        return self.R * self.B

    @property
    def in_features(self) -> int:
        return self.C * self.B

    @property
    def total_blocks(self) -> int:
        return self.R * self.K

    @property
    def total_parameters(self) -> int:
        return self.R * self.K * self.B * self.B

    @property
    def density(self) -> float:
        return self.K / self.C


@dataclass
class BlockELLTensor:
    """values [R, K, B, B] + col_indices [R, K] (reference ``block_ell.py:53-66``)."""

    values: torch.Tensor
    col_indices: torch.Tensor
    config: BlockELLConfig

    def __post_init__(self) -> None:
        cfg = self.config
        ev = (cfg.R, cfg.K, cfg.B, cfg.B)
        ei = (cfg.R, cfg.K)
        if tuple(self.values.shape) != ev:
            raise ValueError(f"values shape {tuple(self.values.shape)} != expected {ev}")
        if tuple(self.col_indices.shape) != ei:
            raise ValueError(f"col_indices shape {tuple(self.col_indices.shape)} != expected {ei}")


def create_random_topology(R: int, C: int, K: int, generator: torch.Generator | int | None = None,
                           device=None) -> torch.Tensor:
    """K unique, unsorted column blocks per row, int32 [R, K] (reference ``block_ell.py:69-76``).

    ``generator`` may be a ``torch.Generator`` or an integer seed (the
    reference takes a JAX key; the draw is uniform without replacement).
    """
    if K > C:
        raise ValueError(f"K ({K}) cannot exceed C ({C})")
    if isinstance(generator, int):
        generator = torch.Generator().manual_seed(generator)
    keys = torch.rand(R, C, generator=generator)
    cols = torch.argsort(keys, dim=1)[:, :K].to(torch.int32)
    return cols.to(device) if device is not None else cols


def create_block_ell_from_dense(dense: torch.Tensor, tile_size: int = 16, density: float = 0.5) -> BlockELLTensor:
    """Dense [out, in] -> Block-ELL keeping the top-K tiles per row by Frobenius norm.

    Reference ``block_ell.py:79-115``: ``K = max(1, int(C * density))``, indices sorted.
    """
    from ..interop import gather_tiles, topk_columns
    out_f, in_f = dense.shape
    B = tile_size
    if out_f % B or in_f % B:
        raise ValueError(f"Dimensions ({out_f}, {in_f}) must be divisible by tile_size {B}")
    R, C = out_f // B, in_f // B
    K = max(1, int(C * density))
    cols = topk_columns(dense, B, K)                                   # ascending, ties to the smaller column
    values = gather_tiles(dense, cols, B)                              # [R, K, B_in, B_out]
    return BlockELLTensor(values=values, col_indices=cols, config=BlockELLConfig(R=R, C=C, K=K, B=B))


def block_ell_to_dense(block_ell: BlockELLTensor) -> torch.Tensor:
    """Scatter to dense [out, in]; each [B_in, B_out] tile lands transposed (reference
    ``block_ell.py:118-146``; the last slot naming a column wins, ``-1`` slots write nothing)."""
    from ..interop import block_ell_to_dense as _to_dense
    cfg = block_ell.config
    return _to_dense(block_ell.values, block_ell.col_indices, cfg.out_features, cfg.in_features)


def block_ell_matmul(x: torch.Tensor, block_ell: BlockELLTensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., in_features] -> [..., out_features] on the GPU (reference ``block_ell.py:149-182``).

    Computes ``y[.., r*B+D] = sum_k sum_d x[.., col[r,k]*B+d] * values[r,k,d,D]``
    with bf16 inputs and fp32 accumulation; dead slots (col = -1) are skipped.
    """
    cfg = block_ell.config
    if x.shape[-1] != cfg.in_features:
        raise ValueError(f"x has {x.shape[-1]} features, weight expects {cfg.in_features}")
    return kernels.block_ell_matmul(x, block_ell.values.to(torch.bfloat16), block_ell.col_indices.to(torch.int32),
                                    bias)
