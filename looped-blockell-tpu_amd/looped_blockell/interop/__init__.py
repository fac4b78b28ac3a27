"""Storage formats: the dense <-> Block-ELL checkpoint bridge and the packed ternary file.

Dense bridge (reference ``interop/convert_checkpoint.py:114-148``; tiles are ``[B_in, B_out]``,
dense weights ``[out, in]`` as in ``nn.Linear``), on GPU tensors through the HIP kernels:

* ``dense_to_block_ell(weight, tile_size)`` -> ``(values [R, C, B, B], col_indices [R, C])`` —
  density 1, sequential columns, as the reference's ``_dense_to_block_ell``;
* ``block_ell_to_dense(values, col_indices, out_features, in_features)`` — the reference's
  ``_block_ell_to_dense`` (later slots overwrite earlier ones; ``-1`` slots write nothing);
* ``gather_tiles(dense, col_indices, tile_size)`` — tiles of any topology (zero tile for a
  sentinel);
* ``topk_columns(dense, tile_size, K)`` — per block row the K columns of largest Frobenius
  norm, ascending (the selection of ``create_block_ell_from_dense``);
* ``load_dense_state_dict(module, state_dict)`` / ``dense_state_dict(module)`` — every
  ``BlockELLLinear`` of a module from / to ``<name>.weight`` + ``<name>.bias`` entries of a
  PyTorch dense checkpoint (tiles gathered at the module's current topology).

Ternary file (this library's own format; the reference has no packed ternary storage):
``save_ternary`` / ``load_ternary``, see ``ternary_file``.

Copies move bits: bf16, fp16 and fp32 weights keep their dtype; the norms of ``topk_columns``
read bf16 or fp32.
"""

from __future__ import annotations

import ctypes as C

import torch

from .. import abi as A
from .ternary_file import TERNARY_FORMAT, TERNARY_VERSION, check_ternary_codes, load_ternary, save_ternary

__all__ = ["dense_to_block_ell", "block_ell_to_dense", "gather_tiles", "topk_columns", "load_dense_state_dict",
           "dense_state_dict", "save_ternary", "load_ternary", "check_ternary_codes", "TERNARY_FORMAT",
           "TERNARY_VERSION"]


def _lib():
    return A.load()


def _p(t):
    return C.c_void_p(t.data_ptr())


def _stream(t):
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _gpu(*ts):
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("looped_blockell.interop converts GPU tensors only; got a CPU tensor "
                               "(load the checkpoint with map_location='cuda')")


def _elem(t: torch.Tensor) -> int:
    n = t.element_size()
    if n not in (2, 4) or t.is_complex():
        raise TypeError(f"unsupported weight dtype {t.dtype} (2- or 4-byte elements)")
    return n


def gather_tiles(dense: torch.Tensor, col_indices: torch.Tensor, tile_size: int = 16) -> torch.Tensor:
    """values[r, k] = dense block (r, col_indices[r, k]) as ``[B_in, B_out]``; zero tile where the
    column is outside [0, C)."""
    _gpu(dense, col_indices)
    B = tile_size
    out_f, in_f = dense.shape
    if out_f % B or in_f % B:
        raise ValueError(f"Dimensions ({out_f}, {in_f}) must be divisible by tile_size {B}")
    R, Cb = out_f // B, in_f // B
    if col_indices.shape[0] != R:
        raise ValueError(f"col_indices has {col_indices.shape[0]} rows, the weight {R} block rows")
    K = col_indices.shape[1]
    d = dense.contiguous()
    c = col_indices.to(torch.int32).contiguous()
    values = torch.empty(R, K, B, B, dtype=d.dtype, device=d.device)
    A.check(_lib().lbk_dense_to_block_ell(_p(d), in_f, _elem(d), R, Cb, B, _p(c), K, _p(values), _stream(d)),
            "dense_to_block_ell")
    return values


def dense_to_block_ell(weight: torch.Tensor, tile_size: int = 16):
    """Reference ``convert_checkpoint.py:114-131``: density 1, ``col_indices[r] = 0..C-1``."""
    _gpu(weight)
    B = tile_size
    R, Cb = weight.shape[0] // B, weight.shape[1] // B
    cols = torch.arange(Cb, dtype=torch.int32, device=weight.device).repeat(R, 1).contiguous()
    return gather_tiles(weight, cols, B), cols


def block_ell_to_dense(values: torch.Tensor, col_indices: torch.Tensor, out_features: int, in_features: int,
                       tile_size: int | None = None) -> torch.Tensor:
    """Reference ``convert_checkpoint.py:134-148``: dense ``[out, in]``, tile ``[B_in, B_out]``
    transposed into block (r, col); for a column that several slots of a row name, the last
    slot wins; ``-1`` slots write nothing."""
    _gpu(values, col_indices)
    R, K, B, B2 = values.shape
    if B != B2 or (tile_size is not None and tile_size != B):
        raise ValueError(f"values tiles are {B}x{B2}, tile_size {tile_size}")
    if out_features != R * B or in_features % B:
        raise ValueError(f"({out_features}, {in_features}) does not match {R} block rows of {B}")
    if tuple(col_indices.shape) != (R, K):
        raise ValueError(f"col_indices shape {tuple(col_indices.shape)} != {(R, K)}")
    v = values.contiguous()
    c = col_indices.to(torch.int32).contiguous()
    dense = torch.empty(out_features, in_features, dtype=v.dtype, device=v.device)
    A.check(_lib().lbk_block_ell_to_dense(_p(v), _p(c), R, K, B, in_features // B, _elem(v), _p(dense), in_features,
                                          _stream(v)), "block_ell_to_dense")
    return dense


def topk_columns(dense: torch.Tensor, tile_size: int, K: int) -> torch.Tensor:
    """Per block row, the K columns with the largest block Frobenius norm (fp32; ties to the
    smaller column), ascending — the selection of the reference's
    ``create_block_ell_from_dense`` (``looped_blockell/layers/block_ell.py:100-106``)."""
    _gpu(dense)
    if dense.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("topk_columns reads bf16 or fp32 weights")
    B = tile_size
    out_f, in_f = dense.shape
    R, Cb = out_f // B, in_f // B
    d = dense.contiguous()
    cols = torch.empty(R, K, dtype=torch.int32, device=d.device)
    A.check(_lib().lbk_block_ell_topk_columns(_p(d), in_f, _elem(d), R, Cb, B, K, _p(cols), _stream(d)),
            "topk_columns")
    return cols


def _block_ell_linears(module):
    from ..layers.mlp import BlockELLLinear
    return [(n, m) for n, m in module.named_modules() if isinstance(m, BlockELLLinear)]


@torch.no_grad()
def load_dense_state_dict(module: torch.nn.Module, state_dict: dict) -> list[str]:
    """Fill every ``BlockELLLinear`` of ``module`` from a dense PyTorch checkpoint: its tiles are
    gathered from ``<name>.weight`` ``[out, in]`` at the layer's current topology (at density 1
    that is the whole matrix, the reference's conversion) and its bias from ``<name>.bias``.
    Returns the names converted; other entries are left to ``module.load_state_dict``."""
    done = []
    for name, lin in _block_ell_linears(module):
        key = f"{name}.weight" if name else "weight"
        if key not in state_dict:
            continue
        w = state_dict[key].to(device=lin.values.device)
        if tuple(w.shape) != (lin.out_features, lin.in_features):
            raise ValueError(f"{key}: shape {tuple(w.shape)} != {(lin.out_features, lin.in_features)}")
        tiles = gather_tiles(w.to(lin.values.dtype), lin.col_indices, lin.tile_size)
        lin.values.copy_(tiles)
        bkey = f"{name}.bias" if name else "bias"
        if lin.bias is not None and bkey in state_dict:
            lin.bias.copy_(state_dict[bkey].to(lin.bias.device, lin.bias.dtype))
        done.append(name)
    return done


@torch.no_grad()
def dense_state_dict(module: torch.nn.Module) -> dict:
    """``<name>.weight`` (dense ``[out, in]``, dead tiles zero) and ``<name>.bias`` for every
    ``BlockELLLinear`` of ``module`` — what a dense PyTorch model loads."""
    out = {}
    for name, lin in _block_ell_linears(module):
        pre = f"{name}." if name else ""
        out[pre + "weight"] = block_ell_to_dense(lin.values.detach(), lin.effective_col_indices(), lin.out_features,
                                                 lin.in_features)
        if lin.bias is not None:
            out[pre + "bias"] = lin.bias.detach().clone()
    return out
