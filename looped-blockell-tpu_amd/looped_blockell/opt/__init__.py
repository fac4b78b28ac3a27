"""Prune-time topology transforms on the GPU (torch tensors, HIP kernels through the C ABI).

Mirrors the functions of the reference's ``looped_blockell/opt/compaction.py`` and
``looped_blockell/opt/column_reorder.py`` with their names and argument meaning:

* ``compact_single_layer(values, col_indices, alive_mask)`` -> ``(values, col_indices,
  alive_mask, K_new)`` — alive tiles packed to the front of each row, K shrunk to the largest
  alive count (at least 1).
* ``compute_column_importance(fc1_alive_mask, fc2_alive_mask, fc1_col_indices,
  fc2_col_indices, C_ff)`` -> float32 ``[C_ff]``.
* ``compute_permutation(importance)`` -> int32 ``[C_ff]`` (stable descending order).
* ``apply_permutation_to_block_ell(values, col_indices, alive_mask, perm, is_column_dim)``.
* ``apply_permutation_to_optimizer(opt_state, perm, param_name, is_column_dim)`` — row mode
  gathers every tensor leaf whose first dimension is C_ff (Adam moments of the d_ff-row weight).
* ``compute_k_active_macros(alive_mask, col_indices, tiles_per_macro, C_ff)`` -> int32 scalar.
* ``full_reorder_step(...)`` — the six steps above in the reference's order.
* ``transposed_index(col_indices, C)`` -> ``(col_ptr [C+1], entries)``: the column-major view
  of a topology (no reference counterpart; what a transposed product walks).

"fc1" is the weight whose column indices address d_ff (here the down projection, rows =
d_model blocks); "fc2" is the weight with one block row per d_ff column (gate and up).

Every function runs on device (bf16 values, int32 indices, bool masks) and, like the rest of
the package, refuses CPU tensors.  ``compact_single_layer`` reads K_new back to the host, as
the reference does with ``int(...)``.
"""

from __future__ import annotations

import ctypes as C

import torch

from .. import abi as A

__all__ = ["compact_single_layer", "compute_column_importance", "compute_permutation",
           "apply_permutation_to_block_ell", "apply_permutation_to_optimizer", "compute_k_active_macros",
           "full_reorder_step", "transposed_index"]


def _lib():
    return A.load()


def _p(t):
    return C.c_void_p(t.data_ptr())


def _stream(t):
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _gpu(*ts):
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("looped_blockell.opt runs on the GPU only; got a CPU tensor")


def _mask(m):
    # a bool tensor is one byte per element holding 0 or 1: reinterpret it, no conversion kernel
    m = m.contiguous()
    return (m if m.dtype == torch.bool else m != 0).view(torch.uint8)


def _same(what, *shapes):
    if any(tuple(s) != tuple(shapes[0]) for s in shapes[1:]):
        raise ValueError(f"{what}: shapes differ: {[tuple(s) for s in shapes]}")


def compact_single_layer(values: torch.Tensor, col_indices: torch.Tensor, alive_mask: torch.Tensor):
    """Reference ``compaction.py:31-60``: alive tiles first, then truncate to K_new."""
    _gpu(values, col_indices, alive_mask)
    _same("compact_single_layer", values.shape[:2], col_indices.shape, alive_mask.shape)
    R, K, B, _ = values.shape
    v = values.to(torch.bfloat16).contiguous()
    c = col_indices.to(torch.int32).contiguous()
    a = _mask(alive_mask)
    counts = torch.empty(R, dtype=torch.int32, device=v.device)
    mx = torch.empty(1, dtype=torch.int32, device=v.device)
    A.check(_lib().lbk_topology_alive_counts(_p(a), R, K, _p(counts), _p(mx), _stream(v)), "alive_counts")
    K_new = max(int(mx.item()), 1)
    ov = torch.empty(R, K_new, B, B, dtype=torch.bfloat16, device=v.device)
    oc = torch.empty(R, K_new, dtype=torch.int32, device=v.device)
    oa = torch.empty(R, K_new, dtype=torch.uint8, device=v.device)
    A.check(_lib().lbk_topology_compact_bf16(_p(v), _p(c), _p(a), R, K, B, K_new, _p(ov), _p(oc), _p(oa),
                                              _stream(v)), "compact")
    return ov, oc, oa.view(torch.bool), K_new


def compute_column_importance(fc1_alive_mask: torch.Tensor, fc2_alive_mask: torch.Tensor,
                              fc1_col_indices: torch.Tensor, fc2_col_indices: torch.Tensor,
                              C_ff: int) -> torch.Tensor:
    """Reference ``column_reorder.py:33-98`` (``fc2_col_indices`` is not used for scoring)."""
    _gpu(fc1_alive_mask, fc2_alive_mask, fc1_col_indices)
    _same("compute_column_importance", fc1_alive_mask.shape, fc1_col_indices.shape)
    if fc2_alive_mask.dim() != 2:
        raise ValueError("compute_column_importance: fc2_alive_mask must be [R, K]")
    R1, K1 = fc1_col_indices.shape
    R2, K2 = fc2_alive_mask.shape
    c1 = fc1_col_indices.to(torch.int32).contiguous()
    a1, a2 = _mask(fc1_alive_mask), _mask(fc2_alive_mask)
    imp = torch.empty(C_ff, dtype=torch.float32, device=c1.device)
    A.check(_lib().lbk_column_importance(_p(c1), _p(a1), R1, K1, _p(a2), R2, K2, C_ff, _p(imp), _stream(c1)),
            "column_importance")
    return imp


def compute_permutation(importance: torch.Tensor) -> torch.Tensor:
    """Reference ``column_reorder.py:103-114``: ``argsort(-importance)`` as int32."""
    _gpu(importance)
    if importance.dim() != 1:
        raise ValueError("compute_permutation: importance must be one-dimensional")
    imp = importance.to(torch.float32).contiguous()
    perm = torch.empty(imp.shape[0], dtype=torch.int32, device=imp.device)
    A.check(_lib().lbk_column_permutation(_p(imp), imp.shape[0], _p(perm), _stream(imp)), "column_permutation")
    return perm


def apply_permutation_to_block_ell(values: torch.Tensor, col_indices: torch.Tensor, alive_mask: torch.Tensor,
                                   perm: torch.Tensor, is_column_dim: bool = True):
    """Reference ``column_reorder.py:121-177``.  Column mode returns ``values`` and
    ``alive_mask`` themselves (the tiles keep their slots) with remapped column indices; row
    mode returns gathered copies of all three."""
    _gpu(values, col_indices, alive_mask, perm)
    _same("apply_permutation_to_block_ell", values.shape[:2], col_indices.shape, alive_mask.shape)
    if perm.dim() != 1:
        raise ValueError("apply_permutation_to_block_ell: perm must be one-dimensional")
    R, K, B, _ = values.shape
    c = col_indices.to(torch.int32).contiguous()
    p = perm.to(torch.int32).contiguous()
    oc = torch.empty_like(c)
    if is_column_dim:
        nul = C.c_void_p(0)
        A.check(_lib().lbk_apply_permutation_bf16(nul, _p(c), nul, R, K, B, _p(p), p.shape[0], 1, nul, _p(oc), nul,
                                                  _stream(c)), "apply_permutation")
        return values, oc, alive_mask
    v = values.to(torch.bfloat16).contiguous()
    a = _mask(alive_mask)
    ov, oa = torch.empty_like(v), torch.empty_like(a)
    A.check(_lib().lbk_apply_permutation_bf16(_p(v), _p(c), _p(a), R, K, B, _p(p), p.shape[0], 0, _p(ov), _p(oc),
                                              _p(oa), _stream(v)), "apply_permutation")
    return ov, oc, oa.view(torch.bool)


def _gather_rows(t: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    src = t.contiguous()
    out = torch.empty_like(src)
    row_bytes = src.numel() // max(src.shape[0], 1) * src.element_size()
    A.check(_lib().lbk_gather_rows(_p(src), src.shape[0], row_bytes, _p(perm), src.shape[0], _p(out),
                                   _stream(src)), "gather_rows")
    return out


def apply_permutation_to_optimizer(opt_state, perm: torch.Tensor, param_name: str = "",
                                   is_column_dim: bool = True):
    """Reference ``column_reorder.py:179-236`` for a torch optimizer state (for instance
    ``optimizer.state[param]``, or any nested dict / list / tuple of tensors): in row mode every
    GPU tensor leaf whose first dimension is C_ff = len(perm) has its rows gathered; column
    mode and all other leaves are returned unchanged (the column-dim weight only renames its
    tile columns, so its moments stay in their slots).  ``param_name`` is accepted for the same
    signature; as in the reference, leaves are matched by shape."""
    _gpu(perm)
    p = perm.to(torch.int32).contiguous()
    C_ff = p.shape[0]

    def leaf(x):
        if isinstance(x, dict):
            return {k: leaf(v) for k, v in x.items()}
        if isinstance(x, (list, tuple)):
            return type(x)(leaf(v) for v in x)
        if torch.is_tensor(x) and not is_column_dim and x.dim() >= 1 and x.shape[0] == C_ff:
            _gpu(x)
            return _gather_rows(x, p)
        return x

    return leaf(opt_state)


def compute_k_active_macros(alive_mask: torch.Tensor, col_indices: torch.Tensor, tiles_per_macro: int,
                            C_ff: int) -> torch.Tensor:
    """Reference ``column_reorder.py:233-269``; ``C_ff`` is accepted for the same signature."""
    _gpu(alive_mask, col_indices)
    _same("compute_k_active_macros", alive_mask.shape, col_indices.shape)
    R, K = col_indices.shape
    c = col_indices.to(torch.int32).contiguous()
    a = _mask(alive_mask)
    out = torch.empty((), dtype=torch.int32, device=c.device)
    A.check(_lib().lbk_k_active_macros(_p(c), _p(a), R, K, tiles_per_macro, _p(out), _stream(c)), "k_active_macros")
    return out


def full_reorder_step(fc1_values, fc1_col_indices, fc1_alive, fc2_values, fc2_col_indices, fc2_alive, opt_state,
                      C_ff: int, tiles_per_macro: int):
    """Reference ``column_reorder.py:279-360``: importance, permutation, fc1 column remap, fc2
    row gather, optimizer rows, active macro-blocks.  Returns ``(fc1_values, fc1_cols,
    fc1_alive, fc2_values, fc2_cols, fc2_alive, opt_state, k_active)``."""
    imp = compute_column_importance(fc1_alive, fc2_alive, fc1_col_indices, fc2_col_indices, C_ff)
    perm = compute_permutation(imp)
    v1, c1, a1 = apply_permutation_to_block_ell(fc1_values, fc1_col_indices, fc1_alive, perm, is_column_dim=True)
    v2, c2, a2 = apply_permutation_to_block_ell(fc2_values, fc2_col_indices, fc2_alive, perm, is_column_dim=False)
    st = apply_permutation_to_optimizer(opt_state, perm, param_name="fc2_values", is_column_dim=False)
    k_active = compute_k_active_macros(a1, c1, tiles_per_macro, C_ff)
    return v1, c1, a1, v2, c2, a2, st, k_active


def transposed_index(col_indices: torch.Tensor, C: int):
    """Column-major view of a topology: ``col_ptr`` int32 [C+1] and ``entries`` int32 [nnz],
    where ``entries[col_ptr[c]:col_ptr[c+1]]`` are the slots ``r*K + k`` with column c in
    ascending order (sentinels and columns >= C left out).  Reads nnz back to the host."""
    _gpu(col_indices)
    R, K = col_indices.shape
    c = col_indices.to(torch.int32).contiguous()
    col_ptr = torch.empty(C + 1, dtype=torch.int32, device=c.device)
    entries = torch.empty(max(R * K, 1), dtype=torch.int32, device=c.device)
    A.check(_lib().lbk_transposed_index(_p(c), R, K, C, _p(col_ptr), _p(entries), _stream(c)), "transposed_index")
    return col_ptr, entries[: int(col_ptr[C].item())]
