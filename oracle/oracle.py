"""CPU oracle for the Block-ELL SwiGLU FFN path — TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of the reference's Block-ELL
SwiGLU forward so that the HIP kernels can be checked against it.  It is the
checker, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The shipped path
(``looped_blockell``) never imports, calls or falls back to anything here.

Every function cites the reference file:line it restates.  How each function is
pinned (closed forms, invariants from the reference's own tests, brute force on
tiny inputs) is listed in ``PINS`` at the bottom of this file; the tests in
``tests/test_oracle.py`` enforce each pin.

Layout conventions (reference ``looped_blockell/layers/block_ell.py:1-8``):
  values      [R, K, B, B]  tile values[r, k] is [B_in, B_out]
  col_indices [R, K] int32  input column-block of each tile; -1 marks a dead
                            slot that contributes nothing
                            (``looped_blockell/opt/cms.py:229-230``)
  weight      [out, in] = [R*B, C*B]
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

__all__ = [
    "BlockELLConfig", "k_for_density", "random_topology", "dense_to_block_ell",
    "permute_optimizer_rows", "transposed_index",
    "block_ell_to_dense", "create_block_ell_from_dense", "block_ell_matmul",
    "silu", "swiglu_fwd", "gelu_tanh", "gelu_mlp_fwd", "rmsnorm", "rmsnorm_bwd", "looped_swiglu",
    "diagonal_injection", "diagonal_injection_bwd",
    "block_ell_matmul_t", "swiglu_bias_grads",
    "block_ell_weight_grad", "swiglu_bwd", "alive_slots", "compact_topology", "column_importance",
    "column_permutation", "apply_permutation", "k_active_macros", "ternary_quantize_blocks",
    "activation_quantize_int8", "encode_ternary", "pack_ternary",
    "unpack_ternary", "ternary_block_partials", "ternary_fixed_point",
    "ternary_matmul", "ternary_swiglu_fwd", "bf16_round",
]


# --------------------------------------------------------------------------
# format
# --------------------------------------------------------------------------

@dataclass
class BlockELLConfig:
    """Geometry of one Block-ELL weight (``looped_blockell/layers/block_ell.py:19-50``)."""

    R: int
    C: int
    K: int
    B: int = 16

    def __post_init__(self) -> None:
        # block_ell.py:26-30
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
    def density(self) -> float:
        return self.K / self.C


def k_for_density(C: int, density: float) -> int:
    """``K = max(1, int(C * density))`` (``looped_blockell/layers/mlp.py:44``)."""
    return max(1, int(C * density))


def random_topology(R: int, C: int, K: int, rng: np.random.Generator) -> np.ndarray:
    """K distinct, unsorted column blocks per row (``block_ell.py:69-76``).

    The reference draws with ``jax.random.choice(replace=False)``; the stream is
    JAX's, so this restatement keeps only the contract (distinct, unsorted,
    uniform) and uses numpy's generator.
    """
    out = np.empty((R, K), dtype=np.int32)
    for r in range(R):
        out[r] = rng.choice(C, size=K, replace=False)
    return out


def dense_to_block_ell(weight: np.ndarray, tile_size: int = 16):
    """Dense [out, in] -> (values [R, C, B_in, B_out], sequential col_indices).

    Restates ``interop/convert_checkpoint.py:114-131`` (density 1.0).
    """
    out_f, in_f = weight.shape
    B = tile_size
    R, C = out_f // B, in_f // B
    blocks = weight.reshape(R, B, C, B).transpose(0, 2, 3, 1)
    col = np.tile(np.arange(C, dtype=np.int32), (R, 1))
    return np.ascontiguousarray(blocks), col


def block_ell_to_dense(values: np.ndarray, col_indices: np.ndarray, out_features: int,
                       in_features: int) -> np.ndarray:
    """Scatter Block-ELL to dense [out, in]; tile [B_in, B_out] lands transposed.

    Restates ``interop/convert_checkpoint.py:134-148`` and
    ``looped_blockell/layers/block_ell.py:118-146``.  Dead slots (col < 0) are
    skipped.
    """
    R, K, B, _ = values.shape
    dense = np.zeros((out_features, in_features), dtype=values.dtype)
    for r in range(R):
        for k in range(K):
            c = int(col_indices[r, k])
            if c < 0:
                continue
            dense[r * B:(r + 1) * B, c * B:(c + 1) * B] = values[r, k].T
    return dense


def create_block_ell_from_dense(dense: np.ndarray, tile_size: int = 16, density: float = 0.5):
    """Top-K tiles per row by Frobenius norm, sorted indices.

    Restates ``looped_blockell/layers/block_ell.py:79-115``.
    """
    out_f, in_f = dense.shape
    B = tile_size
    if out_f % B or in_f % B:
        raise ValueError(f"Dimensions ({out_f}, {in_f}) must be divisible by tile_size {B}")
    R, C = out_f // B, in_f // B
    K = k_for_density(C, density)
    blocks = dense.reshape(R, B, C, B).transpose(0, 2, 3, 1)       # [R, C, B_in, B_out]
    norms = np.sqrt(np.sum(blocks.astype(np.float64) ** 2, axis=(2, 3)))
    top = np.argsort(-norms, axis=1, kind="stable")[:, :K]
    col = np.sort(top, axis=1).astype(np.int32)
    values = np.take_along_axis(blocks, col[:, :, None, None], axis=1)
    return np.ascontiguousarray(values), col, BlockELLConfig(R=R, C=C, K=K, B=B)


# --------------------------------------------------------------------------
# block-sparse matmul and the SwiGLU FFN
# --------------------------------------------------------------------------

def block_ell_matmul(x: np.ndarray, values: np.ndarray, col_indices: np.ndarray,
                     chunk: int = 1024) -> np.ndarray:
    """``y[n, r*B+D] = sum_k sum_d x[n, col[r,k]*B+d] * values[r,k,d,D]``.

    Restates ``looped_blockell/layers/block_ell.py:149-182``: tile the input
    into [.., C, B], gather the K column tiles of every block row, contract over
    (k, d).  The contraction runs as R batched [n, K*B] x [K*B, B] products in
    the dtype of the inputs.  Dead slots (col < 0) contribute zero
    (``looped_blockell/opt/cms.py:229-230``); the JAX layer achieves the same
    by zeroing dead values (``looped_blockell/layers/mlp.py:73-77``).
    Tokens are processed ``chunk`` at a time to bound the gather's memory.
    """
    lead = x.shape[:-1]
    R, K, B, B2 = values.shape
    assert B == B2
    F = x.shape[-1]
    assert F % B == 0, "in_features must be a multiple of B"
    C = F // B
    xf = x.reshape(-1, C, B)
    n = xf.shape[0]
    dtype = np.result_type(x.dtype, values.dtype)
    out = np.zeros((n, R, B), dtype=dtype)
    col = col_indices.astype(np.int64)
    alive = col >= 0
    safe = np.where(alive, col, 0)
    w = np.where(alive[:, :, None, None], values, 0).astype(dtype)          # [R,K,B,B]
    w2 = w.reshape(R, K * B, B)                                             # [R, K*B_in, B_out]
    for s in range(0, n, chunk):
        xs = xf[s:s + chunk].astype(dtype)                                  # [n, C, B]
        g = xs[:, safe.reshape(-1), :].reshape(xs.shape[0], R, K * B)       # [n, R, K*B]
        out[s:s + chunk] = np.matmul(g.transpose(1, 0, 2), w2).transpose(1, 0, 2)
    return out.reshape(*lead, R * B)


def silu(z: np.ndarray) -> np.ndarray:
    """``silu(z) = z * sigmoid(z)`` (``looped_blockell/layers/mlp.py:137``, jax.nn.silu)."""
    z = np.asarray(z)
    return z / (1.0 + np.exp(-z))


def swiglu_fwd(x, gate, up, down, add_residual: bool = False, h_round=None, biases=None):
    """``out = W_down(silu(W_gate x + b_g) * (W_up x + b_u)) + b_d (+ x)``.

    Restates ``looped_blockell/layers/mlp.py:119-145`` (SwiGLU branch, whose three
    ``BlockELLLinear`` projections each add a bias, ``:56-60``, ``:82``) and the
    reference operator's optional residual epilogue
    (``csrc/block_ell/swiglu_fwd.cuh:60-84``).  ``gate``/``up``/``down`` are
    ``(values, col_indices)`` pairs; ``biases`` is ``None`` or ``(b_g, b_u, b_d)`` with
    ``None`` entries for absent biases.  ``h_round`` optionally rounds the hidden
    state (e.g. to bf16) before the down projection.
    Returns ``(out, h, gate_pre_act, up_output)``.
    """
    bg, bu, bd = biases if biases is not None else (None, None, None)
    g = block_ell_matmul(x, *gate)
    u = block_ell_matmul(x, *up)
    if bg is not None:
        g = g + bg
    if bu is not None:
        u = u + bu
    h = silu(g) * u
    if h_round is not None:
        h = h_round(h)
    out = block_ell_matmul(h, *down)
    if bd is not None:
        out = out + bd
    if add_residual:
        out = out + x
    return out, h, g, u


def gelu_tanh(z: np.ndarray) -> np.ndarray:
    """``jax.nn.gelu`` with its default ``approximate=True`` (the GELU MLP of
    ``looped_blockell/layers/mlp.py:156``):
    ``0.5 z (1 + tanh(sqrt(2/pi) (z + 0.044715 z^3)))``."""
    z = np.asarray(z)
    return 0.5 * z * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (z + 0.044715 * z ** 3)))


def gelu_mlp_fwd(x, fc1, fc2, b1=None, b2=None):
    """The GELU branch of ``MLPBlock`` (``looped_blockell/layers/mlp.py:146-164``):
    ``fc2(gelu_tanh(fc1(x) + b1)) + b2``; ``fc1``/``fc2`` are ``(values, col_indices)``."""
    a = block_ell_matmul(x, *fc1)
    if b1 is not None:
        a = a + b1
    y = block_ell_matmul(gelu_tanh(a), *fc2)
    if b2 is not None:
        y = y + b2
    return y


def rmsnorm(x: np.ndarray, scale: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """``x / sqrt(mean(x^2) + eps) * scale`` (``looped_blockell/layers/norms.py:14-15``)."""
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * scale


def rmsnorm_bwd(x: np.ndarray, scale: np.ndarray, dy: np.ndarray, eps: float = 1e-5):
    """Gradients of :func:`rmsnorm` for an output gradient ``dy`` (the chain rule of
    ``looped_blockell/layers/norms.py:14-15``, which the reference differentiates with JAX):
    ``dx = rs * scale * dy - x * rs^3 * mean(scale * dy * x)``, ``dscale = sum_rows dy * x * rs``
    with ``rs = 1 / sqrt(mean(x^2) + eps)``.  Returns ``(dx, dscale)``."""
    x = np.asarray(x, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    scale = np.asarray(scale, dtype=np.float64)
    rs = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    dot = np.mean(scale * dy * x, axis=-1, keepdims=True)
    dx = rs * scale * dy - x * rs ** 3 * dot
    dscale = np.sum((dy * x * rs).reshape(-1, x.shape[-1]), axis=0)
    return dx, dscale


def diagonal_injection(h, e, log_A, log_dt):
    """``decay * h + dt * e`` with ``dt = softplus(log_dt)``, ``decay = exp(-dt * exp(log_A))``
    per feature (``interop/pt_model.py:923-935``, ``DiagonalInjection.forward``)."""
    dt = np.log1p(np.exp(np.asarray(log_dt, dtype=np.float64)))
    decay = np.exp(-dt * np.exp(np.asarray(log_A, dtype=np.float64)))
    return decay * h + dt * e


def diagonal_injection_bwd(h, e, log_A, log_dt, dy):
    """Gradients of :func:`diagonal_injection` for an output gradient ``dy`` (the chain rule of
    ``interop/pt_model.py:931-935``): ``dh = decay * dy``, ``de = dt * dy``,
    ``dlog_A = -sum_n dy * h * decay * dt * A`` and
    ``dlog_dt = sum_n dy * (e - h * decay * A) * sigmoid(log_dt)`` with ``A = exp(log_A)``.
    Returns ``(dh, de, dlog_A, dlog_dt)``."""
    la = np.asarray(log_A, dtype=np.float64)
    ld = np.asarray(log_dt, dtype=np.float64)
    A = np.exp(la)
    dt = np.log1p(np.exp(ld))
    decay = np.exp(-dt * A)
    sig = 1.0 / (1.0 + np.exp(-ld))
    sgh = np.sum(dy * h, axis=0)
    sge = np.sum(dy * e, axis=0)
    return decay * dy, dt * dy, -sgh * decay * dt * A, (sge - sgh * decay * A) * sig


def looped_swiglu(h, norm_scale, gate, up, down, L: int, eps: float = 1e-5, state_round=None, biases=None):
    """L applications of the pre-norm residual FFN block with shared weights.

    ``h <- h + SwiGLU(RMSNorm(h))`` (``looped_blockell/layers/transformer_block.py:84``;
    the MLP part of ``csrc/loop/persistent_core.cu:315-335``), the SwiGLU with the optional
    ``biases`` of :func:`swiglu_fwd`.  ``state_round`` optionally rounds the carried state
    after each iteration (e.g. to bf16).
    """
    for _ in range(L):
        y, *_ = swiglu_fwd(rmsnorm(h, norm_scale, eps), gate, up, down, biases=biases)
        h = h + y
        if state_round is not None:
            h = state_round(h)
    return h


def looped_core(h, e, log_A, log_dt, blocks, L: int, depths=None, seq_len: int = 1, eps: float = 1e-5,
                state_round=None):
    """The looped application of the FFN core: per iteration ``t < L``

    * ``h_agg = h``
    * ``h_new = diagonal_injection(h_agg, e, log_A, log_dt)`` (skipped when ``e`` is None)
    * for each core block ``(norm_scale, gate, up, down, biases)`` in order:
      ``h_new = h_new + SwiGLU(RMSNorm(h_new))``
    * ``h = where(t < depths[n // seq_len], h_new, h_agg)`` per token row ``n``
      (``depths`` None: every row runs all L iterations).

    This is the scan body of ``looped_blockell/looping/looped_model.py:293-331`` (and the
    PyTorch loop ``interop/pt_model.py:1441-1509``) restricted to its FFN path: the injection
    (``:303``), ``n_core`` distinct pre-norm residual blocks (``:310-311``) with the MLP half of
    ``looped_blockell/layers/transformer_block.py:83-84``, and the per-sequence depth freeze
    ``active = step_idx < depths; h = where(active, h_new, h_agg)`` (``:330-331``).  Rows are
    flattened tokens; ``depths`` holds one entry per run of ``seq_len`` consecutive rows (the
    reference's per-sequence depths over ``[B, S]``).  ``state_round`` optionally rounds the
    carried state after each core block.
    """
    h = np.asarray(h, dtype=np.float64)
    N = h.shape[0]
    if depths is not None:
        tok_depth = np.repeat(np.asarray(depths, dtype=np.int64), seq_len)[:N]
        assert tok_depth.shape[0] == N, "depths must cover every row"
    for t in range(L):
        h_agg = h
        h_new = h_agg if e is None else diagonal_injection(h_agg, e, log_A, log_dt)
        for (scale, gate, up, down, biases) in blocks:
            y, *_ = swiglu_fwd(rmsnorm(h_new, scale, eps), gate, up, down, biases=biases)
            h_new = h_new + y
            if state_round is not None:
                h_new = state_round(h_new)
        if depths is None:
            h = h_new
        else:
            h = np.where((t < tok_depth)[:, None], h_new, h_agg)
    return h


# --------------------------------------------------------------------------
# backward of the SwiGLU FFN (derived from the forward's mathematics)
# --------------------------------------------------------------------------

def block_ell_matmul_t(dy: np.ndarray, values: np.ndarray, col_indices: np.ndarray,
                       C: int) -> np.ndarray:
    """Input gradient of ``block_ell_matmul``: ``dx[n, c*B+d] = sum over slots (r, k) with
    col[r,k] = c of sum_D dy[n, r*B+D] * values[r,k,d,D]``, ``C`` input column blocks.

    This is ``dy @ W`` for the dense ``W = block_ell_to_dense(values, col)`` of
    ``looped_blockell/layers/block_ell.py:109-146`` (the gradient of ``x @ W.T``).  Dead
    slots (col < 0 or >= C) contribute nothing (``looped_blockell/opt/cms.py:229-230``).
    """
    R, K, B, _ = values.shape
    lead = dy.shape[:-1]
    yf = dy.reshape(-1, R * B)
    dtype = np.result_type(dy.dtype, values.dtype)
    out = np.zeros((yf.shape[0], C * B), dtype=dtype)
    for r in range(R):
        yr = yf[:, r * B:(r + 1) * B].astype(dtype)
        for k in range(K):
            c = int(col_indices[r, k])
            if 0 <= c < C:
                out[:, c * B:(c + 1) * B] += yr @ values[r, k].astype(dtype).T
    return out.reshape(*lead, C * B)


def block_ell_weight_grad(x: np.ndarray, dy: np.ndarray, col_indices: np.ndarray, B: int) -> np.ndarray:
    """Tile gradients of ``block_ell_matmul``: ``dW[r,k,d,D] = sum_n x[n, col[r,k]*B+d] *
    dy[n, r*B+D]`` (the [B_in, B_out] tile layout of ``looped_blockell/layers/block_ell.py:1-8``);
    dead slots get zero tiles."""
    R, K = col_indices.shape
    xf = x.reshape(-1, x.shape[-1])
    yf = dy.reshape(-1, dy.shape[-1])
    C = xf.shape[1] // B
    dtype = np.result_type(x.dtype, dy.dtype)
    out = np.zeros((R, K, B, B), dtype=dtype)
    for r in range(R):
        yr = yf[:, r * B:(r + 1) * B].astype(dtype)
        for k in range(K):
            c = int(col_indices[r, k])
            if 0 <= c < C:
                out[r, k] = xf[:, c * B:(c + 1) * B].astype(dtype).T @ yr
    return out


def swiglu_bwd(grad_out, x, gate_pre_act, up_output, h, gate, up, down):
    """Backward of ``out = W_down(silu(g) * u) + x`` with ``g = W_gate x``, ``u = W_up x``.

    The operator and its saved inputs are those of the reference's
    ``titan::block_ell_swiglu_bwd`` (``csrc/block_ell/block_ell_ops.cpp:78-97``), and its
    steps follow the reference's launch sequence (``csrc/block_ell/swiglu_bwd.cu:700-834``):
    ``dh = grad_out W_down`` (kernel 1a), ``dW_down = h^T grad_out`` per tile (1b), the
    SiLU*mul backward ``dg = dh * u * silu'(g)``, ``du = dh * silu(g)`` with
    ``silu'(g) = s + g s (1 - s)``, ``s = sigmoid(g)`` (kernel 2, ``:303-340``),
    ``dx = dg W_gate + du W_up`` (3a) plus ``grad_out`` for the residual (3b,
    ``:478``), and ``dW_gate = x^T dg``, ``dW_up = x^T du`` per tile (3c).  The arithmetic is
    the chain rule of the forward, not a copy of those kernels.  ``gate``/``up``/``down`` are
    ``(values, col_indices)`` pairs; returns ``(dx, d_gate_values, d_up_values,
    d_down_values)``.
    """
    dvals, dcol = down
    B = dvals.shape[2]
    d_ff = gate_pre_act.shape[-1]
    d_model = x.shape[-1]
    g = np.asarray(gate_pre_act, dtype=np.float64)
    u = np.asarray(up_output, dtype=np.float64)
    dy = np.asarray(grad_out, dtype=np.float64)
    dh = block_ell_matmul_t(dy, dvals.astype(np.float64), dcol, d_ff // B)
    s = 1.0 / (1.0 + np.exp(-g))
    dg = dh * u * (s + g * s * (1.0 - s))
    du = dh * g * s
    dx = (block_ell_matmul_t(dg, gate[0].astype(np.float64), gate[1], d_model // B)
          + block_ell_matmul_t(du, up[0].astype(np.float64), up[1], d_model // B) + dy)
    xd = np.asarray(x, dtype=np.float64)
    d_gv = block_ell_weight_grad(xd, dg, gate[1], B)
    d_uv = block_ell_weight_grad(xd, du, up[1], B)
    d_dv = block_ell_weight_grad(np.asarray(h, dtype=np.float64), dy, dcol, B)
    return dx, d_gv, d_uv, d_dv


def swiglu_bias_grads(grad_out, gate_pre_act, up_output, down):
    """Bias gradients of the biased SwiGLU of :func:`swiglu_fwd`: the column sums of
    ``dg``, ``du`` (as in :func:`swiglu_bwd`, from the biased pre-activations) and of
    ``grad_out``.  Returns ``(d_b_gate, d_b_up, d_b_down)``."""
    dvals, dcol = down
    B = dvals.shape[2]
    d_ff = gate_pre_act.shape[-1]
    g = np.asarray(gate_pre_act, dtype=np.float64)
    u = np.asarray(up_output, dtype=np.float64)
    dy = np.asarray(grad_out, dtype=np.float64)
    dh = block_ell_matmul_t(dy, dvals.astype(np.float64), dcol, d_ff // B)
    s = 1.0 / (1.0 + np.exp(-g))
    dg = dh * u * (s + g * s * (1.0 - s))
    du = dh * g * s
    return dg.sum(0), du.sum(0), dy.sum(0)


# --------------------------------------------------------------------------
# topology transforms (prune-time compaction and d_ff column reorder)
# --------------------------------------------------------------------------

def alive_slots(col_indices: np.ndarray, alive_mask: np.ndarray, C: int) -> np.ndarray:
    """Slots that hold a tile: alive and a column in [0, C) (the -1 sentinel marks dead slots,
    ``looped_blockell/opt/cms.py:229-230``)."""
    col = np.asarray(col_indices)
    return np.asarray(alive_mask, bool) & (col >= 0) & (col < C)


def compact_topology(values: np.ndarray, col_indices: np.ndarray, alive_mask: np.ndarray):
    """Pack each row's alive tiles to the front, keep K_new = max(1, max alive per row) slots.

    Restates ``looped_blockell/opt/compaction.py:31-60``: a stable sort of each row by
    ``~alive`` (alive slots first, both groups in slot order), then truncation.  Returns
    ``(values[R, K_new, B, B], col[R, K_new], alive[R, K_new], K_new)``.
    """
    alive = np.asarray(alive_mask, bool)
    K_new = max(int(alive.sum(axis=1).max()) if alive.size else 0, 1)
    order = np.argsort(~alive, axis=1, kind="stable")[:, :K_new]
    rows = np.arange(alive.shape[0])[:, None]
    return values[rows, order], col_indices[rows, order], alive[rows, order], K_new


def column_importance(fc1_alive, fc2_alive, fc1_col, C_ff: int) -> np.ndarray:
    """d_ff tile-column importance: alive fc1 tiles whose column index is c (sentinels
    excluded) plus the alive-tile count of fc2 row c (rows padded or truncated to C_ff).
    Restates ``looped_blockell/opt/column_reorder.py:33-98``."""
    imp = np.zeros(C_ff, np.float32)
    cols = np.asarray(fc1_col).reshape(-1)
    al = np.asarray(fc1_alive, bool).reshape(-1)
    ok = cols >= 0
    np.add.at(imp, np.clip(cols[ok], 0, C_ff - 1), al[ok].astype(np.float32))
    rc = np.asarray(fc2_alive, bool).sum(axis=1).astype(np.float32)
    n = min(len(rc), C_ff)
    imp[:n] += rc[:n]
    return imp


def column_permutation(importance: np.ndarray) -> np.ndarray:
    """``argsort(-importance)``, stable (ties keep ascending index), int32
    (``looped_blockell/opt/column_reorder.py:103-114``)."""
    return np.argsort(-np.asarray(importance, np.float32), kind="stable").astype(np.int32)


def apply_permutation(values, col_indices, alive_mask, perm, is_column_dim: bool = True):
    """``looped_blockell/opt/column_reorder.py:121-177``: column mode remaps
    ``col -> inv_perm[col]`` (sentinels stay -1; values and mask unchanged); row mode
    gathers rows ``perm[i]`` of values, col_indices and alive_mask."""
    perm = np.asarray(perm, np.int64)
    if is_column_dim:
        C_ff = perm.shape[0]
        inv = np.zeros(C_ff, np.int32)
        inv[perm] = np.arange(C_ff, dtype=np.int32)
        col = np.asarray(col_indices)
        new = np.where(col < 0, -1, inv[np.clip(col, 0, C_ff - 1)]).astype(np.int32)
        return values, new, alive_mask
    return values[perm], col_indices[perm], alive_mask[perm]


def k_active_macros(alive_mask, col_indices, tiles_per_macro: int) -> int:
    """Macro-block columns needed to cover the largest alive column index
    (``looped_blockell/opt/column_reorder.py:233-269``); 0 when nothing is alive."""
    safe = np.where(np.asarray(alive_mask, bool), np.asarray(col_indices), -1)
    m = int(safe.max()) if safe.size else -1
    return 0 if m < 0 else int(math.ceil((m + 1) / tiles_per_macro))


def permute_optimizer_rows(state, perm, is_column_dim: bool = True):
    """``looped_blockell/opt/column_reorder.py:179-236``: in row mode every array leaf whose
    first dimension is C_ff = len(perm) is gathered ``leaf[perm]``; column mode and other leaves
    are returned unchanged.  ``state`` is a nested dict / list / tuple of arrays."""
    perm = np.asarray(perm, np.int64)

    def leaf(x):
        if isinstance(x, dict):
            return {k: leaf(v) for k, v in x.items()}
        if isinstance(x, (list, tuple)):
            return type(x)(leaf(v) for v in x)
        if isinstance(x, np.ndarray) and not is_column_dim and x.ndim >= 1 and x.shape[0] == perm.shape[0]:
            return x[perm]
        return x

    return leaf(state)


def transposed_index(col_indices, C: int):
    """Column-major (CSC) view of a topology: ``col_ptr[C + 1]`` and the slots ``e = r*K + k``
    of each column block in ascending order, sentinel (-1) and out-of-range slots left out.
    No reference counterpart: the index a transposed product walks (the backward's ``dy W``
    gathers, ``looped_blockell/layers/block_ell.py:149-182`` read column-wise)."""
    col = np.asarray(col_indices).reshape(-1)
    ok = (col >= 0) & (col < C)
    e = np.nonzero(ok)[0]
    order = np.argsort(col[e], kind="stable")
    counts = np.bincount(col[e], minlength=C)[:C]
    col_ptr = np.zeros(C + 1, np.int32)
    col_ptr[1:] = np.cumsum(counts)
    return col_ptr, e[order].astype(np.int32)


# --------------------------------------------------------------------------
# ternary path (weights {-1,0,+1} with one scale per block, int8 activations)
# --------------------------------------------------------------------------

def ternary_quantize_blocks(w: np.ndarray):
    """Per-block absmean ternary quantisation of values [R, K, B, B].

    Restates ``bonsai-test/bitlinear.py:34-55`` with the group = one B x B block:
    ``s = max(mean|w|, 1e-8)``, ``t = clamp(round(w / s), -1, 1)``, computed in
    float32.  Returns ``(t int8 [R,K,B,B], s float32 [R,K])``.
    """
    w = np.asarray(w, dtype=np.float32)
    R, K, B, _ = w.shape
    flat = w.reshape(R * K, B * B)
    s = np.maximum(np.mean(np.abs(flat), axis=1, dtype=np.float32), np.float32(1e-8)).astype(np.float32)
    t = np.clip(np.rint(flat / s[:, None]), -1, 1).astype(np.int8)
    return t.reshape(R, K, B, B), s.reshape(R, K)


def activation_quantize_int8(x: np.ndarray):
    """Per-token absmax int8 quantisation.

    Restates ``bonsai-test/bitlinear.py:58-69`` for 8 bits, kept in integer form:
    ``absmax = max(max|x|, 1e-8)``, ``scale = 128 / absmax`` (float32, correctly
    rounded), ``q = clamp(rint(x * scale), -128, 127)`` (round-half-to-even).
    The dequantisation multiplier returned is ``sx = absmax / 128`` (exact: a
    power-of-two division).  Returns ``(q int8, sx float32 [rows])``.
    """
    x = np.asarray(x, dtype=np.float32)
    absmax = np.maximum(np.max(np.abs(x), axis=-1), np.float32(1e-8)).astype(np.float32)
    scale = (np.float32(128.0) / absmax).astype(np.float32)
    q = np.clip(np.rint(x * scale[..., None]), -128, 127).astype(np.int8)
    sx = (absmax / np.float32(128.0)).astype(np.float32)
    return q, sx


# 2-bit code per weight: 0 -> 0b00, +1 -> 0b01, -1 -> 0b11 (0b10 decodes to 0).
_CODE = {0: 0, 1: 1, -1: 3}
_DECODE = np.array([0, 1, 0, -1], dtype=np.int8)


def encode_ternary(t: np.ndarray) -> np.ndarray:
    """Map {-1,0,+1} to 2-bit codes {0b11, 0b00, 0b01}."""
    t = np.asarray(t)
    if not np.all(np.isin(t, (-1, 0, 1))):
        raise ValueError("ternary codes must be in {-1, 0, +1}")
    return (t.astype(np.int64) & 3).astype(np.uint32)


def pack_ternary(t: np.ndarray) -> np.ndarray:
    """Pack ternary tiles [R, K, B_in, B_out] into uint32 words [R, K, B_out, B_in/16].

    This 2-bit storage format is defined by this build (the reference has no
    packed ternary format; only the arithmetic of ``bonsai-test/bitlinear.py``).
    Word (r, k, D, e) holds the 16 weights t[r, k, 16e + i, D], i = 0..15; the
    2-bit code of input index i sits at bit ``8*(i % 4) + 2*(i // 4)``, so that
    ``(word >> 2q) & 0x03030303`` yields the codes of i = 4q..4q+3 in bytes 0..3.
    """
    t = np.asarray(t)
    R, K, Bi, Bo = t.shape
    if Bi % 16:
        raise ValueError("B must be a multiple of 16 for the packed ternary format")
    codes = encode_ternary(t).transpose(0, 1, 3, 2).reshape(R, K, Bo, Bi // 16, 16)
    i = np.arange(16)
    shifts = (8 * (i % 4) + 2 * (i // 4)).astype(np.uint32)
    words = np.zeros((R, K, Bo, Bi // 16), dtype=np.uint32)
    for j in range(16):
        words |= (codes[..., j] << shifts[j]).astype(np.uint32)
    return words


def unpack_ternary(words: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pack_ternary`; returns int8 [R, K, B_in, B_out]."""
    R, K, Bo, E = words.shape
    i = np.arange(16)
    shifts = (8 * (i % 4) + 2 * (i // 4)).astype(np.uint32)
    codes = (words[..., None] >> shifts) & np.uint32(3)                # [R,K,Bo,E,16]
    t = _DECODE[codes.astype(np.int64)].reshape(R, K, Bo, E * 16)
    return np.ascontiguousarray(t.transpose(0, 1, 3, 2))


def ternary_block_partials(q: np.ndarray, t: np.ndarray, col_indices: np.ndarray) -> np.ndarray:
    """Exact integer block partials ``P[n, r, k, j] = sum_i q[n, col*B+i] * t[r,k,i,j]``.

    The build's definition of the ternary Block-ELL product (the per-group
    arithmetic of ``bonsai-test/bitlinear.py:34-69`` with group = one block).
    Dead slots give P = 0.  Computed in int64.
    """
    n = q.shape[0]
    R, K, B, _ = t.shape
    qf = q.astype(np.int64).reshape(n, -1, B)
    P = np.zeros((n, R, K, B), dtype=np.int64)
    for r in range(R):
        for k in range(K):
            c = int(col_indices[r, k])
            if c < 0:
                continue
            P[:, r, k, :] = qf[:, c, :] @ t[r, k].astype(np.int64)
    return P


def ternary_fixed_point(scales: np.ndarray, col_indices: np.ndarray, B: int):
    """Per-row fixed-point form of the fp32 block scales used by the kernels.

    For each block row r the kernels replace ``s[r,k]`` by ``m[r,k] * 2**-e[r]``
    with integer ``m`` small enough that ``sum_k m * P`` cannot overflow int32
    for any int8 input: ``m_max = floor((2**31 - 1) / (K_alive * B * 128))``
    capped at ``2**16 - 1``; ``e[r]`` is the largest integer with
    ``max_k |s[r,k]| * 2**e <= m_max``; ``m = rint(s * 2**e)``.
    Returns ``(m int64 [R,K], e int64 [R])``.  Rows with no live block get e = 0.
    """
    s = np.asarray(scales, dtype=np.float32)
    R, K = s.shape
    alive = np.asarray(col_indices) >= 0
    m = np.zeros((R, K), dtype=np.int64)
    e = np.zeros(R, dtype=np.int64)
    for r in range(R):
        ka = int(alive[r].sum())
        if ka == 0:
            continue
        mmax = max(1, min((2 ** 31 - 1) // (ka * B * 128), 2 ** 16 - 1))
        smax = float(np.max(np.where(alive[r], np.abs(s[r]), 0)))
        if not (0.0 < smax < math.inf):
            m[r] = np.where(alive[r], np.rint(s[r].astype(np.float64)), 0).astype(np.int64)
            continue
        er = math.floor(math.log2(mmax / smax))
        while smax * 2.0 ** er > mmax:
            er -= 1
        while smax * 2.0 ** (er + 1) <= mmax:
            er += 1
        e[r] = er
        m[r] = np.where(alive[r], np.rint(s[r].astype(np.float64) * 2.0 ** er), 0).astype(np.int64)
    return m, e


def ternary_matmul(q: np.ndarray, sq: np.ndarray, t: np.ndarray, scales: np.ndarray,
                   col_indices: np.ndarray, exact_scales: bool = True):
    """Ternary Block-ELL product with int8 activations.

    ``y[n, r*B+j] = sq[n] * sum_k s[r,k] * P[n,r,k,j]`` (float64) when
    ``exact_scales``; otherwise the kernels' fixed-point form
    ``y = f32(f32(sum_k m*P) * 2**-e) * sq`` evaluated exactly as the kernels do
    (int64 sum, then two float32 roundings).  Returns ``(y, acc)`` where ``acc``
    is the int64 ``sum_k m*P`` (``None`` when ``exact_scales``).
    """
    P = ternary_block_partials(q, t, col_indices)                       # [n,R,K,B]
    n, R, K, B = P.shape
    if exact_scales:
        y = np.einsum("nrkj,rk->nrj", P.astype(np.float64), scales.astype(np.float64))
        return (y * sq.astype(np.float64)[:, None, None]).reshape(n, R * B), None
    m, e = ternary_fixed_point(scales, col_indices, B)
    acc = np.einsum("nrkj,rk->nrj", P, m)                               # int64 [n,R,B]
    assert np.all(np.abs(acc) < 2 ** 31)
    mult = np.ldexp(np.float32(1.0), -e).astype(np.float32)              # [R]
    y = (acc.astype(np.float32) * mult[None, :, None]).astype(np.float32)
    y = (y * sq.astype(np.float32)[:, None, None]).astype(np.float32)
    return y.reshape(n, R * B), acc


def ternary_swiglu_fwd(x: np.ndarray, gate, up, down, add_residual: bool = False,
                       exact_scales: bool = True, h_round=None, hq_given=None):
    """Ternary SwiGLU FFN: int8 x, ternary gate/up, re-quantised h, ternary down.

    ``gate``/``up``/``down`` are ``(t [R,K,B,B] int8, s [R,K] f32, col [R,K])``.
    Activations are quantised per token (``bonsai-test/bitlinear.py:58-69``);
    the hidden state is re-quantised per token over d_ff before the down
    projection.  ``h_round`` rounds h (e.g. to bf16) before re-quantisation, as
    the kernels store h in bf16.  ``hq_given = (hq, sh)`` substitutes the
    kernel's own re-quantised hidden state for the down projection.
    Returns a dict with xq, sx, g, u, h, hq, sh, out (and the integer
    accumulators when ``exact_scales`` is False).
    """
    xq, sx = activation_quantize_int8(x)
    g, acc_g = ternary_matmul(xq, sx, *gate, exact_scales=exact_scales)
    u, acc_u = ternary_matmul(xq, sx, *up, exact_scales=exact_scales)
    h = silu(g) * u
    if h_round is not None:
        h = h_round(h)
    if hq_given is None:
        hq, sh = activation_quantize_int8(h)
    else:
        hq, sh = hq_given
    out, acc_d = ternary_matmul(hq, sh, *down, exact_scales=exact_scales)
    if add_residual:
        out = out + np.asarray(x, dtype=out.dtype)
    return dict(xq=xq, sx=sx, g=g, u=u, h=h, hq=hq, sh=sh, out=out,
                acc_g=acc_g, acc_u=acc_u, acc_d=acc_d)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(nan, a, out).astype(np.float32)


# How each function is pinned (enforced in tests/test_oracle.py).
PINS = {
    "BlockELLConfig": "reference tests/test_block_ell.py:17-22 known answers; K>C and <1 errors",
    "k_for_density": "reference tests/test_block_ell.py:75-88 (K shrinks with density); closed form",
    "random_topology": "reference tests/test_block_ell.py:25-31 (shape, dtype, per-row uniqueness)",
    "dense_to_block_ell": "reference tests/test_interop.py:131-148 (shape (16,4,16,16), sequential cols, round trip)",
    "block_ell_to_dense": "round trips (tests/test_block_ell.py:34-39, test_interop.py:132-140); tile-transpose special case",
    "create_block_ell_from_dense": "round trip at density 1.0; top-K by Frobenius norm on a hand-built matrix",
    "block_ell_matmul": "== x @ W.T of block_ell_to_dense (tests/test_block_ell.py:42-54); brute-force loops; "
                        "identity tiles; sentinel contributes 0; linearity",
    "silu": "closed form values (silu(0)=0, silu(z)-silu(-z)=z)",
    "swiglu_fwd": "brute-force dense SwiGLU on tiny shapes, with and without biases; residual adds x exactly",
    "gelu_tanh": "closed forms (0, odd part z/2, large |z|) and torch's tanh-approximate GELU in float64",
    "gelu_mlp_fwd": "brute-force dense fc1 -> tanh GELU -> fc2 with biases",
    "rmsnorm_bwd": "torch float64 autograd of the closed-form RMSNorm (x and scale); finite differences",
    "swiglu_bias_grads": "torch float64 autograd of the dense biased SwiGLU FFN (the three bias gradients)",
    "rmsnorm": "constant-vector closed form; unit-RMS invariance; scale linearity",
    "looped_swiglu": "L=0 identity; L=1 equals one block; L=2 equals composition",
    "looped_core": "n_core=1 without injection or depths == looped_swiglu; one iteration == injection then "
                   "the blocks in order (persistent_mlp_step); a row of depth d == L=d on that row (d=0 "
                   "keeps h); planted mistakes (injection once, freeze at t <= depth, blocks reversed) differ",
    "diagonal_injection": "closed forms: log_A = -inf keeps h, log_dt = log(e - 1) gives dt = 1; torch's "
                          "DiagonalInjection formula in float64",
    "diagonal_injection_bwd": "torch float64 autograd of the injection (h, e, log_A, log_dt); finite differences",
    "block_ell_matmul_t": "== dy @ W of block_ell_to_dense; adjoint identity <A x, y> = <x, A^T y>; sentinel 0",
    "block_ell_weight_grad": "== torch autograd of block_ell_matmul through the dense weight, gathered per tile",
    "swiglu_bwd": "== torch float64 autograd of the dense SwiGLU FFN with residual (x and every tile); "
                  "finite differences on tiny shapes",
    "alive_slots": "hand-built rows with sentinels, out-of-range columns and masked slots",
    "compact_topology": "hand-worked rows (order kept, K_new = max alive, all-dead row); product unchanged",
    "column_importance": "reference tests/test_column_reorder.py:16-29 (shape, >= 0); brute-force loops",
    "column_permutation": "reference tests/test_column_reorder.py:31-35 known answer; ties in index order",
    "apply_permutation": "reference tests/test_column_reorder.py:38-69, :99-113; the permuted FFN is unchanged",
    "k_active_macros": "reference tests/test_column_reorder.py:71-96 known answers; all-dead case",
    "permute_optimizer_rows": "hand-built moment trees: rows of C_ff-leading leaves permuted, other leaves and column mode untouched",
    "transposed_index": "brute force per column on tiny topologies; every valid slot listed once; sentinels left out",
    "ternary_quantize_blocks": "hand-worked block; round-half-even cases; codes in {-1,0,1}",
    "activation_quantize_int8": "hand-worked rows incl. ties and the -128/127 clamps; bitlinear dequant identity",
    "pack_ternary": "hand-computed words; round trip over all codes",
    "ternary_block_partials": "brute-force scalar loops; |P| <= B*128 extreme case",
    "ternary_fixed_point": "m*2^-e within 2^-15 relative of s; worst-case sum fits int32",
    "ternary_matmul": "exact == dense int matmul of unpacked tiles; fixed-point within 2^-14 of exact",
}
