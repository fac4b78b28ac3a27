"""HIP (gfx950) kernels of the Block-ELL SwiGLU path, exposed as torch operators.

Loading this package loads ``_titan_ext.so`` (built by
``looped-blockell-tpu_amd/build.py``), which registers the ``titan::`` operator
namespace over the C ABI of ``liblbk.so``.  There is no fallback: if the
extension is missing, :func:`ops` raises, and every operator raises on CPU
tensors.

The operator names and schemas follow the reference's torch.library
registrations (``csrc/block_ell/block_ell_ops.cpp:49-98``,
``csrc/loop/loop_ops.cpp:36-67``); the reference package's
``looped_blockell/kernels/__init__.py:1`` is an empty placeholder this module
fills.
"""

from __future__ import annotations

import os

import torch

_HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXT_PATH = os.path.join(_HERE, "_titan_ext.so")
LIB_PATH = os.path.join(_HERE, "liblbk.so")

_loaded = False


def ops():
    """Return ``torch.ops.titan`` after loading the extension (raises if not built)."""
    global _loaded
    if not _loaded:
        if not os.path.exists(EXT_PATH):
            raise ImportError(
                f"titan extension not built ({EXT_PATH} missing); run looped-blockell-tpu_amd/build.py")
        torch.ops.load_library(EXT_PATH)
        _loaded = True
    return torch.ops.titan


def loaded_native_paths() -> list[str]:
    return [EXT_PATH, LIB_PATH]


def _gpu(*ts):
    for t in ts:
        if isinstance(t, torch.Tensor) and not t.is_cuda and t.device.type != "meta":
            raise RuntimeError("looped_blockell kernels run on the GPU only; got a CPU tensor")


# ---------------------------------------------------------------- bf16 path

def block_ell_matmul_bwd(grad_out, x, values, col_indices):
    """``titan::block_ell_matmul_bwd``: ``(dx, d_values)`` of ``y = x W^T``; dead slots get zero
    tile gradients."""
    _gpu(grad_out, x, values, col_indices)
    return ops().block_ell_matmul_bwd(grad_out, x, values, col_indices)


class _BlockELLMatmulFunction(torch.autograd.Function):
    """Differentiable Block-ELL product: the backward is ``titan::block_ell_matmul_bwd`` (dx and
    the tile gradients) plus the bias gradient (the column sums of grad_out); the column
    indices get no gradient."""

    @staticmethod
    def forward(ctx, x2, values, col_indices, bias):
        y = ops().block_ell_matmul(x2, values, col_indices, bias)
        ctx.save_for_backward(x2, values, col_indices)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = bias.dtype if bias is not None else None
        return y

    @staticmethod
    def backward(ctx, gy):
        x2, values, col_indices = ctx.saved_tensors
        dy = gy.to(torch.bfloat16).contiguous()
        dx, dv = ops().block_ell_matmul_bwd(dy, x2, values, col_indices)
        db = gy.float().sum(0).to(ctx.bias_dtype) if ctx.has_bias and ctx.needs_input_grad[3] else None
        return dx, dv, None, db


def block_ell_matmul(x: torch.Tensor, values: torch.Tensor, col_indices: torch.Tensor,
                     bias: torch.Tensor | None = None) -> torch.Tensor:
    """x [..., C*B] -> [..., R*B] through the Block-ELL weight (tiles [B_in, B_out]);
    differentiable in x, values and bias (``titan::block_ell_matmul_bwd``)."""
    _gpu(x, values, col_indices)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous()
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, values, bias)):
        y = _BlockELLMatmulFunction.apply(x2, values, col_indices, bias)
    else:
        y = ops().block_ell_matmul(x2, values, col_indices, bias)
    return y.reshape(*lead, y.shape[-1])


def swiglu_fwd(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual: bool = False):
    """``titan::block_ell_swiglu_fwd``: W_down(silu(W_gate x) * W_up x) (+ x)."""
    _gpu(x, v_gate, v_down)
    return ops().block_ell_swiglu_fwd(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual)


def swiglu_fwd_with_intermediate(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual: bool = False):
    """Returns ``(result, h, gate_pre_act, up_output)`` like the reference op."""
    _gpu(x, v_gate, v_down)
    return ops().block_ell_swiglu_fwd_with_intermediate(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down,
                                                        add_residual)


def swiglu_bwd(grad_out, x, gate_pre_act, up_out, h, v_gate, ci_gate, v_up, ci_up, v_down, ci_down,
               add_residual: bool = True):
    """``titan::block_ell_swiglu_bwd``: returns ``(dx, d_v_gate, d_v_up, d_v_down)`` from the
    forward's saved ``x``, ``gate_pre_act``, ``up_out`` and ``h``.  ``dx`` includes
    ``grad_out`` (the forward's residual) as in the reference operator unless
    ``add_residual`` is False."""
    _gpu(grad_out, x, v_gate, v_down)
    if add_residual:
        return ops().block_ell_swiglu_bwd(grad_out, x, gate_pre_act, up_out, h, v_gate, ci_gate, v_up, ci_up,
                                          v_down, ci_down)
    return ops().block_ell_swiglu_bwd_ex(grad_out, x, gate_pre_act, up_out, h, v_gate, ci_gate, v_up, ci_up,
                                         v_down, ci_down, False)


class _SwiGLUFunction(torch.autograd.Function):
    """Differentiable SwiGLU FFN: the forward saves (x, h, gate_pre_act, up_out), the backward
    is ``titan::block_ell_swiglu_bwd``; the column indices get no gradient."""

    @staticmethod
    def forward(ctx, x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual):
        out, h, gp, uo = swiglu_fwd_with_intermediate(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down,
                                                      add_residual)
        ctx.save_for_backward(x, h, gp, uo, v_gate, ci_gate, v_up, ci_up, v_down, ci_down)
        ctx.add_residual = add_residual
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, h, gp, uo, vg, cg, vu, cu, vd, cd = ctx.saved_tensors
        dx, dvg, dvu, dvd = swiglu_bwd(grad_out.to(torch.bfloat16).contiguous(), x, gp, uo, h, vg, cg, vu, cu,
                                       vd, cd, ctx.add_residual)
        return dx, dvg, None, dvu, None, dvd, None, None


class _SwiGLUBiasFunction(torch.autograd.Function):
    """Differentiable SwiGLU FFN with the projections' biases: forward
    ``titan::block_ell_swiglu_fwd_bias``, backward ``titan::block_ell_swiglu_bwd_bias`` (tile and
    bias gradients); the column indices get no gradient."""

    @staticmethod
    def forward(ctx, x, v_gate, ci_gate, b_gate, v_up, ci_up, b_up, v_down, ci_down, b_down, add_residual):
        out, h, gp, uo = ops().block_ell_swiglu_fwd_bias(x, v_gate, ci_gate, b_gate, v_up, ci_up, b_up, v_down,
                                                          ci_down, b_down, add_residual, True)
        ctx.save_for_backward(x, h, gp, uo, v_gate, ci_gate, v_up, ci_up, v_down, ci_down)
        ctx.add_residual = add_residual
        ctx.bias_dtypes = tuple(b.dtype if b is not None else None for b in (b_gate, b_up, b_down))
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, h, gp, uo, vg, cg, vu, cu, vd, cd = ctx.saved_tensors
        dx, dvg, dvu, dvd, dbg, dbu, dbd = ops().block_ell_swiglu_bwd_bias(
            grad_out.to(torch.bfloat16).contiguous(), x, gp, uo, h, vg, cg, vu, cu, vd, cd, ctx.add_residual)
        db = [d.to(t) if t is not None else None for d, t in zip((dbg, dbu, dbd), ctx.bias_dtypes)]
        return dx, dvg, None, db[0], dvu, None, db[1], dvd, None, db[2], None


def swiglu(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual: bool = False,
           b_gate=None, b_up=None, b_down=None):
    """SwiGLU FFN forward that autograd can differentiate (through ``titan::block_ell_swiglu_bwd``,
    or ``..._bwd_bias`` with biases); without gradients it is ``swiglu_fwd`` (or
    ``titan::block_ell_swiglu_fwd_bias``).  ``b_gate``/``b_up`` [d_ff] and ``b_down`` [d_model]
    are optional biases of the three projections."""
    biased = any(b is not None for b in (b_gate, b_up, b_down))
    grad = torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                           for t in (x, v_gate, v_up, v_down, b_gate, b_up, b_down))
    if biased:
        _gpu(x, v_gate, v_down)
        if grad:
            return _SwiGLUBiasFunction.apply(x, v_gate, ci_gate, b_gate, v_up, ci_up, b_up, v_down, ci_down, b_down,
                                             add_residual)
        return ops().block_ell_swiglu_fwd_bias(x, v_gate, ci_gate, b_gate, v_up, ci_up, b_up, v_down, ci_down,
                                               b_down, add_residual, False)[0]
    if grad:
        return _SwiGLUFunction.apply(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual)
    return swiglu_fwd(x, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual)


def block_ell_matmul_prepack(values, col_indices, in_features: int):
    """``titan::block_ell_matmul_prepack``: the packed tiles ``block_ell_matmul`` reads, built once
    for weights that stay fixed (uint8; empty when the shape takes the row-block kernel)."""
    _gpu(values)
    return ops().block_ell_matmul_prepack(values, col_indices, int(in_features))


def block_ell_matmul_prepacked(x, packed, values, col_indices, bias=None):
    """``block_ell_matmul`` (no gradient) from a ``block_ell_matmul_prepack`` copy."""
    _gpu(x, values)
    return ops().block_ell_matmul_prepacked(x, packed, values, col_indices, bias)


def swiglu_prepack(v_gate, ci_gate, v_up, ci_up, v_down, ci_down):
    """``titan::block_ell_swiglu_prepack``: the packed tile copy the two-kernel forward reads,
    built once for weights that stay fixed across forwards (uint8; empty when the geometry has
    no packed form).  Pack again after the values or the column indices change."""
    _gpu(v_gate, v_down)
    return ops().block_ell_swiglu_prepack(v_gate, ci_gate, v_up, ci_up, v_down, ci_down)


def swiglu_fwd_prepacked(x, packed, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, add_residual: bool = False,
                         b_gate=None, b_up=None, b_down=None):
    """SwiGLU forward (optional biases) from a ``swiglu_prepack`` copy: the gate/up and down
    launches only; same result as ``swiglu_fwd`` / ``titan::block_ell_swiglu_fwd_bias``."""
    _gpu(x, v_gate, v_down)
    return ops().block_ell_swiglu_fwd_prepacked(x, packed, v_gate, ci_gate, b_gate, v_up, ci_up, b_up, v_down,
                                                ci_down, b_down, add_residual)


def looped_swiglu(h, norm_scale, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, L: int, eps: float = 1e-5):
    """L applications of h <- h + SwiGLU(RMSNorm(h)) with shared weights, in one operator call (the
    per-iteration launches, faster than the persistent launch of ``looped_swiglu_persistent`` at
    every token count measured)."""
    _gpu(h, v_gate, v_down)
    return ops().looped_swiglu(h, norm_scale, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, L, eps)


def looped_swiglu_bias(h, norm_scale, v_gate, ci_gate, b_gate, v_up, ci_up, b_up, v_down, ci_down, b_down,
                       L: int, eps: float = 1e-5):
    """``looped_swiglu`` with the projections' (optional) biases, as ``swiglu``'s."""
    _gpu(h, v_gate, v_down)
    return ops().looped_swiglu_bias(h, norm_scale, v_gate, ci_gate, b_gate, v_up, ci_up, b_up, v_down, ci_down,
                                    b_down, L, eps)


def looped_swiglu_persistent(h, norm_scale, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, L: int,
                             eps: float = 1e-5):
    """``looped_swiglu`` in one persistent launch: each workgroup owns a 64-token block for all L
    iterations (same tiles, same summation order, same result as the two-kernel path)."""
    _gpu(h, v_gate, v_down)
    return ops().looped_swiglu_persistent(h, norm_scale, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, L, eps)


def looped_swiglu_launches(h, norm_scale, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, L: int,
                           eps: float = 1e-5):
    """``looped_swiglu`` as a gate/up and a down launch per iteration (the path the library takes
    for shapes outside the persistent kernel's)."""
    _gpu(h, v_gate, v_down)
    return ops().looped_swiglu_launches(h, norm_scale, v_gate, ci_gate, v_up, ci_up, v_down, ci_down, L, eps)


class _RMSNormFunction(torch.autograd.Function):
    """Differentiable RMSNorm: the backward is ``titan::rmsnorm_bwd`` (dx and the scale gradient,
    deterministic)."""

    @staticmethod
    def forward(ctx, x, scale, eps):
        ctx.save_for_backward(x, scale)
        ctx.eps = eps
        return ops().rmsnorm(x, scale, eps)

    @staticmethod
    def backward(ctx, gy):
        x, scale = ctx.saved_tensors
        dx, ds = ops().rmsnorm_bwd(gy.to(torch.bfloat16).contiguous(), x, scale, ctx.eps)
        return dx, ds.to(scale.dtype), None


def rmsnorm(x, scale, eps: float = 1e-5):
    """``x / sqrt(mean(x^2) + eps) * scale`` over rows of a 2-D bf16 x; differentiable in x and
    scale (``titan::rmsnorm_bwd``)."""
    _gpu(x)
    if torch.is_grad_enabled() and (x.requires_grad or scale.requires_grad):
        return _RMSNormFunction.apply(x, scale, eps)
    return ops().rmsnorm(x, scale, eps)


def rmsnorm_bwd(grad_out, x, scale, eps: float = 1e-5):
    """``titan::rmsnorm_bwd``: ``(dx bf16, dscale fp32)``."""
    _gpu(grad_out, x)
    return ops().rmsnorm_bwd(grad_out, x, scale, eps)


class _InjectionFunction(torch.autograd.Function):
    """Differentiable diagonal injection: the backward is ``titan::diagonal_injection_bwd`` (dh, de
    and the deterministic per-feature gradients of log_A and log_dt)."""

    @staticmethod
    def forward(ctx, h, e, log_A, log_dt):
        ctx.save_for_backward(h, e, log_A, log_dt)
        return ops().diagonal_injection(h, e, log_A, log_dt)

    @staticmethod
    def backward(ctx, grad_out):
        h, e, log_A, log_dt = ctx.saved_tensors
        dh, de, dla, dld = ops().diagonal_injection_bwd(grad_out.to(torch.bfloat16).contiguous(), h, e, log_A, log_dt)
        return dh, de, dla.to(log_A.dtype), dld.to(log_dt.dtype)


def diagonal_injection(h, e, log_A, log_dt):
    """``decay * h + dt * e`` per feature (``titan::diagonal_injection``), differentiable in all four
    inputs when gradients are enabled."""
    _gpu(h, e)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (h, e, log_A, log_dt)):
        return _InjectionFunction.apply(h, e, log_A, log_dt)
    return ops().diagonal_injection(h, e, log_A, log_dt)


def persistent_mlp_step(h, e, log_A, log_dt, norm_scales, gate_values, gate_col_idx, up_values, up_col_idx,
                        down_values, down_col_idx):
    """``titan::persistent_mlp_step``: injection, then h += SwiGLU(RMSNorm(h)) per core block."""
    _gpu(h, e)
    return ops().persistent_mlp_step(h, e, log_A, log_dt, list(norm_scales), list(gate_values),
                                     list(gate_col_idx), list(up_values), list(up_col_idx), list(down_values),
                                     list(down_col_idx))


def looped_core(h, e, log_A, log_dt, norm_scales, gate_values, gate_col_idx, up_values, up_col_idx, down_values,
                down_col_idx, L: int, biases=None, depths=None, seq_len: int = 1, eps: float = 1e-5,
                persistent: bool = False):
    """``titan::looped_core``: L iterations of injection (``e`` optional) -> the n_core blocks
    ``h += SwiGLU_c(RMSNorm_c(h))`` in order -> the depth freeze ``h = where(t < depth, h_new, h_agg)``
    with one depth per ``seq_len`` rows (``depths`` optional), the state carried in fp32.
    ``biases``: None or one ``(b_gate, b_up, b_down)`` triple (entries may be None) per block.
    ``persistent`` runs all L iterations in one launch.  Not differentiable (see
    ``looped_blockell.layers.LoopedCore`` for the training path)."""
    _gpu(h, *gate_values, *down_values)
    flat = [] if biases is None else [b for trip in biases for b in trip]
    return ops().looped_core(h, e, log_A, log_dt, list(norm_scales), list(gate_values), list(gate_col_idx),
                             list(up_values), list(up_col_idx), list(down_values), list(down_col_idx), flat, L,
                             depths, seq_len, eps, persistent)


def pin_weights_l2(weights) -> None:
    """Kept for API compatibility; HIP has no access-policy window (no-op)."""
    ops().pin_weights_l2(list(weights))


def unpin_weights_l2() -> None:
    ops().unpin_weights_l2()


def check_columns(col_indices: torch.Tensor, C: int) -> torch.Tensor:
    """Device int32 count of column indices outside [-1, C)."""
    _gpu(col_indices)
    return ops().check_columns(col_indices, C)


# ---------------------------------------------------------------- ternary path

def quantize_act_int8(x):
    """Per-token absmax int8: returns (q int8 [N, F], sx fp32 [N]) with x ~= q * sx."""
    _gpu(x)
    return ops().quantize_act_int8(x)


def pack_ternary(t):
    _gpu(t)
    return ops().pack_ternary(t)


def ternary_quantize_weights(values):
    _gpu(values)
    return ops().ternary_quantize_weights(values)


def ternary_matmul(xq, sx, packed, scales, col_indices, want_partials: bool = False):
    _gpu(xq, packed)
    return ops().ternary_matmul(xq, sx, packed, scales, col_indices, want_partials)


def ternary_swiglu_fwd(xq, sx, gate, up, down, x_resid=None):
    """gate/up/down are (packed, scales, col_indices) triples."""
    _gpu(xq)
    return ops().block_ell_swiglu_fwd_ternary(xq, sx, *gate, *up, *down, x_resid)


def ternary_prepare(gate, up, down):
    """``titan::ternary_prepare``: the prepared weights of the B = 64 ternary kernels, built once for
    (packed, scales, col_indices) triples that stay fixed (uint8; empty when the geometry has no
    prepared form).  Prepare again after any of them changes."""
    _gpu(gate[0])
    return ops().ternary_prepare(*gate, *up, *down)


def ternary_swiglu_fwd_prepared(xq, sx, prepared, gate, up, down, x_resid=None):
    """``ternary_swiglu_fwd`` from a ``ternary_prepare`` buffer (same kernels, same result)."""
    _gpu(xq)
    return ops().block_ell_swiglu_fwd_ternary_prepared(xq, sx, prepared, *gate, *up, *down, x_resid)


def ternary_swiglu_fwd_with_intermediate(xq, sx, gate, up, down, x_resid=None):
    """Returns (out, h bf16, hq int8, sh fp32)."""
    _gpu(xq)
    return ops().block_ell_swiglu_fwd_ternary_with_intermediate(xq, sx, *gate, *up, *down, x_resid)


def ternary_swiglu_fwd_accumulators(xq, sx, gate, up, down, x_resid=None):
    """The ternary SwiGLU with its accumulators before scaling exported.

    Returns ``(out, h, hq, sh, acc_gate, acc_up, acc_down, gate_pre, up_pre)``: the int32
    ``sum_k m[r,k] * P`` of the gate and up products ([N, d_ff]) and of the down product
    ([N, d_model]), and the fp32 pre-activations ``f32(f32(acc) * 2^-e) * sx`` that enter
    ``silu(g) * u`` — the integer accumulate-then-scale of BitLinear
    (reference ``bonsai-test/bitlinear.py:34-69``) with one scale per block."""
    _gpu(xq)
    return ops().block_ell_swiglu_fwd_ternary_accumulators(xq, sx, *gate, *up, *down, x_resid)
