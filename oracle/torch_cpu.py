"""PyTorch CPU restatement of the Block-ELL SwiGLU FFN path — TEST INFRASTRUCTURE ONLY.

The CPU baseline that ``bench.py`` times beside the GPU (its ``cpu_baseline`` leg
is, with ``tests/``, the only importer).  It restates the reference's own array
program in PyTorch CPU float32 — the gather + einsum of
``looped_blockell/layers/block_ell.py:149-182`` composed as the SwiGLU of
``looped_blockell/layers/mlp.py:119-145`` — chunked over tokens to bound the
gather's memory.  Nothing in the shipped path imports it.

Each function is pinned against the numpy oracle (``oracle.oracle``) in
``tests/test_oracle.py``: same inputs, float32 against float64, within 1e-5 of
the output's maximum (1e-3 through the re-quantised hidden state of the ternary
FFN); the int8 activation quantisation is compared exactly.
"""

from __future__ import annotations

import torch

__all__ = ["block_ell_matmul", "swiglu_fwd", "rmsnorm", "looped_swiglu", "activation_quantize_int8",
           "ternary_matmul", "ternary_swiglu_fwd"]

CHUNK = 1024


def block_ell_matmul(x: torch.Tensor, values: torch.Tensor, col_indices: torch.Tensor) -> torch.Tensor:
    """``y[n, r, D] = sum_k x[n, col[r,k], :] @ values[r, k]`` — the gather of column tiles and
    the ``'nrkd,rkdD->nrD'`` einsum of ``looped_blockell/layers/block_ell.py:158-182``; slots
    holding the -1 sentinel contribute nothing (``looped_blockell/opt/cms.py:229-230``)."""
    R, K, B, _ = values.shape
    n = x.shape[0]
    C = x.shape[1] // B
    dead = col_indices < 0
    cols = col_indices.clamp(min=0).reshape(-1).long()
    vals = values.masked_fill(dead[:, :, None, None], 0.0) if bool(dead.any()) else values
    out = torch.empty(n, R * B, dtype=torch.float32)
    for s in range(0, n, CHUNK):
        xt = x[s:s + CHUNK].reshape(-1, C, B)
        xg = xt[:, cols, :].reshape(xt.shape[0], R, K, B)
        out[s:s + CHUNK] = torch.einsum("nrkd,rkdD->nrD", xg, vals).reshape(xt.shape[0], R * B)
    return out


def swiglu_fwd(x, gate, up, down, add_residual: bool = False) -> torch.Tensor:
    """``W_down(silu(W_gate x) * W_up x) (+ x)`` (``looped_blockell/layers/mlp.py:121-145``),
    one token chunk at a time so the hidden state stays in cache-sized pieces."""
    out = torch.empty(x.shape[0], down[0].shape[0] * down[0].shape[2], dtype=torch.float32)
    for s in range(0, x.shape[0], CHUNK):
        xc = x[s:s + CHUNK]
        h = torch.nn.functional.silu(block_ell_matmul(xc, *gate)) * block_ell_matmul(xc, *up)
        y = block_ell_matmul(h, *down)
        out[s:s + CHUNK] = y + xc if add_residual else y
    return out


def rmsnorm(x: torch.Tensor, scale: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * scale`` (``looped_blockell/layers/norms.py:14-15``)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * scale


def looped_swiglu(h, norm_scale, gate, up, down, L: int, eps: float = 1e-5) -> torch.Tensor:
    """L applications of ``h <- h + SwiGLU(RMSNorm(h))`` with shared weights, the core loop of
    ``looped_blockell/looping/looped_model.py:293-350``."""
    for _ in range(L):
        h = h + swiglu_fwd(rmsnorm(h, norm_scale, eps), gate, up, down)
    return h


def activation_quantize_int8(x: torch.Tensor):
    """Per-token absmax int8 quantisation kept in integer form (``bonsai-test/bitlinear.py:58-69``
    at 8 bits): ``q = clamp(round(x * 128/absmax), -128, 127)``, ``sx = absmax / 128``."""
    absmax = x.abs().amax(-1).clamp(min=1e-8)
    q = torch.round(x * (128.0 / absmax)[:, None]).clamp(-128, 127)
    return q, absmax / 128.0


def ternary_matmul(q, sx, t, scales, col_indices) -> torch.Tensor:
    """``y[n, r*B+j] = sx[n] * sum_k s[r,k] * P[n,r,k,j]`` with the integer block partials
    ``P = q_tile @ t[r,k]`` (``bonsai-test/bitlinear.py:34-69``, group = one B x B block).  The
    partials are exact in float32: |P| <= 128 * B < 2^24 for B <= 64 and every product and sum is
    an integer."""
    R, K, B, _ = t.shape
    cols = col_indices.clamp(min=0).reshape(-1).long()
    s = scales.masked_fill(col_indices < 0, 0.0)
    out = torch.empty(q.shape[0], R * B, dtype=torch.float32)
    C = q.shape[1] // B
    for c0 in range(0, q.shape[0], CHUNK):
        qt = q[c0:c0 + CHUNK].reshape(-1, C, B)
        qg = qt[:, cols, :].reshape(qt.shape[0], R, K, B)
        part = torch.einsum("nrkd,rkdD->nrkD", qg, t)                   # exact integer partials
        y = torch.einsum("nrkD,rk->nrD", part, s)
        out[c0:c0 + CHUNK] = (y * sx[c0:c0 + CHUNK, None, None]).reshape(qt.shape[0], R * B)
    return out


def ternary_swiglu_fwd(x, gate, up, down) -> torch.Tensor:
    """Ternary SwiGLU FFN from float activations: int8 x, ternary gate/up, the hidden state
    re-quantised per token, ternary down.  ``gate``/``up``/``down`` are
    ``(t [R,K,B,B] float32 in {-1,0,1}, s [R,K], col [R,K])``."""
    q, sx = activation_quantize_int8(x)
    h = torch.nn.functional.silu(ternary_matmul(q, sx, *gate)) * ternary_matmul(q, sx, *up)
    hq, sh = activation_quantize_int8(h)
    return ternary_matmul(hq, sh, *down)
