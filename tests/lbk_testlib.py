"""Shared helpers for the tests: seeded synthetic inputs and C-ABI calls.

GPU parity tests call the kernels through the C ABI (ctypes over liblbk.so)
with device memory owned by torch, and compare against the CPU oracle.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from oracle import oracle as O


# ------------------------------------------------------------------ inputs

def bell_weight(rng, R, C_, K, B, std=0.02, sentinel=()):
    """(values float32 bf16-representable [R,K,B,B], col int32 [R,K]) with optional dead slots."""
    vals = O.bf16_round((rng.standard_normal((R, K, B, B)) * std).astype(np.float32))
    col = O.random_topology(R, C_, K, rng)
    for (r, k) in sentinel:
        col[r, k] = -1
    return vals, col


def ffn_weights(rng, d_model, d_ff, B, density, sentinel_frac=0.0, std=0.02):
    Cm, Cf = d_model // B, d_ff // B
    Kg = O.k_for_density(Cm, density)
    Kd = O.k_for_density(Cf, density)
    Rf, Rm = d_ff // B, d_model // B
    g = bell_weight(rng, Rf, Cm, Kg, B, std)
    u = bell_weight(rng, Rf, Cm, Kg, B, std)
    d = bell_weight(rng, Rm, Cf, Kd, B, std)
    if sentinel_frac > 0:
        for w in (g, u, d):
            mask = rng.random(w[1].shape) < sentinel_frac
            w[1][mask] = -1
    return g, u, d


def act(rng, N, F):
    return O.bf16_round(rng.standard_normal((N, F)).astype(np.float32))


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = max(np.abs(ref).max(), 1e-30)
    return float(np.abs(y - ref).max() / den), float(np.abs(y - ref).max())


# ------------------------------------------------------------------ torch <-> numpy

def to_gpu_bf16(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).cuda()


def to_gpu(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def to_np(t):
    import torch
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.detach().cpu().numpy()


# ------------------------------------------------------------------ C ABI through ctypes

def abi():
    from looped_blockell import abi as A
    A.load()
    return A


def stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else C.c_void_p(0)


def bell_struct(vals_t, col_t):
    A = abi()
    R, K, B, _ = vals_t.shape
    return A.Bell(vals_t.data_ptr(), col_t.data_ptr(), R, K, B)


def tern_struct(packed_t, scales_t, col_t):
    A = abi()
    R, K, B, _ = packed_t.shape
    return A.BellTernary(packed_t.data_ptr(), scales_t.data_ptr(), col_t.data_ptr(), R, K, B)


def gpu_weight(w):
    import torch
    vals, col = w
    return to_gpu_bf16(vals), to_gpu(col.astype(np.int32))


def abi_matmul(x_t, w_t, bias_t=None):
    import torch
    A = abi()
    vals_t, col_t = w_t
    N, F = x_t.shape
    R, K, B, _ = vals_t.shape
    y = torch.empty(N, R * B, dtype=torch.bfloat16, device=x_t.device)
    wb = bell_struct(vals_t, col_t)
    A.check(A.load().lbk_block_ell_matmul_bf16(ptr(x_t), N, F, F, C.byref(wb), ptr(bias_t), ptr(y), R * B,
                                               stream()), "matmul")
    return y


def abi_matmul_ws(x_t, w_t, bias_t=None):
    """lbk_block_ell_matmul_ws_bf16 (packed tiles on the SwiGLU kernels where the shape allows)."""
    import torch
    A = abi()
    lib = A.load()
    vals_t, col_t = w_t
    N, F = x_t.shape
    R, K, B, _ = vals_t.shape
    y = torch.empty(N, R * B, dtype=torch.bfloat16, device=x_t.device)
    wb = bell_struct(vals_t, col_t)
    wsb = lib.lbk_block_ell_matmul_workspace_bytes(N, F, C.byref(wb))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x_t.device)
    A.check(lib.lbk_block_ell_matmul_ws_bf16(ptr(x_t), N, F, C.byref(wb), ptr(bias_t), ptr(y), ptr(ws), wsb,
                                             stream()), "matmul_ws")
    return y, wsb


PATHS = {0: "none", 1: "decode", 2: "split", 3: "rowblock"}


def swiglu_path(N, d_model, g_t, u_t, d_t, intermediates=False):
    """Which kernels lbk_swiglu_fwd_bf16 runs for this geometry: "decode", "split" (two-kernel
    gate/up + down), "rowblock", or "none" (lbk_swiglu_forward_path)."""
    A = abi()
    gb, ub, db = bell_struct(*g_t), bell_struct(*u_t), bell_struct(*d_t)
    return PATHS[A.load().lbk_swiglu_forward_path(N, d_model, C.byref(gb), C.byref(ub), C.byref(db),
                                                  1 if intermediates else 0)]


def abi_swiglu(x_t, g_t, u_t, d_t, add_residual=False, intermediates=False):
    import torch
    A = abi()
    lib = A.load()
    N, dm = x_t.shape
    gb, ub, db = bell_struct(*g_t), bell_struct(*u_t), bell_struct(*d_t)
    d_ff = g_t[0].shape[0] * g_t[0].shape[2]
    out = torch.empty(N, dm, dtype=torch.bfloat16, device=x_t.device)
    h = gp = uo = None
    if intermediates:
        h, gp, uo = (torch.empty(N, d_ff, dtype=torch.bfloat16, device=x_t.device) for _ in range(3))
    wsb = lib.lbk_swiglu_workspace_bytes(N, dm, C.byref(gb), C.byref(ub), C.byref(db), 1 if intermediates else 0)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x_t.device)
    A.check(lib.lbk_swiglu_fwd_bf16(ptr(x_t), N, dm, C.byref(gb), C.byref(ub), C.byref(db),
                                    1 if add_residual else 0, ptr(out), ptr(h), ptr(gp), ptr(uo),
                                    ptr(ws) if wsb else C.c_void_p(0), wsb, stream()), "swiglu")
    return out, h, gp, uo


def abi_looped(h_t, scale_t, g_t, u_t, d_t, L, eps, persistent=False, out=None, launches=False):
    """The looped block through the C ABI: lbk_looped_swiglu_bf16 (the library's choice of path),
    with persistent=True the one-launch lbk_looped_swiglu_persistent_bf16, with launches=True the
    per-iteration launches of lbk_looped_swiglu_launches_bf16 (one workspace size for all)."""
    import torch
    A = abi()
    lib = A.load()
    N, dm = h_t.shape
    gb, ub, db = bell_struct(*g_t), bell_struct(*u_t), bell_struct(*d_t)
    out = torch.empty_like(h_t) if out is None else out
    wsb = lib.lbk_looped_workspace_bytes(N, dm, C.byref(gb), C.byref(ub), C.byref(db))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=h_t.device)
    fn = (lib.lbk_looped_swiglu_persistent_bf16 if persistent else
          lib.lbk_looped_swiglu_launches_bf16 if launches else lib.lbk_looped_swiglu_bf16)
    A.check(fn(ptr(h_t), N, dm, ptr(scale_t), C.c_float(eps), L, C.byref(gb), C.byref(ub), C.byref(db), ptr(out),
               ptr(ws) if wsb else C.c_void_p(0), wsb, stream()), "looped_persistent" if persistent else "looped")
    return out


def abi_swiglu_bwd(dy_t, x_t, g_t, u_t, h_t, gate_t, up_t, down_t, add_residual=True):
    """Backward through the C ABI; returns (dx, d_gate_values, d_up_values, d_down_values)."""
    import torch
    A = abi()
    lib = A.load()
    N, d_model = x_t.shape
    gb, ub, db = (bell_struct(*w) for w in (gate_t, up_t, down_t))
    wsb = lib.lbk_swiglu_bwd_workspace_bytes(N, d_model, C.byref(gb), C.byref(ub), C.byref(db))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    dx = torch.empty(N, d_model, dtype=torch.bfloat16, device="cuda")
    dvs = [torch.empty_like(w[0]) for w in (gate_t, up_t, down_t)]
    A.check(lib.lbk_swiglu_bwd_bf16(ptr(dy_t), ptr(x_t), ptr(g_t), ptr(u_t), ptr(h_t), N, d_model, C.byref(gb),
                                    C.byref(ub), C.byref(db), 1 if add_residual else 0, ptr(dx), ptr(dvs[0]),
                                    ptr(dvs[1]), ptr(dvs[2]),
                                    ptr(ws), wsb, stream()), "swiglu_bwd")
    return dx, dvs[0], dvs[1], dvs[2]


def core_blocks(rng, n_core, d_model, d_ff, B, density, bias=False, shared=False, sentinel_frac=0.0):
    """n_core looped-core blocks as numpy: (norm_scale, gate, up, down, biases) with
    gate/up/down = (values, col) (bf16-representable float32) and biases None or a triple."""
    out = []
    for _ in range(n_core):
        g, u, d = ffn_weights(rng, d_model, d_ff, B, density, sentinel_frac=sentinel_frac)
        if shared:
            u = (u[0], g[1])
        scale = (1.0 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
        bs = None
        if bias:
            bs = tuple(O.bf16_round((0.05 * rng.standard_normal(n)).astype(np.float32)) for n in (d_ff, d_ff, d_model))
        out.append((scale, g, u, d, bs))
    return out


def core_blocks_gpu(blocks):
    """GPU tensors of core_blocks (the up weight shares the gate's column tensor where the
    numpy columns are the same object)."""
    res = []
    for (scale, g, u, d, bs) in blocks:
        vg, cg = gpu_weight(g)
        vu = to_gpu_bf16(u[0])
        cu = cg if u[1] is g[1] else to_gpu(u[1].astype(np.int32))
        vd, cd = gpu_weight(d)
        bt = None if bs is None else tuple(to_gpu(b) for b in bs)
        res.append((to_gpu(scale), (vg, cg), (vu, cu), (vd, cd), bt))
    return res


def abi_looped_core(h_t, blocks_t, L, eps=1e-5, e_t=None, log_A_t=None, log_dt_t=None, depths_t=None, seq_len=1,
                    persistent=False, out=None, expect=0):
    """lbk_looped_core_bf16 (or the persistent form) through the C ABI; returns the output, or
    the status when it is not the expected one (``expect``)."""
    import torch
    A = abi()
    lib = A.load()
    N, dm = h_t.shape
    arr = (A.CoreBlock * max(1, len(blocks_t)))()
    for c, (sc, g, u, d, bt) in enumerate(blocks_t):
        arr[c].norm_scale = sc.data_ptr()
        arr[c].gate = bell_struct(*g)
        arr[c].up = bell_struct(*u)
        arr[c].down = bell_struct(*d)
        if bt is not None:
            arr[c].b_gate, arr[c].b_up, arr[c].b_down = (b.data_ptr() if b is not None else None for b in bt)
    out = torch.empty_like(h_t) if out is None else out
    wsb = lib.lbk_looped_core_workspace_bytes(N, dm, len(blocks_t), arr)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=h_t.device)
    fn = lib.lbk_looped_core_persistent_bf16 if persistent else lib.lbk_looped_core_bf16
    st = fn(ptr(h_t), ptr(e_t), ptr(log_A_t), ptr(log_dt_t), N, dm, len(blocks_t), arr, C.c_float(eps), L,
            ptr(depths_t), seq_len, ptr(out), ptr(ws), wsb, stream())
    if st != expect:
        A.check(st, "looped_core")
        raise AssertionError(f"looped_core returned OK, expected status {expect}")
    return out if st == 0 else st
