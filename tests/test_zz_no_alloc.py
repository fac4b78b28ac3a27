"""GPU test of lbk_swiglu_fwd_bf16_noalloc: the SwiGLU forward served from the library's fixed
device scratch array instead of a caller workspace.  Checked against lbk_swiglu_fwd_bf16 (the
same kernels on a caller workspace: bit-identical) on two calls in a row, the second with a
smaller input, for a decode shape (decode kernels: only h in the scratch) and a two-kernel shape
(packed tiles at the start of the scratch, h after them); a call captured in a HIP graph and
replayed; and the refusal of a geometry that needs more than the array, with nothing launched."""

import ctypes as C

import numpy as np
import pytest

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _align256(n):
    return (n + 255) // 256 * 256


def _noalloc(x_t, g_t, u_t, d_t, add_residual, out=None):
    import torch
    A = T.abi()
    lib = A.load()
    N, dm = x_t.shape
    gb, ub, db = T.bell_struct(*g_t), T.bell_struct(*u_t), T.bell_struct(*d_t)
    if out is None:
        out = torch.empty(N, dm, dtype=torch.bfloat16, device=x_t.device)
    st = lib.lbk_swiglu_fwd_bf16_noalloc(T.ptr(x_t), N, dm, C.byref(gb), C.byref(ub), C.byref(db),
                                         1 if add_residual else 0, T.ptr(out), T.stream())
    return st, out


@pytest.mark.parametrize("case", [
    # (d_model, d_ff, B, density, N first call, N second call, two-kernel path)
    (4096, 14336, 64, 0.10, 16, 5, False),   # the decode geometry (decode kernels, h in the scratch)
    (512, 2048, 32, 0.25, 130, 70, True),    # two-kernel path: packed tiles + h in the scratch (2.1 MB)
])
def test_noalloc_matches_workspace_entry(gpu, case):
    import torch
    d_model, d_ff, B, dens, n1, n2, split = case
    print(f"noalloc {case}", flush=True)
    A = T.abi()
    lib = A.load()
    assert lib.lbk_noalloc_scratch_bytes() == 4 << 20
    rng = np.random.default_rng(77 + B)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=0.05)
    ws = [T.gpu_weight(w) for w in (g, u, d)]
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    for n, resid in ((n1, True), (n2, False)):
        gb, ub, db = (T.bell_struct(*w) for w in ws)
        need = lib.lbk_swiglu_workspace_bytes(n, d_model, C.byref(gb), C.byref(ub), C.byref(db), 0)
        assert 0 < need <= 4 << 20
        # the two-kernel path keeps the packed tiles in the workspace beside h; the decode path
        # holds h only
        if split:
            assert need > _align256(n * d_ff * 2), (need, n)
        else:
            assert need == _align256(n * d_ff * 2), (need, n)
        x = T.act(rng, n, d_model)
        xt = T.to_gpu_bf16(x)
        st, out = _noalloc(xt, *ws, resid)
        A.check(st, "swiglu_noalloc")
        ref_ws, *_ = T.abi_swiglu(xt, *ws, add_residual=resid)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_ws)
        ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=resid)
        rel, ab = T.rel_err(T.to_np(out), ref)
        assert rel <= 1e-2, f"rel {rel} abs {ab}"


def test_noalloc_graph_capture(gpu):
    """The no-alloc call captured in a HIP graph (after lbk_noalloc_init and one eager call of the
    geometry) and replayed three times with new inputs copied in between, eager work and
    synchronisations between the replays: every replay equals the eager workspace entry point."""
    import torch
    A = T.abi()
    lib = A.load()
    d_model, d_ff, B, dens, n = 512, 2048, 32, 0.25, 130
    print(f"noalloc graph capture {(d_model, d_ff, B, dens, n)}", flush=True)
    rng = np.random.default_rng(901)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=0.05)
    ws = [T.gpu_weight(w) for w in (g, u, d)]
    A.check(lib.lbk_noalloc_init(), "noalloc_init")
    x_static = T.to_gpu_bf16(T.act(rng, n, d_model))
    out_static = torch.empty(n, d_model, dtype=torch.bfloat16, device="cuda")
    st, _ = _noalloc(x_static, *ws, True, out=out_static)   # eager: kernel attributes set
    A.check(st, "swiglu_noalloc eager")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            st, _ = _noalloc(x_static, *ws, True, out=out_static)
    A.check(st, "swiglu_noalloc captured")
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        x_new = T.to_gpu_bf16(T.act(rng, n, d_model))
        x_static.copy_(x_new)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref_ws, *_ = T.abi_swiglu(x_new, *ws, add_residual=True)
        torch.cuda.synchronize()
        assert torch.equal(out_static, ref_ws), f"replay {rep}"


def test_noalloc_refuses_too_large(gpu):
    """16384 tokens of the headline geometry need ~140 MB of workspace: refused before any launch."""
    import torch
    A = T.abi()
    rng = np.random.default_rng(3)
    d_model, d_ff, B, N = 1024, 4096, 32, 16384
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    ws = [T.gpu_weight(w) for w in (g, u, d)]
    xt = T.to_gpu_bf16(T.act(rng, N, d_model))
    st, out = _noalloc(xt, *ws, False)
    assert st == A.LBK_ERR_TOO_LARGE
    assert "scratch" in A.status_string(st)
