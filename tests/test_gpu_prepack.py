"""GPU tests of the prepacked SwiGLU forward: lbk_swiglu_prepack_bf16 + lbk_swiglu_fwd_prepacked_bf16
against lbk_swiglu_fwd_bias_bf16 (same kernels: bit-identical) on the two-kernel, decode and
general paths, with and without biases; the operator pair and MLPBlock's per-version weight
cache for gradient-free forwards."""

import ctypes as C

import numpy as np
import pytest
import torch

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bias(rng, n):
    return T.to_gpu((0.1 * rng.standard_normal(n)).astype(np.float32))


def _fwd_bias(lib, xt, gb, ub, db, biases, resid):
    N, dm = xt.shape
    out = torch.empty(N, dm, dtype=torch.bfloat16, device=xt.device)
    need = lib.lbk_swiglu_workspace_bytes(N, dm, C.byref(gb), C.byref(ub), C.byref(db), 0)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=xt.device)
    st = lib.lbk_swiglu_fwd_bias_bf16(T.ptr(xt), N, dm, C.byref(gb), C.byref(ub), C.byref(db),
                                      *[T.ptr(b) if b is not None else None for b in biases], int(resid), T.ptr(out),
                                      None, None, None, T.ptr(ws), need, T.stream())
    return st, out


def _fwd_prepacked(lib, xt, gb, ub, db, packed, biases, resid):
    N, dm = xt.shape
    out = torch.empty(N, dm, dtype=torch.bfloat16, device=xt.device)
    need = lib.lbk_swiglu_prepacked_workspace_bytes(N, dm, C.byref(gb), C.byref(ub), C.byref(db), 0)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=xt.device)
    pp = T.ptr(packed) if packed.numel() else None
    st = lib.lbk_swiglu_fwd_prepacked_bf16(T.ptr(xt), N, dm, C.byref(gb), C.byref(ub), C.byref(db), pp,
                                           packed.numel(), *[T.ptr(b) if b is not None else None for b in biases],
                                           int(resid), T.ptr(out), None, None, None, T.ptr(ws), need, T.stream())
    return st, out, need


@pytest.mark.parametrize("case", [
    # (d_model, d_ff, B, density, token counts, path)
    (1024, 4096, 32, 0.25, (300, 64), "two-kernel"),
    (256, 1024, 16, 0.25, (130, 7), "two-kernel / decode"),
    (4096, 14336, 64, 0.10, (16, 3), "decode"),
    (512, 2048, 64, 0.25, (70, 33), "general"),
])
def test_prepacked_matches_per_call_pack(gpu, case):
    d_model, d_ff, B, dens, ns, path = case
    print(f"prepack {case}", flush=True)
    A = T.abi()
    lib = A.load()
    rng = np.random.default_rng(500 + B + d_model)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=0.05)
    wt = [T.gpu_weight(w) for w in (g, u, d)]
    gb, ub, db = (T.bell_struct(*w) for w in wt)
    pbytes = lib.lbk_swiglu_prepacked_bytes(d_model, C.byref(gb), C.byref(ub), C.byref(db))
    assert (pbytes > 0) == (B in (16, 32)), path
    packed = torch.empty(pbytes, dtype=torch.uint8, device="cuda")
    A.check(lib.lbk_swiglu_prepack_bf16(d_model, C.byref(gb), C.byref(ub), C.byref(db),
                                        T.ptr(packed) if pbytes else None, pbytes, T.stream()), "prepack")
    biases = (_bias(rng, d_ff), None, _bias(rng, d_model))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    for n, resid, bs in ((ns[0], True, biases), (ns[1], False, (None, None, None))):
        x = T.act(rng, n, d_model)
        xt = T.to_gpu_bf16(x)
        st, want = _fwd_bias(lib, xt, gb, ub, db, bs, resid)
        A.check(st, "fwd_bias")
        st, got, need = _fwd_prepacked(lib, xt, gb, ub, db, packed, bs, resid)
        A.check(st, "fwd_prepacked")
        torch.cuda.synchronize()
        assert torch.equal(got, want), (path, n)
        if pbytes:   # the prepacked call needs only h (or nothing for decode shapes)
            assert need <= lib.lbk_swiglu_workspace_bytes(n, d_model, C.byref(gb), C.byref(ub), C.byref(db), 0)
        b_np = [None if b is None else T.to_np(b).astype(np.float64) for b in bs]
        ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=resid,
                               biases=None if all(b is None for b in b_np) else tuple(b_np))
        assert T.rel_err(T.to_np(got), ref)[0] <= 1e-2


def test_prepacked_argument_errors(gpu):
    A = T.abi()
    lib = A.load()
    rng = np.random.default_rng(9)
    d_model, d_ff, B = 512, 2048, 32
    wt = [T.gpu_weight(w) for w in T.ffn_weights(rng, d_model, d_ff, B, 0.25)]
    gb, ub, db = (T.bell_struct(*w) for w in wt)
    pbytes = lib.lbk_swiglu_prepacked_bytes(d_model, C.byref(gb), C.byref(ub), C.byref(db))
    assert pbytes > 0
    small = torch.empty(pbytes - 256, dtype=torch.uint8, device="cuda")
    assert lib.lbk_swiglu_prepack_bf16(d_model, C.byref(gb), C.byref(ub), C.byref(db), T.ptr(small),
                                       small.numel(), T.stream()) == A.LBK_ERR_WORKSPACE
    xt = T.to_gpu_bf16(T.act(rng, 40, d_model))
    st, _, _ = _fwd_prepacked(lib, xt, gb, ub, db, small, (None, None, None), False)
    assert st == A.LBK_ERR_WORKSPACE
    st, _, _ = _fwd_prepacked(lib, xt, gb, ub, db, torch.empty(0, dtype=torch.uint8, device="cuda"),
                              (None, None, None), False)
    assert st == A.LBK_ERR_NULL
    from looped_blockell import kernels
    with pytest.raises(RuntimeError, match="packed holds"):
        kernels.swiglu_fwd_prepacked(xt, small[:128], *[t for w in wt for t in w])


def test_mlpblock_inference_cache_follows_weight_versions(gpu):
    from looped_blockell import kernels
    from looped_blockell.layers import MLPBlock
    torch.manual_seed(5)
    m = MLPBlock(256, 1024, use_swiglu=True, tile_size=32, density=0.25, device="cuda")
    with torch.no_grad():
        for lin in (m.w_gate, m.w_up, m.w_down):
            lin.bias.copy_(torch.randn_like(lin.bias) * 0.1)
    x = torch.randn(3, 40, 256, device="cuda").to(torch.bfloat16)

    def fresh():
        bg, bu, bd = m.swiglu_biases()
        with torch.no_grad():
            return kernels.ops().block_ell_swiglu_fwd_bias(x.reshape(-1, 256), *_interleave(m.swiglu_weights(),
                                                           (bg, bu, bd)), False, False)[0].reshape(3, 40, 256)

    with torch.no_grad():
        y0 = m(x)
        assert m._frozen is not None
        assert torch.equal(y0, fresh())
        m.w_down.values.mul_(1.5)                  # in-place update: new version, cache rebuilt
        y1 = m(x)
    assert torch.equal(y1, fresh()) and not torch.equal(y1, y0)
    m.w_gate.alive_mask[1, 0] = False              # topology change
    with torch.inference_mode():
        y2 = m(x)
    assert torch.equal(y2, fresh()) and not torch.equal(y2, y1)
    y3 = m(x)                                      # with gradients: the autograd path, same values
    assert y3.requires_grad and T.rel_err(T.to_np(y3.detach()), T.to_np(y2).astype(np.float64))[0] <= 1e-3
    m.release_inference_cache()
    assert m._frozen is None


def _interleave(w, b):
    vg, cg, vu, cu, vd, cd = w
    return vg, cg, b[0], vu, cu, b[1], vd, cd, b[2]


@pytest.mark.parametrize("case", [
    # (in_features, out_features, B, K, N)
    (1024, 4096, 32, 8, 150),      # panel path
    (4096, 512, 32, 12, 90),       # staged path
    (256, 256, 64, 2, 33),         # row-block (no packed form)
])
def test_matmul_prepacked_matches_ws_entry(gpu, case):
    fin, fout, B, K, N = case
    print(f"matmul prepacked {case}", flush=True)
    A = T.abi()
    lib = A.load()
    rng = np.random.default_rng(fin + fout + 3)
    vals, col = T.bell_weight(rng, fout // B, fin // B, K, B, sentinel=[(0, 0)])
    wt = (T.to_gpu_bf16(vals), T.to_gpu(col))
    wb = T.bell_struct(*wt)
    pb = lib.lbk_block_ell_matmul_prepacked_bytes(fin, C.byref(wb))
    assert (pb > 0) == (B != 64)
    packed = torch.empty(max(pb, 1), dtype=torch.uint8, device="cuda")
    A.check(lib.lbk_block_ell_matmul_prepack_bf16(fin, C.byref(wb), T.ptr(packed), pb, T.stream()), "prepack")
    bias = T.to_gpu((0.1 * rng.standard_normal(fout)).astype(np.float32))
    for n in (N, 7):
        x = T.to_gpu_bf16(T.act(rng, n, fin))
        want, _ = T.abi_matmul_ws(x, wt, bias)
        got = torch.empty(n, fout, dtype=torch.bfloat16, device="cuda")
        A.check(lib.lbk_block_ell_matmul_prepacked_bf16(T.ptr(x), n, fin, C.byref(wb), T.ptr(packed) if pb else None,
                                                        pb, T.ptr(bias), T.ptr(got), T.stream()), "prepacked")
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_linear_inference_cache(gpu):
    from looped_blockell.layers import BlockELLLinear, MLPBlock
    torch.manual_seed(9)
    lin = BlockELLLinear(1024, 512, tile_size=32, density=0.25, device="cuda")
    with torch.no_grad():
        lin.bias.copy_(torch.randn_like(lin.bias) * 0.1)
    x = torch.randn(3, 50, 512, device="cuda").to(torch.bfloat16)
    y_grad = lin(x)                                   # autograd path, packs per call
    with torch.no_grad():
        y0 = lin(x)
        assert lin._frozen is not None
        assert torch.equal(y0, y_grad.detach())
        lin.values.mul_(0.5)
        y1 = lin(x)
    assert torch.equal(y1, lin(x).detach()) and not torch.equal(y1, y0)
    lin.alive_mask[0, 0] = False
    with torch.inference_mode():
        y2 = lin(x)
    assert torch.equal(y2, lin(x).detach()) and not torch.equal(y2, y1)
    lin.release_inference_cache()
    assert lin._frozen is None
    # the GELU MLPBlock runs its two projections from the cached copies
    m = MLPBlock(512, 1024, use_swiglu=False, tile_size=32, density=0.5, device="cuda")
    with torch.no_grad():
        ym = m(x)
    assert m.fc1._frozen is not None and torch.equal(ym, m(x).detach())
