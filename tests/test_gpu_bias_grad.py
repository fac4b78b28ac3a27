"""GPU tests of the biased SwiGLU (forward on every kernel path, backward with the bias
gradients, the looped block), the RMSNorm backward, the tanh GELU MLP, and the autograd guard
on operators without a derivative — each against the CPU oracle."""

import numpy as np
import pytest
import torch

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _say(msg):
    print(msg, flush=True)


def f64(w):
    return (w[0].astype(np.float64), w[1])


def _biases(rng, d_model, d_ff, scale=0.05):
    return tuple(O.bf16_round((scale * rng.standard_normal(n)).astype(np.float32)) for n in (d_ff, d_ff, d_model))


BIAS_CASES = [
    # (d_model, d_ff, B, density, N, kernels of the plain forward)
    (1024, 4096, 32, 0.25, 130, "split"),
    (256, 1024, 16, 0.25, 70, "split"),
    (512, 1024, 64, 0.25, 33, "decode"),
    (512, 1024, 64, 0.25, 100, "rowblock"),
    (1024, 3072, 64, 0.125, 16, "decode"),
    (512, 1024, 32, 0.25, 9, "decode"),
]


@pytest.mark.parametrize("case", BIAS_CASES)
def test_swiglu_bias_forward_and_intermediates(gpu, case):
    from looped_blockell import kernels
    d_model, d_ff, B, dens, N, path = case
    _say(f"swiglu bias {case}")
    rng = np.random.default_rng(abs(hash(case[:5])) % 2 ** 31)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=0.05)
    bs = _biases(rng, d_model, d_ff)
    x = T.act(rng, N, d_model)
    ws = [t for w in (g, u, d) for t in T.gpu_weight(w)]
    assert T.swiglu_path(N, d_model, ws[0:2], ws[2:4], ws[4:6]) == path
    bt = [T.to_gpu(b) for b in bs]
    xt = T.to_gpu_bf16(x)
    args = (xt, ws[0], ws[1], bt[0], ws[2], ws[3], bt[1], ws[4], ws[5], bt[2])
    out, *_ = kernels.ops().block_ell_swiglu_fwd_bias(*args, True, False)
    ref, h_ref, g_ref, u_ref = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True,
                                            biases=tuple(b.astype(np.float64) for b in bs))
    assert T.rel_err(T.to_np(out), ref)[0] <= TOL
    r, h, gp, uo = kernels.ops().block_ell_swiglu_fwd_bias(*args, True, True)
    for got, want in ((r, ref), (h, h_ref), (gp, g_ref), (uo, u_ref)):
        assert T.rel_err(T.to_np(got), want)[0] <= TOL
    # without biases the biased op equals the plain one bit for bit
    plain = kernels.swiglu_fwd(xt, *ws, add_residual=True)
    nob, *_ = kernels.ops().block_ell_swiglu_fwd_bias(xt, ws[0], ws[1], None, ws[2], ws[3], None, ws[4], ws[5], None,
                                                     True, False)
    assert torch.equal(plain, nob)


@pytest.mark.parametrize("case", [(1024, 4096, 32, 0.25, 130), (256, 512, 64, 0.5, 40)])
def test_swiglu_bias_backward(gpu, case):
    from looped_blockell import kernels
    d_model, d_ff, B, dens, N = case
    _say(f"swiglu bias backward {case}")
    rng = np.random.default_rng(abs(hash(case)) % 2 ** 31 + 1)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=0.05)
    bs = _biases(rng, d_model, d_ff)
    x, dy = T.act(rng, N, d_model), T.act(rng, N, d_model)
    ws = [t for w in (g, u, d) for t in T.gpu_weight(w)]
    bt = [T.to_gpu(b) for b in bs]
    _, h, gp, uo = kernels.ops().block_ell_swiglu_fwd_bias(T.to_gpu_bf16(x), ws[0], ws[1], bt[0], ws[2], ws[3], bt[1],
                                                           ws[4], ws[5], bt[2], True, True)
    dx, dvg, dvu, dvd, dbg, dbu, dbd = kernels.ops().block_ell_swiglu_bwd_bias(
        T.to_gpu_bf16(dy), T.to_gpu_bf16(x), gp, uo, h, *ws, True)
    gpn, uon, hn = T.to_np(gp).astype(np.float64), T.to_np(uo).astype(np.float64), T.to_np(h).astype(np.float64)
    rdx, rdg, rdu, rdd = O.swiglu_bwd(dy, x, gpn, uon, hn, f64(g), f64(u), f64(d))
    for got, want in ((dx, rdx), (dvg, rdg), (dvu, rdu), (dvd, rdd)):
        assert T.rel_err(T.to_np(got), want)[0] <= TOL
    rbg, rbu, rbd = O.swiglu_bias_grads(dy, gpn, uon, f64(d))
    for got, want in ((dbg, rbg), (dbu, rbu), (dbd, rbd)):
        assert T.rel_err(T.to_np(got), want)[0] <= TOL
    # deterministic
    again = kernels.ops().block_ell_swiglu_bwd_bias(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), gp, uo, h, *ws, True)
    assert all(torch.equal(a, b) for a, b in zip(again, (dx, dvg, dvu, dvd, dbg, dbu, dbd)))


@pytest.mark.parametrize("case", [(1024, 4096, 32, 0.25, 130, 4), (256, 1024, 16, 0.25, 50, 3),
                                  (128, 512, 64, 0.5, 40, 2)])
def test_looped_bias(gpu, case):
    from looped_blockell import kernels
    d_model, d_ff, B, dens, N, L = case
    _say(f"looped bias {case}")
    rng = np.random.default_rng(abs(hash(case)) % 2 ** 31 + 2)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens)
    bs = _biases(rng, d_model, d_ff)
    h = T.act(rng, N, d_model)
    scale = (1.0 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
    ws = [t for w in (g, u, d) for t in T.gpu_weight(w)]
    bt = [T.to_gpu(b) for b in bs]
    out = kernels.looped_swiglu_bias(T.to_gpu_bf16(h), T.to_gpu(scale), ws[0], ws[1], bt[0], ws[2], ws[3], bt[1],
                                     ws[4], ws[5], bt[2], L=L)
    ref = O.looped_swiglu(h.astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L=L,
                          biases=tuple(b.astype(np.float64) for b in bs))
    assert T.rel_err(T.to_np(out), ref)[0] <= TOL


def test_rmsnorm_backward(gpu):
    from looped_blockell import kernels
    rng = np.random.default_rng(31)
    for N, dm in ((70, 1024), (1, 256), (200, 96)):
        x, dy = T.act(rng, N, dm), T.act(rng, N, dm)
        s = (1 + 0.2 * rng.standard_normal(dm)).astype(np.float32)
        dx, ds = kernels.rmsnorm_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), T.to_gpu(s), 1e-5)
        rdx, rds = O.rmsnorm_bwd(x, s, dy, 1e-5)
        assert T.rel_err(T.to_np(dx), rdx)[0] <= TOL
        assert T.rel_err(T.to_np(ds), rds)[0] <= 1e-4
        dx2, ds2 = kernels.rmsnorm_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), T.to_gpu(s), 1e-5)
        assert torch.equal(dx, dx2) and torch.equal(ds, ds2)


def test_layer_gradients_flow(gpu):
    """RMSNorm, the biased SwiGLU MLPBlock and LoopedSwiGLU train: gradients reach the norm scale,
    every tile and every bias, and match the oracle's for RMSNorm -> MLPBlock."""
    from looped_blockell.layers import LoopedSwiGLU, MLPBlock, RMSNorm
    torch.manual_seed(5)
    dm, dff, N = 256, 1024, 48
    norm = RMSNorm(dm, device="cuda")
    mlp = MLPBlock(dm, dff, use_swiglu=True, tile_size=32, density=0.5, device="cuda")
    with torch.no_grad():
        norm.scale.copy_(1 + 0.1 * torch.randn(dm))
        for lin in (mlp.w_gate, mlp.w_up, mlp.w_down):
            lin.bias.copy_(0.05 * torch.randn_like(lin.bias))
    x = torch.randn(N, dm, device="cuda").to(torch.bfloat16).requires_grad_(True)
    dy = torch.randn(N, dm, device="cuda").to(torch.bfloat16)
    y = mlp(norm(x))
    (y.float() * dy.float()).sum().backward()
    for p in (norm.scale, mlp.w_gate.values, mlp.w_down.values, mlp.w_gate.bias, mlp.w_up.bias, mlp.w_down.bias):
        assert p.grad is not None and torch.isfinite(p.grad).all() and p.grad.abs().sum() > 0
    # the bias gradient of down is the column sum of dy (exact math), of the norm scale the oracle's
    np.testing.assert_allclose(T.to_np(mlp.w_down.bias.grad), T.to_np(dy).sum(0), rtol=1e-3, atol=1e-3)
    xn = T.to_np(x).astype(np.float64)
    n_ref = O.rmsnorm(xn, T.to_np(norm.scale).astype(np.float64))
    bs = tuple(T.to_np(l.bias).astype(np.float64) for l in (mlp.w_gate, mlp.w_up, mlp.w_down))

    def w(lin):
        return lin.values.detach().to(torch.bfloat16).float().cpu().numpy().astype(np.float64), \
            lin.col_indices.cpu().numpy()

    # x gradient through SwiGLU (oracle backward, residual excluded) then RMSNorm (oracle backward)
    _, hh, gpre, upre = O.swiglu_fwd(n_ref, w(mlp.w_gate), w(mlp.w_up), w(mlp.w_down), biases=bs)
    dn, *_ = O.swiglu_bwd(T.to_np(dy).astype(np.float64), n_ref, gpre, upre, hh, w(mlp.w_gate), w(mlp.w_up),
                          w(mlp.w_down))
    dn = dn - T.to_np(dy).astype(np.float64)
    dx_ref, ds_ref = O.rmsnorm_bwd(xn, T.to_np(norm.scale).astype(np.float64), dn)
    assert T.rel_err(T.to_np(x.grad), dx_ref)[0] <= 2 * TOL
    assert T.rel_err(T.to_np(norm.scale.grad), ds_ref)[0] <= 2 * TOL
    # looped block: the training path (L applications of the differentiable pieces)
    m = LoopedSwiGLU(dm, dff, L=3, tile_size=32, density=0.5, device="cuda")
    h = torch.randn(N, dm, device="cuda").to(torch.bfloat16).requires_grad_(True)
    out = m(h)
    with torch.no_grad():
        inf = m(h.detach())
    assert T.rel_err(T.to_np(out), T.to_np(inf))[0] <= TOL
    out.float().sum().backward()
    assert h.grad is not None and m.norm.scale.grad is not None and m.mlp.w_up.values.grad is not None


def test_gelu_mlp_tanh_form(gpu):
    from looped_blockell.layers import MLPBlock
    torch.manual_seed(3)
    m = MLPBlock(128, 512, use_swiglu=False, tile_size=16, density=0.5, device="cuda")
    with torch.no_grad():
        m.fc1.bias.copy_(0.5 * torch.randn(512))
        m.fc2.bias.copy_(0.1 * torch.randn(128))
        m.fc1.values.mul_(40.0)        # pre-activations of order 1, where the two GELU forms differ
    x = torch.randn(9, 128, device="cuda").to(torch.bfloat16)
    y = m(x)

    def w(lin):
        return lin.values.detach().to(torch.bfloat16).float().cpu().numpy().astype(np.float64), \
            lin.col_indices.cpu().numpy()

    ref = O.gelu_mlp_fwd(T.to_np(x).astype(np.float64), w(m.fc1), w(m.fc2), T.to_np(m.fc1.bias).astype(np.float64),
                         T.to_np(m.fc2.bias).astype(np.float64))
    assert T.rel_err(T.to_np(y), ref)[0] <= TOL


def test_ops_without_derivative_raise_on_backward(gpu):
    """An operator with no autograd formula, called on inputs that require grad, gives outputs whose
    backward raises instead of silently returning no gradient."""
    from looped_blockell import kernels
    rng = np.random.default_rng(41)
    g, u, d = T.ffn_weights(rng, 256, 1024, 32, 0.25)
    ws = [t for w in (g, u, d) for t in T.gpu_weight(w)]
    h = T.to_gpu_bf16(T.act(rng, 20, 256)).requires_grad_(True)
    scale = torch.ones(256, device="cuda", requires_grad=True)
    out = kernels.ops().looped_swiglu(h, scale, *ws, 2, 1e-5)
    with pytest.raises(RuntimeError):
        out.float().sum().backward()


def test_b16_shared_topology_bias_full_size(gpu):
    """The reference-default layer (tile 16, gate and up from one seed, so one shared topology,
    with biases) at full size: 16384 + 5 tokens at d_model 1024, d_ff 4096, density 0.25 take the
    16-wave gate/up kernel's shared-topology, bias instantiations (the plain forward) and their
    normalising forms (the looped block).  The up weight is given the gate's column-index tensor
    itself; sampled rows against the float64 oracle."""
    from looped_blockell import kernels
    rng = np.random.default_rng(1618)
    d_model, d_ff, B, N, L = 1024, 4096, 16, 16384 + 5, 2
    _say("b16 shared topology + biases d1024 ff4096 N16389 full size")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25, sentinel_frac=0.05)
    u = (u[0], g[1])                       # one topology for gate and up
    bs = _biases(rng, d_model, d_ff)
    bs64 = tuple(b.astype(np.float64) for b in bs)
    x = T.act(rng, N, d_model)
    vg, cg = T.gpu_weight(g)
    vu = T.to_gpu_bf16(u[0])
    vd, cd = T.gpu_weight(d)
    bt = [T.to_gpu(b) for b in bs]
    xt = T.to_gpu_bf16(x)
    rows = np.concatenate([np.sort(rng.choice(N, 192, replace=False)), [0, N - 1]])

    out, *_ = kernels.ops().block_ell_swiglu_fwd_bias(xt, vg, cg, bt[0], vu, cg, bt[1], vd, cd, bt[2], True, False)
    ref, *_ = O.swiglu_fwd(x[rows].astype(np.float64), f64(g), f64(u), f64(d), add_residual=True, biases=bs64)
    rel, ab = T.rel_err(T.to_np(out)[rows], ref)
    assert rel <= TOL, f"forward rel {rel} abs {ab}"

    scale = (1.0 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
    lo = kernels.ops().looped_swiglu_bias(xt, T.to_gpu(scale), vg, cg, bt[0], vu, cg, bt[1], vd, cd, bt[2], L, 1e-5)
    ref = O.looped_swiglu(x[rows].astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L, 1e-5,
                          biases=bs64)
    rel, ab = T.rel_err(T.to_np(lo)[rows], ref)
    assert rel <= TOL, f"looped rel {rel} abs {ab}"
