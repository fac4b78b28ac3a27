"""GPU tests of the torch-facing API: layer modules, titan:: operators and their
error behaviour, checked against the CPU oracle."""

import numpy as np
import pytest
import torch

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
TOL = 1e-2


def f64(w):
    return (w[0].astype(np.float64), w[1])


def test_titan_swiglu_ops_match_oracle(gpu):
    from looped_blockell import kernels
    rng = np.random.default_rng(21)
    g, u, d = T.ffn_weights(rng, 1024, 4096, 32, 0.25)
    x = T.act(rng, 96, 1024)
    ws = [t for w in (g, u, d) for t in T.gpu_weight(w)]
    out = kernels.swiglu_fwd(T.to_gpu_bf16(x), *ws, add_residual=True)
    ref, h_ref, g_ref, u_ref = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
    assert T.rel_err(T.to_np(out), ref)[0] <= TOL
    r, h, gp, uo = kernels.swiglu_fwd_with_intermediate(T.to_gpu_bf16(x), *ws, add_residual=True)
    for got, want in ((r, ref), (h, h_ref), (gp, g_ref), (uo, u_ref)):
        assert T.rel_err(T.to_np(got), want)[0] <= TOL


def test_mlpblock_layer(gpu):
    from looped_blockell.layers import MLPBlock
    torch.manual_seed(0)
    m = MLPBlock(256, 1024, use_swiglu=True, tile_size=16, density=0.25, device="cuda")
    m.w_down.alive_mask[3, 2] = False           # a pruned tile
    x = torch.randn(2, 50, 256, device="cuda").to(torch.bfloat16)
    y = m(x)
    assert y.shape == (2, 50, 256) and y.dtype == torch.bfloat16

    def w(lin):
        col = lin.col_indices.cpu().numpy().copy()
        col[~lin.alive_mask.cpu().numpy()] = -1
        return lin.values.detach().to(torch.bfloat16).float().cpu().numpy().astype(np.float64), col

    ref, *_ = O.swiglu_fwd(T.to_np(x).reshape(100, 256).astype(np.float64), w(m.w_gate), w(m.w_up), w(m.w_down))
    assert T.rel_err(T.to_np(y).reshape(100, 256), ref)[0] <= TOL


def test_gelu_mlpblock_and_linear_bias(gpu):
    from looped_blockell.layers import BlockELLLinear, MLPBlock
    torch.manual_seed(1)
    lin = BlockELLLinear(128, 256, tile_size=32, density=0.5, device="cuda")
    with torch.no_grad():
        lin.bias.copy_(torch.randn(128) * 0.1)
    x = torch.randn(7, 256, device="cuda").to(torch.bfloat16)
    y = lin(x)
    ref = O.block_ell_matmul(T.to_np(x).astype(np.float64),
                             lin.values.detach().to(torch.bfloat16).float().cpu().numpy().astype(np.float64),
                             lin.col_indices.cpu().numpy()) + lin.bias.detach().cpu().numpy()
    assert T.rel_err(T.to_np(y), ref)[0] <= TOL
    m = MLPBlock(128, 512, use_swiglu=False, tile_size=16, density=1.0, device="cuda")
    assert m(x[:, :128].contiguous()).shape == (7, 128)


def test_rmsnorm_and_injection_ops(gpu):
    from looped_blockell import kernels
    from looped_blockell.layers import RMSNorm
    rng = np.random.default_rng(22)
    x = T.act(rng, 33, 1024)
    norm = RMSNorm(1024, device="cuda")
    with torch.no_grad():
        norm.scale.copy_(torch.from_numpy((1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)))
    y = norm(T.to_gpu_bf16(x))
    ref = O.rmsnorm(x.astype(np.float64), norm.scale.detach().cpu().numpy().astype(np.float64), 1e-5)
    assert T.rel_err(T.to_np(y), ref)[0] <= TOL
    e = T.act(rng, 33, 1024)
    la = (0.3 * rng.standard_normal(1024)).astype(np.float32)
    ld = (0.5 * rng.standard_normal(1024)).astype(np.float32)
    hi = kernels.diagonal_injection(T.to_gpu_bf16(x), T.to_gpu_bf16(e), T.to_gpu(la), T.to_gpu(ld))
    dt = np.log1p(np.exp(ld.astype(np.float64)))
    ref = np.exp(-dt * np.exp(la.astype(np.float64))) * x + dt * e        # interop/pt_model.py:930-935
    assert T.rel_err(T.to_np(hi), ref)[0] <= TOL


def test_persistent_mlp_step_matches_reference_semantics(gpu):
    from looped_blockell import kernels
    rng = np.random.default_rng(23)
    d_model, d_ff, B, N = 256, 1024, 16, 70
    blocks = [T.ffn_weights(rng, d_model, d_ff, B, 0.25) for _ in range(2)]
    scales = [(1 + 0.1 * rng.standard_normal(d_model)).astype(np.float32) for _ in range(2)]
    h, e = T.act(rng, N, d_model), T.act(rng, N, d_model)
    la = (0.2 * rng.standard_normal(d_model)).astype(np.float32)
    ld = (0.2 * rng.standard_normal(d_model)).astype(np.float32)
    gw = [[T.gpu_weight(w) for w in blk] for blk in blocks]
    out = kernels.persistent_mlp_step(
        T.to_gpu_bf16(h), T.to_gpu_bf16(e), T.to_gpu(la), T.to_gpu(ld), [T.to_gpu_bf16(s) for s in scales],
        [b[0][0] for b in gw], [b[0][1] for b in gw], [b[1][0] for b in gw], [b[1][1] for b in gw],
        [b[2][0] for b in gw], [b[2][1] for b in gw])
    # reference: csrc/loop/persistent_core.cu:273-338 (injection once, then per core block, eps 1e-6)
    dt = np.log1p(np.exp(ld.astype(np.float64)))
    cur = np.exp(-dt * np.exp(la.astype(np.float64))) * h + dt * e
    for blk, s in zip(blocks, scales):
        sb = O.bf16_round(s).astype(np.float64)
        cur = cur + O.swiglu_fwd(O.rmsnorm(cur, sb, 1e-6), *(f64(w) for w in blk))[0]
    assert T.rel_err(T.to_np(out), cur)[0] <= TOL
    kernels.pin_weights_l2([b[0][0] for b in gw])      # no-ops kept for API compatibility
    kernels.unpin_weights_l2()


def test_persistent_mlp_step_rounding(gpu):
    """The rounding persistent_mlp_step uses, pinned: per core block the residual add happens in
    fp32 and the state is rounded to bf16 once (= titan::looped_swiglu with L = 1, eps 1e-6, bit for
    bit), where the reference rounds mlp_out to bf16 and adds in bf16 (csrc/loop/persistent_core.cu:
    317-334); the two differ by at most a couple of bf16 ulps of the state."""
    from looped_blockell import kernels
    rng = np.random.default_rng(24)
    d_model, d_ff, B, N = 256, 1024, 16, 64
    blocks = [T.ffn_weights(rng, d_model, d_ff, B, 0.25) for _ in range(2)]
    scales = [(1 + 0.1 * rng.standard_normal(d_model)).astype(np.float32) for _ in range(2)]
    h, e = T.act(rng, N, d_model), T.act(rng, N, d_model)
    la = (0.2 * rng.standard_normal(d_model)).astype(np.float32)
    ld = (0.2 * rng.standard_normal(d_model)).astype(np.float32)
    gw = [[T.gpu_weight(w) for w in blk] for blk in blocks]
    st = [T.to_gpu_bf16(s) for s in scales]
    out = kernels.persistent_mlp_step(
        T.to_gpu_bf16(h), T.to_gpu_bf16(e), T.to_gpu(la), T.to_gpu(ld), st,
        [b[0][0] for b in gw], [b[0][1] for b in gw], [b[1][0] for b in gw], [b[1][1] for b in gw],
        [b[2][0] for b in gw], [b[2][1] for b in gw])
    cur = kernels.diagonal_injection(T.to_gpu_bf16(h), T.to_gpu_bf16(e), T.to_gpu(la), T.to_gpu(ld))
    for b, s in zip(gw, st):
        cur = kernels.looped_swiglu(cur, s, b[0][0], b[0][1], b[1][0], b[1][1], b[2][0], b[2][1], L=1, eps=1e-6)
    assert torch.equal(out, cur)
    # the reference's double rounding, evaluated from the same injected state on the CPU
    x0 = T.to_np(kernels.diagonal_injection(T.to_gpu_bf16(h), T.to_gpu_bf16(e), T.to_gpu(la), T.to_gpu(ld)))
    ref = x0.astype(np.float64)
    for blk, s in zip(blocks, scales):
        normed = O.bf16_round(O.rmsnorm(ref, O.bf16_round(s).astype(np.float64), 1e-6).astype(np.float32))
        mlp = O.bf16_round(O.swiglu_fwd(normed.astype(np.float64), *(f64(w) for w in blk))[0].astype(np.float32))
        ref = O.bf16_round((mlp.astype(np.float64) + ref).astype(np.float32)).astype(np.float64)
    assert T.rel_err(T.to_np(out), ref)[0] <= TOL


def test_looped_layer(gpu):
    from looped_blockell.layers import LoopedSwiGLU
    torch.manual_seed(2)
    m = LoopedSwiGLU(1024, 4096, L=4, tile_size=32, density=0.25, device="cuda")
    h = torch.randn(3, 40, 1024, device="cuda").to(torch.bfloat16)
    y = m(h)
    mlp = m.mlp

    def w(lin):
        return lin.values.detach().to(torch.bfloat16).float().cpu().numpy().astype(np.float64), lin.col_indices.cpu().numpy()

    ref = O.looped_swiglu(T.to_np(h).reshape(120, 1024).astype(np.float64), np.ones(1024), w(mlp.w_gate),
                          w(mlp.w_up), w(mlp.w_down), L=4, eps=1e-5)
    assert T.rel_err(T.to_np(y).reshape(120, 1024), ref)[0] <= TOL


def test_ternary_layer(gpu):
    from looped_blockell.layers import TernaryMLPBlock
    m = TernaryMLPBlock.random(512, 2048, 64, 0.125, device="cuda", seed=4)
    x = torch.randn(2, 30, 512, device="cuda").to(torch.bfloat16)
    y = m(x)
    assert y.shape == x.shape and torch.isfinite(y.float()).all()

    def w(tw):
        packed = tw.packed.cpu().numpy().view(np.uint32)
        return O.unpack_ternary(packed), tw.scales.cpu().numpy(), tw.col_indices.cpu().numpy()

    ref = O.ternary_swiglu_fwd(T.to_np(x).reshape(60, 512), w(m.w_gate), w(m.w_up), w(m.w_down),
                               exact_scales=True, h_round=O.bf16_round)
    from test_gpu_ternary import ffn_vs_exact
    ffn_vs_exact(T.to_np(y).reshape(60, 512), ref["out"])


def test_op_errors(gpu):
    from looped_blockell import kernels
    x = torch.zeros(4, 64, device="cuda", dtype=torch.bfloat16)
    v = torch.zeros(2, 2, 32, 32, device="cuda", dtype=torch.bfloat16)
    c = torch.zeros(2, 2, device="cuda", dtype=torch.int32)
    with pytest.raises(RuntimeError):          # fp32 values
        kernels.block_ell_matmul(x, v.float(), c)
    with pytest.raises(RuntimeError):          # int64 columns
        kernels.block_ell_matmul(x, v, c.long())
    with pytest.raises(RuntimeError):          # B = 24
        kernels.block_ell_matmul(torch.zeros(4, 48, device="cuda", dtype=torch.bfloat16),
                                 torch.zeros(2, 2, 24, 24, device="cuda", dtype=torch.bfloat16), c)
    v3 = torch.zeros(3, 2, 32, 32, device="cuda", dtype=torch.bfloat16)
    c3 = torch.zeros(3, 2, device="cuda", dtype=torch.int32)
    with pytest.raises(RuntimeError):          # down R*B = 96 inconsistent with d_model = 64
        kernels.swiglu_fwd(x, v, c, v, c, v3, c3)
    bad = kernels.check_columns(torch.tensor([[0, 1], [-1, 7], [2, -3]], device="cuda", dtype=torch.int32), 4)
    assert int(bad) == 2
    empty = kernels.block_ell_matmul(torch.zeros(0, 64, device="cuda", dtype=torch.bfloat16), v, c)
    assert empty.shape == (0, 64)


@pytest.mark.parametrize("shape", ["decode", "split", "ternary"])
def test_graph_capture_replays(gpu, shape):
    """The forward operators captured into a HIP graph: every replay (with eager work and a
    synchronisation between replays) matches the eager result bit for bit.  No forward path
    records a memset node: the kernels clear nothing through hipMemsetAsync."""
    import torch
    from looped_blockell import kernels
    _say(f"graph capture {shape}")
    rng = np.random.default_rng(40)
    if shape == "ternary":
        d_model, d_ff, B, N = 512, 2048, 64, 200
        def tw(R, C_, K):
            t = rng.integers(-1, 2, size=(R, K, B, B)).astype(np.int8)
            s = (rng.random((R, K)) * 0.01 + 0.01).astype(np.float32)
            col = O.random_topology(R, C_, K, rng)
            return (T.to_gpu(O.pack_ternary(t).view(np.int32)), T.to_gpu(s), T.to_gpu(col.astype(np.int32)))
        g, u, d = tw(d_ff // B, d_model // B, 2), tw(d_ff // B, d_model // B, 2), tw(d_model // B, d_ff // B, 4)
        x = T.to_gpu_bf16(T.act(rng, N, d_model))
        xq, sx = kernels.quantize_act_int8(x)
        fn = lambda: kernels.ternary_swiglu_fwd(xq, sx, g, u, d, x)
    else:
        d_model, d_ff, B, N = (1024, 4096, 64, 16) if shape == "decode" else (512, 2048, 32, 300)
        g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.125 if shape == "decode" else 0.25)
        gt, ut, dt = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
        x = T.to_gpu_bf16(T.act(rng, N, d_model))
        fn = lambda: kernels.swiglu_fwd(x, *gt, *ut, *dt, add_residual=True)
    ref = fn().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = fn()
    junk = torch.empty(1 << 20, device="cuda")
    for rep in range(4):
        junk.normal_()                         # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {rep} differs"


def test_diagonal_injection_backward(gpu):
    """Gradients of the injection (h, e, log_A, log_dt) through the autograd wrapper against the
    float64 oracle; the C ABI entry with optional outputs; bit-identical repeated calls."""
    import ctypes as C
    from looped_blockell import kernels
    rng = np.random.default_rng(61)
    N, d = 130, 384                      # three 64-row blocks, the last ragged
    h, e, dy = T.act(rng, N, d), T.act(rng, N, d), T.act(rng, N, d)
    la = (0.3 * rng.standard_normal(d)).astype(np.float32)
    ld = (0.5 * rng.standard_normal(d)).astype(np.float32)
    th, te = T.to_gpu_bf16(h).requires_grad_(True), T.to_gpu_bf16(e).requires_grad_(True)
    tla, tld = T.to_gpu(la).requires_grad_(True), T.to_gpu(ld).requires_grad_(True)
    out = kernels.diagonal_injection(th, te, tla, tld)
    out.backward(T.to_gpu_bf16(dy))
    ref = O.diagonal_injection_bwd(h.astype(np.float64), e.astype(np.float64), la.astype(np.float64),
                                   ld.astype(np.float64), dy.astype(np.float64))
    for got, want, tol in ((th.grad, ref[0], TOL), (te.grad, ref[1], TOL), (tla.grad, ref[2], 1e-4),
                           (tld.grad, ref[3], 1e-4)):
        assert T.rel_err(T.to_np(got), want)[0] <= tol
    # through the C ABI: only the parameter gradients, twice, bit-identical
    A = T.abi()
    lib = A.load()
    wsb = lib.lbk_diagonal_injection_bwd_workspace_bytes(N, d)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    res = []
    tdy = T.to_gpu_bf16(dy)
    for _ in range(2):
        g1, g2 = torch.empty(d, device="cuda"), torch.empty(d, device="cuda")
        A.check(lib.lbk_diagonal_injection_bwd_bf16(T.ptr(tdy), T.ptr(th.detach()), T.ptr(te.detach()),
                                                    T.ptr(tla.detach()), T.ptr(tld.detach()), N, d, None, None,
                                                    T.ptr(g1), T.ptr(g2), T.ptr(ws), wsb, T.stream()), "inj_bwd")
        torch.cuda.synchronize()
        res.append((g1, g2))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    assert torch.equal(res[0][0], tla.grad) and torch.equal(res[0][1], tld.grad)
    assert lib.lbk_diagonal_injection_bwd_bf16(None, None, None, T.ptr(tla.detach()), T.ptr(tld.detach()), N, d,
                                               None, None, None, None, T.ptr(ws), wsb, T.stream()) == A.LBK_ERR_NULL
