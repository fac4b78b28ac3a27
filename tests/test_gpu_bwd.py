"""Parity of the SwiGLU FFN backward (lbk_swiglu_bwd_bf16) against the oracle.

Cases cover both implementations of each transposed product (LDS panel / staged kernels and the
per-entry gather kernel they fall back to).  The saved forward tensors (gate_pre_act, up_output, h)
are computed by the oracle and rounded
to bf16, then given to both sides; the oracle differentiates in float64.  Bar: max-abs error
<= 1e-2 of max |reference| for dx and every tile gradient (the kernel rounds dg and du to bf16
between its products, as the reference operator does).
"""

import ctypes as C

import numpy as np
import pytest

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _say(msg):
    print(f"[bwd] {msg}", flush=True)


def _inputs(rng, d_model, d_ff, B, dens, N, sf):
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=sf)
    x = T.act(rng, N, d_model)
    dy = T.act(rng, N, d_model)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    _, h, gp, uo = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d))
    gp, uo, h = (O.bf16_round(a.astype(np.float32)) for a in (gp, uo, h))
    return g, u, d, x, dy, gp, uo, h


def _run(g, u, d, x, dy, gp, uo, h):
    G = T.to_gpu_bf16
    return T.abi_swiglu_bwd(G(dy), G(x), G(gp), G(uo), G(h), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d))


BWD_CASES = [
    # (d_model, d_ff, B, density, N, sentinel_frac)
    (256, 1024, 16, 0.25, 100, 0.1),
    (512, 1024, 16, 0.125, 90, 0.05),      # 32 output blocks: dx with 16 waves of two blocks
    (1024, 512, 16, 0.125, 70, 0.0),       # 64 output blocks: 16 waves of four
    (256, 1024, 16, 0.25, 2100, 0.05),     # B = 16 tile gradients: two token chunks, 128-token slices, ragged tail
    (512, 1024, 32, 0.25, 130, 0.05),
    (128, 512, 64, 0.5, 70, 0.0),
    (1024, 4096, 32, 0.25, 2100, 0.0),     # two token chunks of the tile gradients, ragged tail
    (2048, 1024, 32, 0.125, 40, 0.05),     # 64 output blocks: dx over four workgroups per token block
    (4096, 512, 64, 0.25, 20, 0.0),        # d_model > 2048: dh through the per-entry gather kernel too
    (2048, 512, 16, 1.0, 70, 0.0),         # every h block read by 128 down slots: dh over two 64-entry list windows
    (2048, 1024, 32, 1.0, 130, 0.05),      # every h block read by up to 64 slots (one full window), dead slots
]


@pytest.mark.parametrize("case", BWD_CASES)
def test_swiglu_bwd_parity(gpu, case):
    d_model, d_ff, B, dens, N, sf = case
    _say(f"parity {case}")
    rng = np.random.default_rng(hash(case) % 2 ** 31)
    g, u, d, x, dy, gp, uo, h = _inputs(rng, d_model, d_ff, B, dens, N, sf)
    got = _run(g, u, d, x, dy, gp, uo, h)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = O.swiglu_bwd(dy, x, gp, uo, h, f64(g), f64(u), f64(d))
    for gt, rf, name in zip(got, ref, ("dx", "d_gate", "d_up", "d_down")):
        rel, ab = T.rel_err(T.to_np(gt), rf)
        assert rel <= TOL, f"{name}: rel {rel} abs {ab}"
    # dead slots get exactly zero tiles
    for gt, w in zip(got[1:], (g, u, d)):
        dead = w[1] < 0
        if dead.any():
            assert np.all(T.to_np(gt)[dead] == 0)


def test_swiglu_bwd_duplicate_columns_and_deterministic(gpu):
    """Two slots of a row on one column get identical gradients; two calls agree bit for bit."""
    _say("duplicates + determinism")
    rng = np.random.default_rng(5)
    d_model, d_ff, B, N = 256, 512, 32, 300
    g, u, d, x, dy, gp, uo, h = _inputs(rng, d_model, d_ff, B, 0.25, N, 0.0)
    d[1][3, 1] = d[1][3, 0]
    g[1][5, 1] = g[1][5, 0]
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    _, h, gp, uo = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d))
    gp, uo, h = (O.bf16_round(a.astype(np.float32)) for a in (gp, uo, h))
    a = _run(g, u, d, x, dy, gp, uo, h)
    b = _run(g, u, d, x, dy, gp, uo, h)
    for ta, tb in zip(a, b):
        assert np.array_equal(T.to_np(ta), T.to_np(tb))
    ref = O.swiglu_bwd(dy, x, gp, uo, h, f64(g), f64(u), f64(d))
    for gt, rf, name in zip(a, ref, ("dx", "d_gate", "d_up", "d_down")):
        rel, ab = T.rel_err(T.to_np(gt), rf)
        assert rel <= TOL, f"{name}: rel {rel} abs {ab}"
    dd = T.to_np(a[3])
    assert np.array_equal(dd[3, 1], dd[3, 0])
    dg = T.to_np(a[1])
    assert np.array_equal(dg[5, 1], dg[5, 0])


def test_swiglu_bwd_zero_tokens(gpu):
    """N = 0: no input gradient, all tile gradients zero."""
    import torch
    _say("N = 0")
    rng = np.random.default_rng(6)
    g, u, d = T.ffn_weights(rng, 128, 256, 16, 0.5)
    e = torch.empty(0, 128, dtype=torch.bfloat16, device="cuda")
    e2 = torch.empty(0, 256, dtype=torch.bfloat16, device="cuda")
    gw, uw, dw = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    dx, dg, du, dd = T.abi_swiglu_bwd(e, e, e2, e2, e2, gw, uw, dw)
    for t in (dg, du, dd):
        assert torch.count_nonzero(t).item() == 0


def test_torch_op_matches_abi_and_residual_flag(gpu):
    """titan::block_ell_swiglu_bwd equals the C ABI bit for bit; without the residual dx lacks grad_out."""
    from looped_blockell import kernels
    _say("torch op + residual flag")
    rng = np.random.default_rng(7)
    g, u, d, x, dy, gp, uo, h = _inputs(rng, 512, 1024, 32, 0.25, 90, 0.1)
    G = T.to_gpu_bf16
    gw, uw, dw = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    args = (G(dy), G(x), G(gp), G(uo), G(h), gw[0], gw[1], uw[0], uw[1], dw[0], dw[1])
    op = kernels.swiglu_bwd(*args)
    ab = T.abi_swiglu_bwd(args[0], args[1], args[2], args[3], args[4], gw, uw, dw)
    for a_, b_ in zip(op, ab):
        assert np.array_equal(T.to_np(a_), T.to_np(b_))
    nores = kernels.swiglu_bwd(*args, add_residual=False)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = O.swiglu_bwd(dy, x, gp, uo, h, f64(g), f64(u), f64(d))
    rel, absd = T.rel_err(T.to_np(nores[0]), ref[0] - dy)
    assert rel <= TOL, f"dx without residual: rel {rel} abs {absd}"
    for a_, b_ in zip(nores[1:], op[1:]):
        assert np.array_equal(T.to_np(a_), T.to_np(b_))


def test_layer_autograd(gpu):
    """MLPBlock(use_swiglu=True) backward through the HIP operator matches the oracle."""
    import torch
    from looped_blockell.layers import MLPBlock
    _say("layer autograd")
    torch.manual_seed(3)
    m = MLPBlock(256, 1024, use_swiglu=True, tile_size=32, density=0.25, device="cuda")
    m.w_up.alive_mask[2, 1] = False            # a pruned tile gets no gradient
    x = torch.randn(2, 40, 256, device="cuda").to(torch.bfloat16).requires_grad_(True)
    y = m(x)
    dy = torch.randn_like(y)
    y.backward(dy)

    def w(lin):
        col = lin.col_indices.cpu().numpy().copy()
        col[~lin.alive_mask.cpu().numpy()] = -1
        return lin.values.detach().to(torch.bfloat16).float().cpu().numpy().astype(np.float64), col

    xs = T.to_np(x.detach()).reshape(80, 256).astype(np.float64)
    wg, wu, wd = w(m.w_gate), w(m.w_up), w(m.w_down)
    _, h, gp, uo = O.swiglu_fwd(xs, wg, wu, wd)
    gp, uo, h = (O.bf16_round(a.astype(np.float32)) for a in (gp, uo, h))
    dys = T.to_np(dy).reshape(80, 256)
    dx, dvg, dvu, dvd = O.swiglu_bwd(dys, xs, gp, uo, h, wg, wu, wd)
    dx = dx - dys                               # the layer has no residual
    assert T.rel_err(T.to_np(x.grad).reshape(80, 256), dx)[0] <= TOL
    for lin, ref in ((m.w_gate, dvg), (m.w_up, dvu), (m.w_down, dvd)):
        assert T.rel_err(T.to_np(lin.values.grad), ref)[0] <= TOL
    assert torch.count_nonzero(m.w_up.values.grad[2, 1]).item() == 0


# ------------------------------------------------------------------ block_ell_matmul backward

MM_CASES = [
    # (out_features, in_features, B, density, N, sentinel_frac)
    (256, 512, 32, 0.25, 130, 0.1),
    (128, 256, 16, 0.5, 77, 0.0),
    (512, 256, 64, 0.25, 40, 0.05),
    (1024, 4096, 32, 0.25, 2100, 0.0),      # two token chunks of the tile gradients
    (256, 2048, 16, 0.125, 33, 0.0),       # 128 output blocks over 8 workgroups per token block
    (256, 2048, 16, 0.125, 16400, 0.05),   # 128 output blocks at 257 token blocks: the deep-ring dx kernel
    (256, 800, 32, 0.25, 150, 0.1),        # 25 output blocks: the second workgroup of a token block has 7 idle waves
    (2048, 256, 32, 0.5, 70, 0.0),         # one source, 32 list entries per output block over 4 stages
]


def _abi_matmul_bwd(dy_t, x_t, w_t, want_dx=True, want_dv=True):
    import torch
    A = T.abi()
    lib = A.load()
    vals_t, col_t = w_t
    N, F = x_t.shape
    wb = T.bell_struct(vals_t, col_t)
    wsb = lib.lbk_block_ell_matmul_bwd_workspace_bytes(N, F, C.byref(wb))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    dx = torch.empty(N, F, dtype=torch.bfloat16, device="cuda") if want_dx else None
    dv = torch.empty_like(vals_t) if want_dv else None
    A.check(lib.lbk_block_ell_matmul_bwd_bf16(T.ptr(dy_t), T.ptr(x_t), N, F, C.byref(wb), T.ptr(dx), T.ptr(dv),
                                              T.ptr(ws), wsb, T.stream()), "block_ell_matmul_bwd")
    return dx, dv


@pytest.mark.parametrize("case", MM_CASES)
def test_block_ell_matmul_bwd_parity(gpu, case):
    out_f, in_f, B, dens, N, sf = case
    _say(f"matmul bwd {case}")
    rng = np.random.default_rng(abs(hash(case)) % 2 ** 31)
    R, Cb = out_f // B, in_f // B
    vals, col = T.bell_weight(rng, R, Cb, O.k_for_density(Cb, dens), B)
    col[rng.random(col.shape) < sf] = -1
    x, dy = T.act(rng, N, in_f), T.act(rng, N, out_f)
    dx, dv = _abi_matmul_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), T.gpu_weight((vals, col)))
    rdx = O.block_ell_matmul_t(dy.astype(np.float64), vals.astype(np.float64), col, Cb)
    rdv = O.block_ell_weight_grad(x.astype(np.float64), dy.astype(np.float64), col, B)
    for got, ref, name in ((dx, rdx, "dx"), (dv, rdv, "d_values")):
        rel, ab = T.rel_err(T.to_np(got), ref)
        assert rel <= TOL, f"{name}: rel {rel} abs {ab}"
    assert np.all(T.to_np(dv)[col < 0] == 0)


@pytest.mark.parametrize("case", [
    # (out_features, in_features, B, N, topology, sentinel_frac).  Enough workgroups (column-block
    # groups x token chunks, or row groups x chunks) that the tile gradients take the blocked kernels:
    # B = 32: the transposed-list kernel (8 input column blocks per workgroup)
    (512, 8192, 32, 8192 + 5, "random", 0.0),          # 16 output blocks, 32 column-block groups, 5 chunks
    (1024, 4096, 32, 16384 + 3, "concentrated", 0.05),  # every row reads blocks 0-31: 256 slots per group, 3 passes
    (256, 8192, 32, 16384 + 40, "random", 0.1),         # 8 output blocks, dead and out-of-range slots
    # B = 16: the transposed-list kernel with 16 waves (16 column blocks per workgroup)
    (1024, 8192, 16, 8192 + 5, "random", 0.0),          # 64 output blocks, 32 groups, 9 chunks
    (512, 4096, 16, 16384 + 3, "concentrated", 0.05),   # every row reads blocks 0-63: 512 slots per group, 2 passes
    (256, 4096, 16, 16384 + 40, "random", 0.1),         # 16 output blocks, dead and out-of-range slots
    # B = 16: the row-blocked kernel (16 block rows per workgroup, input rows of 512)
    (8192, 512, 16, 16384 + 9, "random", 0.05),         # 512 block rows, 8 slots each, 32 row groups x 9 chunks
])
def test_block_ell_matmul_bwd_blocked_tile_grads(gpu, case):
    """Tile gradients through the blocked kernels (transposed lists of the input column blocks, or
    16 block rows per workgroup at B = 16): every tile against float32 x^T dy (bf16 inputs, exact
    products), dead and out-of-range slots zero, two calls bit-identical."""
    import torch
    out_f, in_f, B, N, topo, sf = case
    _say(f"matmul bwd blocked tile gradients {case}")
    rng = np.random.default_rng(out_f + in_f + N + B)
    R, Cb = out_f // B, in_f // B
    K = O.k_for_density(Cb, 0.25)
    if topo == "concentrated":
        col = np.stack([rng.permutation(K) for _ in range(R)]).astype(np.int32)
        vals = (rng.standard_normal((R, K, B, B)) * 0.02).astype(np.float32)
        vals = O.bf16_round(vals)
    else:
        vals, col = T.bell_weight(rng, R, Cb, K, B)
    dead = rng.random(col.shape) < sf
    col[dead] = -1
    if sf > 0:
        col[0, 0] = Cb + 3                               # out of range: a dead slot too
    x, dy = T.act(rng, N, in_f), T.act(rng, N, out_f)
    w = T.gpu_weight((vals, col))
    dx, dv = _abi_matmul_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), w)
    dx2, dv2 = _abi_matmul_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), w)
    assert torch.equal(dv, dv2) and torch.equal(dx, dx2)
    full = x.astype(np.float32).T @ dy.astype(np.float32)          # [in_f, out_f]
    got = T.to_np(dv)
    ref = np.zeros_like(got, dtype=np.float32)
    for r in range(R):
        for k in range(K):
            c = col[r, k]
            if 0 <= c < Cb:
                ref[r, k] = full[c * B:(c + 1) * B, r * B:(r + 1) * B]
    rel, ab = T.rel_err(got, ref)
    assert rel <= TOL, f"d_values: rel {rel} abs {ab}"
    live = (col >= 0) & (col < Cb)
    assert np.all(got[~live] == 0)
    rdx = O.block_ell_matmul_t(dy[:64].astype(np.float64), vals.astype(np.float64), col, Cb)
    rel, ab = T.rel_err(T.to_np(dx)[:64], rdx)
    assert rel <= TOL, f"dx (first 64 rows): rel {rel} abs {ab}"


def test_block_ell_matmul_bwd_optional_outputs_and_no_tiles(gpu):
    """Either output may be skipped; a weight whose slots are all dead gives dx = 0."""
    import torch
    _say("matmul bwd optional outputs")
    rng = np.random.default_rng(8)
    vals, col = T.bell_weight(rng, 8, 8, 4, 16)
    x, dy = T.act(rng, 50, 128), T.act(rng, 50, 128)
    w = T.gpu_weight((vals, col))
    dx, dv = _abi_matmul_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), w)
    dx2, none = _abi_matmul_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), w, want_dv=False)
    none2, dv2 = _abi_matmul_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), w, want_dx=False)
    assert none is None and none2 is None
    assert torch.equal(dx, dx2) and torch.equal(dv, dv2)
    dead = (w[0], torch.full_like(w[1], -1))
    dx3, dv3 = _abi_matmul_bwd(T.to_gpu_bf16(dy), T.to_gpu_bf16(x), dead)
    assert torch.count_nonzero(dx3).item() == 0 and torch.count_nonzero(dv3).item() == 0


def test_block_ell_linear_autograd_matches_dense_fp32(gpu):
    """BlockELLLinear (bias, one pruned tile) trained through titan::block_ell_matmul_bwd: the
    gradients of x, the tiles and the bias match a dense float32 torch reference; the
    reference's gradient-flow test (non-zero tile gradients of the right shape) holds."""
    import torch
    from looped_blockell.layers import BlockELLLinear
    _say("BlockELLLinear autograd")
    torch.manual_seed(4)
    lin = BlockELLLinear(96, 128, tile_size=16, density=0.5, device="cuda")
    with torch.no_grad():
        lin.bias.copy_(torch.randn(96, device="cuda") * 0.1)
    lin.alive_mask[1, 2] = False
    x = torch.randn(3, 7, 128, device="cuda").requires_grad_(True)
    y = lin(x)
    gy = torch.randn_like(y.float())
    y.float().backward(gy)
    # dense fp32 reference on the same bf16-rounded operands
    vals = lin.values.detach().to(torch.bfloat16).float().cpu().numpy()
    col = lin.effective_col_indices().cpu().numpy()
    W = torch.from_numpy(O.block_ell_to_dense(vals, col, 96, 128)).requires_grad_(True)
    xr = x.detach().to(torch.bfloat16).float().cpu().requires_grad_(True)
    br = lin.bias.detach().float().cpu().requires_grad_(True)
    yr = xr @ W.T + br
    gyr = gy.to(torch.bfloat16).float().cpu()
    yr.backward(gyr)
    assert T.rel_err(T.to_np(y.detach().float()), yr.detach().numpy())[0] <= TOL
    assert T.rel_err(T.to_np(x.grad), xr.grad.numpy())[0] <= TOL
    assert T.rel_err(T.to_np(lin.bias.grad), br.grad.numpy())[0] <= TOL
    ref_tiles = O.dense_to_block_ell(W.grad.numpy(), 16)[0]                  # [R, C, B_in, B_out]
    got = T.to_np(lin.values.grad)
    for r in range(lin.R):
        for k in range(lin.K):
            c = col[r, k]
            ref = ref_tiles[r, c] if c >= 0 else np.zeros((16, 16), np.float32)
            assert T.rel_err(got[r, k], ref)[1] <= TOL * max(np.abs(ref_tiles).max(), 1e-30)
    assert lin.values.grad.shape == lin.values.shape and torch.count_nonzero(lin.values.grad).item() > 0
    assert torch.count_nonzero(lin.values.grad[1, 2]).item() == 0


def test_gelu_mlpblock_backward_runs(gpu):
    """MLPBlock(use_swiglu=False): both Block-ELL products are differentiable; the gradients of
    x match a float32 torch recomputation with the same tiles."""
    import torch
    import torch.nn.functional as F
    from looped_blockell.layers import MLPBlock
    _say("GELU MLPBlock autograd")
    torch.manual_seed(6)
    m = MLPBlock(128, 256, use_swiglu=False, tile_size=32, density=0.5, device="cuda")
    x = torch.randn(40, 128, device="cuda").to(torch.bfloat16).requires_grad_(True)
    y = m(x)
    gy = torch.randn_like(y.float())
    y.float().backward(gy)

    def dense(lin):
        v = lin.values.detach().to(torch.bfloat16).float().cpu().numpy()
        return torch.from_numpy(O.block_ell_to_dense(v, lin.effective_col_indices().cpu().numpy(), lin.out_features,
                                                     lin.in_features))

    W1, W2 = dense(m.fc1), dense(m.fc2)
    xr = x.detach().float().cpu().requires_grad_(True)
    h = F.gelu(xr @ W1.T + m.fc1.bias.detach().float().cpu())
    yr = h.to(torch.bfloat16).float() @ W2.T + m.fc2.bias.detach().float().cpu()
    yr.backward(gy.to(torch.bfloat16).float().cpu())
    assert T.rel_err(T.to_np(x.grad), xr.grad.numpy())[0] <= 3 * TOL
    for lin in (m.fc1, m.fc2):
        assert lin.values.grad is not None and torch.count_nonzero(lin.values.grad).item() > 0
        assert lin.bias.grad is not None


@pytest.mark.parametrize("case", [
    # (d_model, d_ff, N, sentinel_frac, B)
    (1024, 4096, 16384, 0.0, 32),          # the headline shape
    (512, 4096, 16384 + 37, 0.1, 32),      # 16 input column blocks, dead slots, a ragged last token chunk
    (1024, 4096, 16384 + 5, 0.05, 16),     # the headline geometry at B = 16 (the blocked tile gradients)
    (768, 4096, 16384, 0.0, 32),           # 24 input column blocks: a width the row-blocked kernel has no form for
])
def test_swiglu_bwd_full_size_sampled(gpu, case):
    """Full token counts (the tile gradients take the blocked kernels from 256 workgroups on),
    saved tensors from the GPU forward: dx checked on sampled token rows (a row of dx depends only
    on that row), the tile gradients on sampled tiles (each a sum over all the tokens, recomputed in
    float64 from the same saved tensors; dead slots zero); two calls agree bit for bit."""
    import torch
    d_model, d_ff, N, frac, B = case
    _say(f"full size d_model={d_model} d_ff={d_ff} B={B} N={N} sentinel {frac} (sampled)")
    rng = np.random.default_rng(2024 + d_model)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25, sentinel_frac=frac)
    x, dy = T.act(rng, N, d_model), T.act(rng, N, d_model)
    gw, uw, dw = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    x_t, dy_t = T.to_gpu_bf16(x), T.to_gpu_bf16(dy)
    _, h_t, gp_t, uo_t = T.abi_swiglu(x_t, gw, uw, dw, add_residual=True, intermediates=True)
    got = T.abi_swiglu_bwd(dy_t, x_t, gp_t, uo_t, h_t, gw, uw, dw)
    again = T.abi_swiglu_bwd(dy_t, x_t, gp_t, uo_t, h_t, gw, uw, dw)
    for a_, b_ in zip(got, again):
        assert torch.equal(a_, b_)
    gp, uo, h = (T.to_np(t) for t in (gp_t, uo_t, h_t))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    # dx on sampled rows
    rows = np.sort(rng.choice(N, 96, replace=False))
    rdx = O.swiglu_bwd(dy[rows], x[rows], gp[rows], uo[rows], h[rows], f64(g), f64(u), f64(d))[0]
    rel, ab = T.rel_err(T.to_np(got[0])[rows], rdx)
    assert rel <= TOL, f"dx rows: rel {rel} abs {ab}"
    # tile gradients on sampled tiles
    Wd, dcol = d[0].astype(np.float64), d[1]

    def dh_block(r):            # dh[:, r-th d_ff block] = sum over down slots reading it of dy[:, rm] Wd^T
        out = np.zeros((N, B))
        for rm, kk in zip(*np.nonzero(dcol == r)):
            out += dy[:, rm * B:(rm + 1) * B].astype(np.float64) @ Wd[rm, kk].T
        return out

    def check(name, got_t, col, ref_tile):
        R, K = col.shape
        picks = [(int(r), int(k)) for r, k in zip(rng.integers(0, R, 12), rng.integers(0, K, 12))]
        gt = T.to_np(got_t)
        refs = [ref_tile(r, k) if col[r, k] >= 0 else np.zeros((B, B)) for r, k in picks]
        den = max(np.abs(np.stack(refs)).max(), 1e-30)
        picks += [(int(r), int(k)) for r, k in zip(*np.nonzero(col < 0))][:4]   # dead slots
        refs += [np.zeros((B, B))] * (len(picks) - len(refs))
        for (r, k), ref in zip(picks, refs):
            err = np.abs(gt[r, k] - ref).max() / den
            assert err <= TOL, f"{name} tile ({r},{k}): rel {err}"

    def gate_up_tile(which):
        def tile(r, k):
            c = (g if which == "gate" else u)[1][r, k]
            dh = dh_block(r)
            gg = gp[:, r * B:(r + 1) * B].astype(np.float64)
            uu = uo[:, r * B:(r + 1) * B].astype(np.float64)
            s = 1.0 / (1.0 + np.exp(-gg))
            gy = dh * uu * (s + gg * s * (1.0 - s)) if which == "gate" else dh * gg * s
            return x[:, c * B:(c + 1) * B].astype(np.float64).T @ gy
        return tile

    check("d_gate", got[1], g[1], gate_up_tile("gate"))
    check("d_up", got[2], u[1], gate_up_tile("up"))
    check("d_down", got[3], dcol,
          lambda r, k: h[:, dcol[r, k] * B:(dcol[r, k] + 1) * B].astype(np.float64).T
          @ dy[:, r * B:(r + 1) * B].astype(np.float64))
