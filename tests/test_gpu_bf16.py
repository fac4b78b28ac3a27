"""GPU parity of the bf16 Block-ELL kernels against the CPU oracle (through the C ABI).

Tolerance (bf16 path): max|y - y_ref| <= 1e-2 * max|y_ref|, y_ref the oracle
evaluated in float64 on the same bf16-rounded inputs; the absolute error is
reported in the assertion message.
"""

import numpy as np
import pytest

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("B", [16, 32, 64])
@pytest.mark.parametrize("N", [1, 5, 33, 64, 130])
def test_matmul_parity(gpu, B, N):
    rng = np.random.default_rng(100 + B + N)
    R, C_, K = 5, 7, 3
    _say(f"matmul B={B} N={N}")
    w = T.bell_weight(rng, R, C_, K, B, sentinel=[(1, 2), (4, 0)])
    x = T.act(rng, N, C_ * B)
    bias = rng.standard_normal(R * B).astype(np.float32) * 0.1
    y = T.to_np(T.abi_matmul(T.to_gpu_bf16(x), T.gpu_weight(w), T.to_gpu(bias)))
    ref = O.block_ell_matmul(x.astype(np.float64), w[0].astype(np.float64), w[1]) + bias
    rel, ab = T.rel_err(y, ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


@pytest.mark.parametrize("case", [
    # (in_features, out_features, B, K, N, path)
    (256, 512, 16, 4, 77, "panel"),
    (256, 512, 16, 5, 77, "panel"),             # odd K: the last slot pair's second half is the zero tile
    (2048, 512, 16, 9, 70, "panel"),            # the same on 32-token panels (in_features 2048)
    (1024, 4096, 32, 8, 200, "panel"),          # the headline gate shape
    (2048, 1024, 32, 8, 70, "panel"),           # 32-token panels
    (4096, 1024, 32, 32, 130, "staged"),        # the headline down shape
    (96, 64, 32, 2, 33, "staged"),              # in_features not a multiple of 128
    (4096, 512, 16, 40, 17, "staged"),
    (2048, 512, 16, 128, 300, "staged"),        # 128 slots per row: two slot chunks per lane
    (4096, 512, 16, 129, 40, "row-block"),      # beyond 128 slots
    (256, 256, 64, 2, 40, "row-block"),         # B = 64
])
def test_matmul_ws_paths(gpu, case):
    """The workspace entry's three paths against the oracle and the row-block entry, with a bias,
    dead slots and out-of-range columns."""
    fin, fout, B, K, N, path = case
    _say(f"matmul_ws {case}")
    rng = np.random.default_rng(fin + fout + B + N)
    R, C_ = fout // B, fin // B
    vals, col = T.bell_weight(rng, R, C_, K, B)
    col[0, 0] = -1
    col[R - 1, K - 1] = C_ + 3                   # out of range: skipped
    x = T.act(rng, N, fin)
    bias = (0.1 * rng.standard_normal(fout)).astype(np.float32)
    wt = (T.to_gpu_bf16(vals), T.to_gpu(col))
    y, wsb = T.abi_matmul_ws(T.to_gpu_bf16(x), wt, T.to_gpu(bias))
    assert (wsb > 0) == (path != "row-block")
    col_ref = col.copy()
    col_ref[col_ref >= C_] = -1
    ref = O.block_ell_matmul(x.astype(np.float64), vals.astype(np.float64), col_ref) + bias
    rel, ab = T.rel_err(T.to_np(y), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
    y_rb = T.abi_matmul(T.to_gpu_bf16(x), wt, T.to_gpu(bias))
    assert T.rel_err(T.to_np(y), T.to_np(y_rb).astype(np.float64))[0] <= TOL
    y2, _ = T.abi_matmul_ws(T.to_gpu_bf16(x), wt, None)      # no bias
    assert T.rel_err(T.to_np(y2), ref - bias)[0] <= TOL


def test_matmul_density_one_equals_dense(gpu):
    # reference tests/test_block_ell.py:42-54 on the GPU: Block-ELL at density 1.0 == x @ W.T
    rng = np.random.default_rng(7)
    W = O.bf16_round(rng.standard_normal((64, 128)).astype(np.float32))
    v, c, _ = O.create_block_ell_from_dense(W, tile_size=32, density=1.0)
    x = T.act(rng, 40, 128)
    y = T.to_np(T.abi_matmul(T.to_gpu_bf16(x), (T.to_gpu_bf16(v), T.to_gpu(c))))
    rel, ab = T.rel_err(y, x.astype(np.float64) @ W.T.astype(np.float64))
    assert rel <= TOL, f"rel {rel} abs {ab}"


def test_matmul_out_of_range_column_is_skipped(gpu):
    rng = np.random.default_rng(8)
    vals, col = T.bell_weight(rng, 3, 4, 2, 32)
    col[0, 1] = 4            # == C: out of range, contributes nothing
    col[2, 0] = 1000
    x = T.act(rng, 9, 128)
    y = T.to_np(T.abi_matmul(T.to_gpu_bf16(x), (T.to_gpu_bf16(vals), T.to_gpu(col))))
    col_ref = col.copy()
    col_ref[col_ref >= 4] = -1
    ref = O.block_ell_matmul(x.astype(np.float64), vals.astype(np.float64), col_ref)
    assert T.rel_err(y, ref)[0] <= TOL


SWIGLU_CASES = [
    # (d_model, d_ff, B, density, N, sentinel_frac, kernels the library picks)
    (256, 1024, 16, 0.25, 512, 0.0, "split"),      # the small CPU-runnable geometry
    (256, 1024, 16, 0.25, 77, 0.1, "split"),       # ragged N, dead slots
    (512, 1024, 32, 0.25, 130, 0.0, "split"),
    (512, 256, 32, 0.5, 90, 0.1, "split"),         # 8 h rows: fewer than the 12 gate/up waves
    (256, 1408, 32, 0.25, 100, 0.05, "split"),     # 44 h rows in 5 uneven row slices (few token blocks)
    (1024, 4096, 32, 0.25, 200, 0.05, "split"),    # the headline geometry, small N
    (128, 512, 64, 0.5, 70, 0.0, "rowblock"),      # B = 64 -> general row-block kernels
    (2048, 1024, 32, 0.125, 40, 0.0, "decode"),    # d_model > 1024 at decode size
    (2048, 1024, 32, 0.125, 100, 0.0, "split"),    # d_model > 1024: 32-token gate/up panels, 64 down rows
    (2048, 2048, 16, 0.125, 100, 0.05, "split"),   # 128 down rows: 16 row groups per token block
]


@pytest.mark.parametrize("case", SWIGLU_CASES)
@pytest.mark.parametrize("resid", [False, True])
def test_swiglu_parity(gpu, case, resid):
    d_model, d_ff, B, dens, N, sf, path = case
    _say(f"swiglu {case} resid={resid}")
    rng = np.random.default_rng(hash(case[:6]) % 2 ** 31)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=sf)
    x = T.act(rng, N, d_model)
    gw, uw, dw = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    assert T.swiglu_path(N, d_model, gw, uw, dw) == path
    out, *_ = T.abi_swiglu(T.to_gpu_bf16(x), gw, uw, dw, add_residual=resid)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=resid)
    rel, ab = T.rel_err(T.to_np(out), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


def _offset_bf16(a, elems):
    """A bf16 GPU copy of `a` that starts `elems` elements (2 bytes each) into a larger buffer."""
    import torch
    flat = T.to_gpu_bf16(np.asarray(a, np.float32).reshape(-1))
    buf = torch.zeros(flat.numel() + elems, dtype=torch.bfloat16, device=flat.device)
    buf[elems:] = flat
    return buf[elems:].view(*np.shape(a))


@pytest.mark.parametrize("case", [(256, 1024, 16, 0.25, 60), (1024, 4096, 32, 0.25, 70)])
def test_swiglu_weights_8_byte_aligned(gpu, case):
    """Weight values only 8-byte aligned (the ABI's minimum): the packing kernel's 8-byte loads."""
    d_model, d_ff, B, dens, N = case
    _say(f"swiglu 8-byte aligned weights {case}")
    rng = np.random.default_rng(31 + B)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=0.05)
    x = T.act(rng, N, d_model)
    w = [(_offset_bf16(v, 4), T.to_gpu(c.astype(np.int32))) for v, c in (g, u, d)]
    assert all(t[0].data_ptr() % 16 == 8 for t in w)
    out, *_ = T.abi_swiglu(T.to_gpu_bf16(x), *w, add_residual=True)
    f64 = lambda w_: (w_[0].astype(np.float64), w_[1])
    ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
    rel, ab = T.rel_err(T.to_np(out), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
    aligned, *_ = T.abi_swiglu(T.to_gpu_bf16(x), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d),
                               add_residual=True)
    assert np.array_equal(T.to_np(out), T.to_np(aligned))     # same packed tiles, same result


@pytest.mark.parametrize("case", [(256, 1024, 16, 0.25, 100), (1024, 4096, 32, 0.25, 64), (128, 256, 64, 1.0, 33)])
def test_swiglu_with_intermediates(gpu, case):
    d_model, d_ff, B, dens, N = case
    _say(f"swiglu intermediates {case}")
    rng = np.random.default_rng(11)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens)
    x = T.act(rng, N, d_model)
    out, h, gp, uo = T.abi_swiglu(T.to_gpu_bf16(x), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d),
                                  add_residual=False, intermediates=True)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, h_ref, g_ref, u_ref = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d))
    for got, want, name in ((out, ref, "out"), (h, h_ref, "h"), (gp, g_ref, "gate"), (uo, u_ref, "up")):
        rel, ab = T.rel_err(T.to_np(got), want)
        assert rel <= TOL, f"{name}: rel {rel} abs {ab}"


@pytest.mark.parametrize("Kd", [63, 64, 65, 127, 128, 129])
@pytest.mark.parametrize("case", [(256, 1024, 16), (128, 512, 16), (1024, 4096, 32)])
def test_swiglu_duplicate_and_empty_columns(gpu, case, Kd):
    """Rows that name one column block several times sum every copy (as the oracle's
    per-slot sum does); a down row whose slots all fall in the first LDS stage
    gives that stage a full hit list; empty rows give zeros.  Kd <= 64 runs the
    two-kernel split path with one slot per lane, Kd <= 128 with two, Kd = 129 the row-block
    path."""
    d_model, d_ff, B = case
    _say(f"swiglu duplicate columns {case} Kd={Kd}")
    rng = np.random.default_rng(21)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    g[1][0, :] = g[1][0, 0]                      # every gate slot of row 0 -> one column
    u[1][1, :] = -1                              # up row 1 empty -> h row block 1 == 0
    Cf = d_ff // B
    dv = O.bf16_round((rng.standard_normal((d_model // B, Kd, B, B)) * 0.02).astype(np.float32))
    dc = rng.integers(0, Cf, size=(d_model // B, Kd)).astype(np.int32)
    dc[0, :] = rng.integers(0, min(Cf, 256 // B), size=Kd)   # row 0: all slots in the first stage
    d = (dv, dc)
    x = T.act(rng, 70, d_model)
    gw, uw, dw = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    assert T.swiglu_path(70, d_model, gw, uw, dw) == ("split" if Kd <= 128 else "rowblock")
    out, *_ = T.abi_swiglu(T.to_gpu_bf16(x), gw, uw, dw, add_residual=True)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
    rel, ab = T.rel_err(T.to_np(out), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


@pytest.mark.parametrize("N", [8192 + 5, 300])
@pytest.mark.parametrize("geom", [(512, 2048, 1.0), (2048, 8192, 0.25)])
def test_reference_default_layer_geometry(gpu, geom, N):
    """The reference's default tile-16 layer on the two-kernel path at its ablation geometry
    (configs/ablation.yaml: d_model 512, d_ff 2048, initial density 1.0 -> K_gate = 32, K_down =
    128) and at its large geometry pruned to 25 % (configs/large.yaml: d_model 2048, d_ff 8192 ->
    K_gate = 32, K_down = 128, 16384-entry gate/up column tables, 32-token gate/up panels): the
    down kernel with two slot chunks per lane and two rows per wave (8192 + 5 tokens), rows 0 and 1
    (one wave's) with all 128 slots in the first stage (258 list positions), and the fewer-token
    shapes (300 tokens)."""
    d_model, d_ff, dens = geom
    B = 16
    _say(f"reference default layer d{d_model} ff{d_ff} B16 density {dens} N={N}")
    rng = np.random.default_rng(d_model + N)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens)
    assert d[1].shape[1] == 128 and g[1].shape[1] == 32
    dc = d[1]
    dc[0, :] = rng.integers(0, 512 // B, size=128)          # all in the first 512-column stage
    dc[1, :] = rng.integers(0, 512 // B, size=128)
    dc[5, 3] = -1                                           # a dead slot
    x = T.act(rng, N, d_model)
    gw, uw, dw = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    assert T.swiglu_path(N, d_model, gw, uw, dw) == "split"
    out = T.to_np(T.abi_swiglu(T.to_gpu_bf16(x), gw, uw, dw, add_residual=True)[0])
    rows = np.concatenate([np.sort(rng.choice(N, min(N, 160), replace=False)), [0, N - 1]])
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x[rows].astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
    rel, ab = T.rel_err(out[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


@pytest.mark.parametrize("case", [(1024, 4096, 32, 4096 + 5), (512, 1024, 16, 300), (1024, 2048, 32, 70),
                                  # B = 16 with 5 slots per row (slot pairs, the last one half zero);
                                  # 16389 tokens take the one-slice 12-wave kernel
                                  (320, 1024, 16, 300), (320, 1024, 16, 16384 + 5)])
@pytest.mark.parametrize("intermediates", [False, True])
def test_swiglu_shared_topology(gpu, case, intermediates):
    """Gate and up passing one column-index buffer (the shared-topology gate/up kernel, one
    panel read for both products) give the same bits as the same topology in two buffers,
    and match the oracle; covers the intermediates and the looped block too."""
    d_model, d_ff, B, N = case
    _say(f"swiglu shared topology {case} intermediates={intermediates}")
    rng = np.random.default_rng(23)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25, sentinel_frac=0.1)
    u = (u[0], g[1].copy())
    x = T.act(rng, N, d_model)
    xt = T.to_gpu_bf16(x)
    gt, ut, dt = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    shared_u = (ut[0], gt[1])                     # the same buffer as gate's indices
    r_sep = T.abi_swiglu(xt, gt, ut, dt, add_residual=True, intermediates=intermediates)
    r_sh = T.abi_swiglu(xt, gt, shared_u, dt, add_residual=True, intermediates=intermediates)
    for a, b in zip(r_sep, r_sh):
        if a is not None:
            assert np.array_equal(T.to_np(a), T.to_np(b))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
    rel, ab = T.rel_err(T.to_np(r_sh[0]), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


@pytest.mark.parametrize("geom", [(1024, 4096, 32), (512, 2048, 16)])
def test_looped_shared_topology(gpu, geom):
    """The looped block with gate and up sharing one index buffer equals the same topology in
    two buffers, bit for bit; at B = 16 the shared topology takes the slot-pair gate/up form (in
    the persistent kernel on the panel its down phase writes), the two buffers the single-slot
    form, in both looped forms."""
    from looped_blockell import kernels
    import torch
    rng = np.random.default_rng(24)
    d_model, d_ff, B = geom
    N = 1000
    _say(f"looped shared topology {geom}")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    u = (u[0], g[1].copy())
    gt, ut, dt = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    h = T.to_gpu_bf16(T.act(rng, N, d_model))
    scale = torch.ones(d_model, device="cuda")
    forms = [kernels.looped_swiglu]
    if B == 16:
        forms += [kernels.looped_swiglu_persistent, kernels.looped_swiglu_launches]
    for f in forms:
        a = f(h, scale, *gt, *ut, *dt, L=3)
        b = f(h, scale, *gt, ut[0], gt[1], *dt, L=3)
        assert np.array_equal(T.to_np(a), T.to_np(b)), f.__name__


def test_swiglu_zero_k(gpu):
    """K = 0 everywhere: h == 0, so out == x (with the residual) / 0 (without)."""
    rng = np.random.default_rng(22)
    d_model, d_ff, B = 256, 512, 16
    z = lambda R: (np.zeros((R, 0, B, B), np.float32), np.zeros((R, 0), np.int32))
    x = T.act(rng, 40, d_model)
    out, h, _, _ = T.abi_swiglu(T.to_gpu_bf16(x), T.gpu_weight(z(d_ff // B)), T.gpu_weight(z(d_ff // B)),
                                T.gpu_weight(z(d_model // B)), add_residual=True, intermediates=True)
    assert np.array_equal(T.to_np(out), x)
    assert not T.to_np(h).any()


def test_swiglu_full_headline_sampled_rows(gpu):
    """The headline FFN (d_model 1024, d_ff 4096, B 32, density 0.25) at its full 16384 tokens; rows are
    independent, so sampled rows are checked."""
    rng = np.random.default_rng(1002)
    d_model, d_ff, B, N = 1024, 4096, 32, 16384
    _say("swiglu d1024 ff4096 B32 N16384 full size")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    x = T.act(rng, N, d_model)
    out, *_ = T.abi_swiglu(T.to_gpu_bf16(x), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d))
    out = T.to_np(out)
    rows = np.sort(rng.choice(N, 384, replace=False))
    rows = np.concatenate([rows, [0, N - 1]])
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x[rows].astype(np.float64), f64(g), f64(u), f64(d))
    rel, ab = T.rel_err(out[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
    assert np.isfinite(out).all()


@pytest.mark.parametrize("case", [
    # (d_model, d_ff, density, N, sentinel_frac, residual, biases, prepacked)
    (640, 4352, 0.27, 8192 + 7, 0.15, True, False, False),   # 20 down rows, 136 column blocks
    (1024, 4096, 0.25, 16384 - 40, 0.0, False, True, True),  # headline geometry, biases, prepacked
])
def test_swiglu_deep_ring_down_sampled_rows(gpu, case):
    """The B = 32 down kernel of the large-token forward (a ring over each row's slots across the
    512-column h stages): a second row group with 4 of its 16 waves holding rows, a last stage of
    8 column blocks, 36 slots per row with dead slots, a row with no live slot, a column past the
    end, a ragged last token block; biases through the prepacked forward.  Sampled rows against the
    fp64 oracle."""
    import torch
    from looped_blockell import kernels
    d_model, d_ff, dens, N, frac, resid, biases, prepacked = case
    B = 32
    _say(f"swiglu deep-ring down {case}")
    rng = np.random.default_rng(2024 + d_model)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=frac)
    if frac:
        d[1][3, :] = -1                       # a down row with no live slot
        d[1][5, 0] = d_ff // B + 2            # past the last column block: skipped
    x = T.act(rng, N, d_model)
    bs = [None, None, None]
    if biases:
        bs = [rng.standard_normal(n).astype(np.float32) * 0.1 for n in (d_ff, d_ff, d_model)]
    xg = T.to_gpu_bf16(x)
    wg, wu, wd = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    if prepacked or biases:
        pk = kernels.swiglu_prepack(*wg, *wu, *wd)
        bt = [None if b is None else torch.as_tensor(b, device="cuda") for b in bs]
        out = kernels.swiglu_fwd_prepacked(xg, pk, *wg, *wu, *wd, add_residual=resid, b_gate=bt[0], b_up=bt[1],
                                           b_down=bt[2])
    else:
        out, *_ = T.abi_swiglu(xg, wg, wu, wd, add_residual=resid)
    out = T.to_np(out)
    rows = np.concatenate([np.sort(rng.choice(N, 256, replace=False)), np.arange(N - 8, N), [0]])
    # the kernels skip a column past the end as they skip -1: the reference takes it as -1
    d_ref = (d[0], np.where(d[1] < d_ff // B, d[1], -1))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x[rows].astype(np.float64), f64(g), f64(u), f64(d_ref), add_residual=resid,
                           biases=tuple(None if b is None else b.astype(np.float64) for b in bs))
    rel, ab = T.rel_err(out[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
    assert np.isfinite(out).all()


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("biases", [False, True])
def test_swiglu_b16_wide_panel_sampled_rows(gpu, shared, biases):
    """B = 16 at d_model 2048 on 8192 + 3 tokens (32-token gate/up panels, one row slice: the
    16-wave gate/up kernel) with and without a shared gate/up topology and biases, dead slots, a
    ragged last block; sampled rows against the fp64 oracle."""
    import torch
    from looped_blockell import kernels
    d_model, d_ff, B, N = 2048, 2048, 16, 8192 + 3
    _say(f"swiglu B16 d_model 2048 shared={shared} biases={biases}")
    rng = np.random.default_rng(2048 + 2 * shared + biases)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25, sentinel_frac=0.05)
    if shared:
        u = (u[0], g[1].copy())
    x = T.act(rng, N, d_model)
    bs = [rng.standard_normal(n).astype(np.float32) * 0.1 for n in (d_ff, d_ff, d_model)] if biases else [None] * 3
    xg = T.to_gpu_bf16(x)
    wg, wu, wd = T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d)
    if shared:
        wu = (wu[0], wg[1])                           # gate's column buffer: the shared-topology kernel
    pk = kernels.swiglu_prepack(*wg, *wu, *wd)
    bt = [None if b is None else torch.as_tensor(b, device="cuda") for b in bs]
    out = T.to_np(kernels.swiglu_fwd_prepacked(xg, pk, *wg, *wu, *wd, add_residual=True, b_gate=bt[0],
                                               b_up=bt[1], b_down=bt[2]))
    rows = np.concatenate([np.sort(rng.choice(N, 192, replace=False)), np.arange(N - 4, N), [0]])
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x[rows].astype(np.float64), f64(g), f64(u), f64(d), add_residual=True,
                           biases=tuple(None if b is None else b.astype(np.float64) for b in bs))
    rel, ab = T.rel_err(out[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


def test_swiglu_b16_full_size_sampled_rows(gpu):
    """B = 16 at d_model 1024, d_ff 4096, density 0.25 (64 down slots per row) on 16384 + 5 tokens:
    one row slice per token block (the 12-wave gate/up kernel), a ragged last block; sampled rows."""
    rng = np.random.default_rng(1016)
    d_model, d_ff, B, N = 1024, 4096, 16, 16384 + 5
    _say("swiglu d1024 ff4096 B16 N16389 full size")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25, sentinel_frac=0.05)
    x = T.act(rng, N, d_model)
    out, *_ = T.abi_swiglu(T.to_gpu_bf16(x), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d), add_residual=True)
    out = T.to_np(out)
    rows = np.concatenate([np.sort(rng.choice(N, 256, replace=False)), [0, N - 1]])
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x[rows].astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
    rel, ab = T.rel_err(out[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


def test_looped_b16_full_size_sampled_rows(gpu):
    """The looped block (the operator's per-iteration launches) at B = 16 on 16384 tokens, L = 3:
    the normalising 12-wave gate/up kernel; sampled rows."""
    rng = np.random.default_rng(1017)
    d_model, d_ff, B, N, L = 512, 2048, 16, 16384, 3
    _say("looped L3 d512 ff2048 B16 N16384 full size")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    h = T.act(rng, N, d_model)
    scale = (1.0 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
    out = T.to_np(T.abi_looped(T.to_gpu_bf16(h), T.to_gpu(scale), T.gpu_weight(g), T.gpu_weight(u),
                               T.gpu_weight(d), L, 1e-5))
    rows = np.sort(rng.choice(N, 128, replace=False))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = O.looped_swiglu(h[rows].astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L=L,
                          eps=1e-5)
    rel, ab = T.rel_err(out[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


@pytest.mark.parametrize("shape", [(1024, 4096), (4096, 1024)])
def test_matmul_full_size_sampled_rows(gpu, shape):
    """The plain product at the headline gate and down shapes, 16384 tokens, through the workspace
    entry (panel and staged paths), with a bias; sampled rows against the oracle, and the
    prepacked entry bit-identical."""
    fin, fout = shape
    B, N = 32, 16384
    _say(f"matmul full size {fin}->{fout}")
    rng = np.random.default_rng(fin + 1)
    vals, col = T.bell_weight(rng, fout // B, fin // B, max(1, (fin // B) // 4), B)
    x = T.act(rng, N, fin)
    bias = (0.1 * rng.standard_normal(fout)).astype(np.float32)
    wt = (T.to_gpu_bf16(vals), T.to_gpu(col))
    y, wsb = T.abi_matmul_ws(T.to_gpu_bf16(x), wt, T.to_gpu(bias))
    assert wsb > 0
    yn = T.to_np(y)
    rows = np.concatenate([np.sort(rng.choice(N, 256, replace=False)), [0, N - 1]])
    ref = O.block_ell_matmul(x[rows].astype(np.float64), vals.astype(np.float64), col) + bias
    rel, ab = T.rel_err(yn[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
    assert np.isfinite(yn).all()


def test_swiglu_deterministic(gpu):
    rng = np.random.default_rng(5)
    g, u, d = T.ffn_weights(rng, 512, 2048, 32, 0.25)
    x = T.to_gpu_bf16(T.act(rng, 300, 512))
    ws = [T.gpu_weight(w) for w in (g, u, d)]
    a = T.to_np(T.abi_swiglu(x, *ws)[0])
    b = T.to_np(T.abi_swiglu(x, *ws)[0])
    assert np.array_equal(a, b)


LOOP_CASES = [
    # (d_model, d_ff, B, density, N, L)
    (256, 1024, 16, 0.25, 100, 3),
    (1024, 4096, 32, 0.25, 130, 8),       # the looped-block geometry
    (128, 512, 64, 0.5, 40, 2),           # general path (per-iteration launches)
    (2048, 2048, 32, 0.125, 70, 2),       # 64 down rows: 8 row groups per token block
    (1024, 4096, 32, 0.25, 16, 4),        # <= 64 tokens: RMSNorm of the state + the decode kernels
    (256, 1024, 16, 0.25, 64, 3),
    (512, 1024, 32, 0.25, 1, 2),
]


@pytest.mark.parametrize("case", LOOP_CASES)
def test_looped_parity(gpu, case):
    d_model, d_ff, B, dens, N, L = case
    _say(f"looped {case}")
    rng = np.random.default_rng(hash(case) % 2 ** 31)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens)
    h = T.act(rng, N, d_model)
    scale = (1.0 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
    out = T.abi_looped(T.to_gpu_bf16(h), T.to_gpu(scale), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d), L,
                       1e-5)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = O.looped_swiglu(h.astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L=L, eps=1e-5)
    rel, ab = T.rel_err(T.to_np(out), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


def test_looped_full_size_sampled_rows(gpu):
    """The looped block at full size (32 x 512 tokens, d_model 1024, d_ff 4096, B 32, L = 8, norm scale
    ones); sampled rows vs the oracle."""
    rng = np.random.default_rng(1004)
    d_model, d_ff, B, N, L = 1024, 4096, 32, 32 * 512, 8
    _say("looped L8 d1024 ff4096 B32 N16384 full size")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    h = T.act(rng, N, d_model)
    scale = np.ones(d_model, np.float32)
    out = T.to_np(T.abi_looped(T.to_gpu_bf16(h), T.to_gpu(scale), T.gpu_weight(g), T.gpu_weight(u),
                               T.gpu_weight(d), L, 1e-5))
    rows = np.sort(rng.choice(N, 128, replace=False))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = O.looped_swiglu(h[rows].astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L=L)
    rel, ab = T.rel_err(out[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


PERSISTENT_CASES = [
    # (d_model, d_ff, B, density, N, L, shared gate/up topology)
    (256, 1024, 16, 0.25, 100, 3, False),
    (1024, 4096, 32, 0.25, 130, 8, False),      # the looped-block geometry, ragged token tail
    (1024, 4096, 32, 0.25, 64, 2, True),
    (512, 2048, 32, 0.5, 1, 1, False),
    (384, 1536, 32, 0.25, 200, 4, False),       # 12 down rows: a partial row group
    (1024, 2048, 16, 0.25, 70, 3, False),       # 64 down rows: two row groups, norm not fused
]


@pytest.mark.parametrize("case", PERSISTENT_CASES)
def test_looped_persistent_matches_two_kernel_path(gpu, case):
    """The one-launch persistent looped block runs the same tiles in the same order as the
    per-iteration gate/up + down launches; its down phase computes the next iteration's RMSNorm
    (per-token sums of squares in another order), so the two agree to bf16 rounding, and both
    are within TOL of the oracle.  With one iteration, or two row groups (norm not fused), they
    are bit-identical above 64 tokens (at most 64, the launches run the decode kernels)."""
    d_model, d_ff, B, dens, N, L, shared = case
    _say(f"looped persistent {case}")
    rng = np.random.default_rng(abs(hash(case)) % 2 ** 31)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=0.05)
    if shared:
        u = (u[0], g[1].copy())
    h = T.act(rng, N, d_model)
    scale = (1.0 + 0.1 * rng.standard_normal(d_model)).astype(np.float32)
    ws = [T.gpu_weight(w) for w in (g, u, d)]
    if shared:
        ws[1] = (ws[1][0], ws[0][1])   # one index buffer: the shared-topology kernels
    ht, st = T.to_gpu_bf16(h), T.to_gpu(scale)
    two = T.to_np(T.abi_looped(ht, st, *ws, L, 1e-5, launches=True))
    one = T.to_np(T.abi_looped(ht, st, *ws, L, 1e-5, persistent=True))
    assert np.array_equal(two, T.to_np(T.abi_looped(ht, st, *ws, L, 1e-5)))   # the default path
    # bit-identical where the launches run the two-kernel path (above 64 tokens; at most 64 they
    # run the decode kernels, which sum the slots in another order)
    if (L == 1 or d_model // B > 32) and N > 64:
        assert np.array_equal(one, two)
    else:
        assert T.rel_err(one, two)[0] <= TOL
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = O.looped_swiglu(h.astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L=L, eps=1e-5)
    rel, ab = T.rel_err(one, ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


def test_looped_persistent_full_size_and_in_place(gpu):
    """The persistent looped block at full size (32 x 512 tokens, L = 8) on sampled rows, and
    called in place (h_out = h_in)."""
    import torch
    rng = np.random.default_rng(1004)
    d_model, d_ff, B, N, L = 1024, 4096, 32, 32 * 512, 8
    _say("looped persistent L8 d1024 ff4096 B32 N16384 full size")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    h = T.act(rng, N, d_model)
    scale = np.ones(d_model, np.float32)
    ws = [T.gpu_weight(w) for w in (g, u, d)]
    ht, st = T.to_gpu_bf16(h), T.to_gpu(scale)
    two = T.abi_looped(ht, st, *ws, L, 1e-5, launches=True)
    inplace = ht.clone()
    T.abi_looped(inplace, st, *ws, L, 1e-5, persistent=True, out=inplace)
    again = T.abi_looped(ht, st, *ws, L, 1e-5, persistent=True)
    assert torch.equal(inplace, again)                       # in place == out of place, deterministic
    assert T.rel_err(T.to_np(inplace), T.to_np(two))[0] <= TOL
    rows = np.sort(rng.choice(N, 128, replace=False))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = O.looped_swiglu(h[rows].astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L=L)
    rel, ab = T.rel_err(T.to_np(inplace)[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


def test_looped_persistent_rejects_other_shapes(gpu):
    """Shapes outside the persistent kernel's (B = 64, d_model > 1024) are refused, not run."""
    import ctypes
    A = T.abi()
    rng = np.random.default_rng(5)
    for (dm, dff, B) in [(128, 512, 64), (2048, 2048, 32)]:
        g, u, d = T.ffn_weights(rng, dm, dff, B, 0.25)
        ws = [T.gpu_weight(w) for w in (g, u, d)]
        with pytest.raises(RuntimeError, match="inconsistent shapes"):
            T.abi_looped(T.to_gpu_bf16(T.act(rng, 8, dm)), T.to_gpu(np.ones(dm, np.float32)), *ws, 2, 1e-5,
                         persistent=True)


def test_looped_L0_and_L1(gpu):
    rng = np.random.default_rng(9)
    g, u, d = T.ffn_weights(rng, 256, 1024, 16, 0.25)
    h = T.act(rng, 20, 256)
    scale = np.ones(256, np.float32)
    ws = [T.gpu_weight(w) for w in (g, u, d)]
    o0 = T.to_np(T.abi_looped(T.to_gpu_bf16(h), T.to_gpu(scale), *ws, 0, 1e-5))
    assert np.array_equal(o0, h)
    o1 = T.to_np(T.abi_looped(T.to_gpu_bf16(h), T.to_gpu(scale), *ws, 1, 1e-5))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref = h + O.swiglu_fwd(O.rmsnorm(h.astype(np.float64), np.ones(256)), f64(g), f64(u), f64(d))[0]
    assert T.rel_err(o1, ref)[0] <= TOL


DECODE_CASES = [
    # (d_model, d_ff, B, density, N, sentinel_frac)   N <= 64: the decode kernels
    # (at most 32 down slots per row)
    (256, 1024, 16, 0.25, 16, 0.0),
    (512, 1024, 32, 0.25, 5, 0.1),
    (1024, 2048, 64, 0.25, 1, 0.0),
    (1024, 3072, 64, 0.125, 16, 0.1),
    (128, 512, 64, 1.0, 9, 0.0),
    (256, 2048, 16, 0.25, 8, 0.1),      # 32 down slots per row: four slots per wave
    (1024, 4096, 32, 0.25, 16, 0.05),   # the headline geometry at 16 tokens (32 down slots)
    (1024, 4096, 32, 0.25, 64, 0.0),    # four 16-token tiles
    (512, 1024, 32, 0.25, 33, 0.1),     # three tiles' worth: four tiles, the last ones partial
    (256, 1024, 16, 0.25, 20, 0.05),    # two tiles
    (1024, 3072, 64, 0.125, 47, 0.1),   # B = 64, four tiles
    (256, 4096, 16, 0.25, 8, 0.1),      # 64 down slots per row: beyond the kernels' 32, other path
]


@pytest.mark.parametrize("case", DECODE_CASES)
@pytest.mark.parametrize("resid", [False, True])
def test_decode_parity(gpu, case, resid):
    d_model, d_ff, B, dens, N, sf = case
    _say(f"decode {case} resid={resid}")
    rng = np.random.default_rng(hash(case) % 2 ** 31 + 3)
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, dens, sentinel_frac=sf)
    x = T.act(rng, N, d_model)
    out, *_ = T.abi_swiglu(T.to_gpu_bf16(x), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d), add_residual=resid)
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=resid)
    rel, ab = T.rel_err(T.to_np(out), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"


def test_decode_duplicates_and_workspace_reuse(gpu):
    """Duplicate down columns, one workspace reused by consecutive calls, and bitwise
    determinism of the decode kernels."""
    import torch
    A = T.abi()
    lib = A.load()
    rng = np.random.default_rng(31)
    d_model, d_ff, B, N = 512, 2048, 64, 16
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    d[1][0, :] = d[1][0, 0]
    ws_t = [T.gpu_weight(w) for w in (g, u, d)]
    gb, ub, db = (T.bell_struct(*w) for w in ws_t)
    wsb = lib.lbk_swiglu_workspace_bytes(N, d_model, T.C.byref(gb), T.C.byref(ub), T.C.byref(db), 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    outs = []
    for trial in range(3):
        x = T.act(rng, N, d_model) if trial < 2 else xs
        if trial == 0:
            xs = x
        xt = T.to_gpu_bf16(x)
        out = torch.empty(N, d_model, dtype=torch.bfloat16, device="cuda")
        A.check(lib.lbk_swiglu_fwd_bf16(T.ptr(xt), N, d_model, T.C.byref(gb), T.C.byref(ub), T.C.byref(db), 1,
                                        T.ptr(out), None, None, None, T.ptr(ws), wsb, T.stream()), "decode")
        ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
        rel, ab = T.rel_err(T.to_np(out), ref)
        assert rel <= TOL, f"trial {trial}: rel {rel} abs {ab}"
        outs.append(T.to_np(out))
    assert np.array_equal(outs[0], outs[2])


def test_decode_full_geometry(gpu):
    """The decode geometry: 16 tokens, d_model 4096, d_ff 14336, B 64, density 0.10."""
    rng = np.random.default_rng(1005)
    d_model, d_ff, B, N = 4096, 14336, 64, 16
    _say("decode N16 d4096 ff14336 B64 full size")
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.10)
    x = T.act(rng, N, d_model)
    out, *_ = T.abi_swiglu(T.to_gpu_bf16(x), T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    ref, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d))
    rel, ab = T.rel_err(T.to_np(out), ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
