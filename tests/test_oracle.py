"""Pins for the CPU oracle (oracle/oracle.py).

Each test checks one oracle function against something the oracle's own formula
does not restate: the reference's test invariants and known answers, closed
forms, or brute-force scalar loops on tiny inputs.  Planted-mistake tests at
the end show that the checks would catch a transposed tile, a dropped block or
a wrong rounding mode.
"""

import math

import numpy as np
import pytest

from oracle import oracle as O


def rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- format

def test_config_properties_known_answers():
    # reference tests/test_block_ell.py:17-22
    cfg = O.BlockELLConfig(R=4, C=8, K=3, B=16)
    assert cfg.out_features == 64
    assert cfg.in_features == 128
    assert cfg.density == 0.375
    assert cfg.total_blocks == 12


def test_config_validation():
    with pytest.raises(ValueError):
        O.BlockELLConfig(R=1, C=2, K=3, B=16)
    with pytest.raises(ValueError):
        O.BlockELLConfig(R=0, C=2, K=1, B=16)


def test_k_for_density():
    # reference looped_blockell/layers/mlp.py:44 and tests/test_block_ell.py:75-88
    assert O.k_for_density(32, 0.25) == 8
    assert O.k_for_density(128, 0.25) == 32
    assert O.k_for_density(32, 0.125) == 4
    assert O.k_for_density(64, 0.10) == 6
    assert O.k_for_density(224, 0.10) == 22
    assert O.k_for_density(3, 0.1) == 1
    assert O.k_for_density(6, 0.5) < O.k_for_density(6, 1.0)


def test_random_topology_unique_unsorted():
    # reference tests/test_block_ell.py:25-31
    col = O.random_topology(64, 32, 8, rng(1))
    assert col.shape == (64, 8) and col.dtype == np.int32
    for r in range(64):
        assert len(np.unique(col[r])) == 8
    assert col.min() >= 0 and col.max() < 32
    assert any(np.any(np.diff(col[r]) < 0) for r in range(64))  # not sorted


def test_dense_to_block_ell_shapes_and_round_trip():
    # reference tests/test_interop.py:131-148
    w = rng(2).standard_normal((256, 64)).astype(np.float32)
    values, col = O.dense_to_block_ell(w, tile_size=16)
    assert values.shape == (16, 4, 16, 16)
    assert col.shape == (16, 4)
    np.testing.assert_array_equal(col, np.tile(np.arange(4, dtype=np.int32), (16, 1)))
    back = O.block_ell_to_dense(values, col, 256, 64)
    np.testing.assert_allclose(back, w, atol=1e-6)


def test_tile_orientation_special_case():
    # A single tile whose [B_in, B_out] entry (d=1, D=3) is 1 must land at dense[out=3, in=c*B+1].
    B = 4
    values = np.zeros((1, 1, B, B), dtype=np.float32)
    values[0, 0, 1, 3] = 1.0
    col = np.array([[2]], dtype=np.int32)
    dense = O.block_ell_to_dense(values, col, B, 3 * B)
    expect = np.zeros((B, 3 * B), dtype=np.float32)
    expect[3, 2 * B + 1] = 1.0
    np.testing.assert_array_equal(dense, expect)


def test_from_dense_round_trip_and_topk():
    # reference tests/test_block_ell.py:34-39
    w = rng(3).standard_normal((64, 128)).astype(np.float32)
    v, c, cfg = O.create_block_ell_from_dense(w, tile_size=16, density=1.0)
    np.testing.assert_allclose(O.block_ell_to_dense(v, c, 64, 128), w, atol=1e-5)
    # hand-built: row 0 has big tiles at columns 3 and 1; density 0.5 of C=4 -> K=2
    w = np.full((16, 64), 0.01, dtype=np.float32)
    w[:, 48:64] = 5.0
    w[:, 16:32] = 2.0
    v, c, cfg = O.create_block_ell_from_dense(w, tile_size=16, density=0.5)
    assert cfg.K == 2
    np.testing.assert_array_equal(c, [[1, 3]])       # sorted
    np.testing.assert_array_equal(v[0, 1], np.full((16, 16), 5.0, dtype=np.float32))


# ---------------------------------------------------------------- matmul

def brute_matmul(x, values, col):
    n, F = x.shape
    R, K, B, _ = values.shape
    y = np.zeros((n, R * B))
    for t in range(n):
        for r in range(R):
            for k in range(K):
                c = col[r, k]
                if c < 0:
                    continue
                for d in range(B):
                    xv = x[t, c * B + d]
                    for D in range(B):
                        y[t, r * B + D] += xv * values[r, k, d, D]
    return y


def test_matmul_matches_dense_at_density_one():
    # reference tests/test_block_ell.py:42-54
    g = rng(4)
    W = g.standard_normal((32, 64))
    x = g.standard_normal((2, 8, 64))
    v, c, _ = O.create_block_ell_from_dense(W, tile_size=16, density=1.0)
    np.testing.assert_allclose(O.block_ell_matmul(x, v, c), x @ W.T, atol=1e-10)


def test_matmul_matches_dense_expansion_sparse():
    g = rng(5)
    R, C, K, B = 6, 5, 2, 8
    values = g.standard_normal((R, K, B, B))
    col = O.random_topology(R, C, K, g)
    x = g.standard_normal((7, C * B))
    W = O.block_ell_to_dense(values, col, R * B, C * B)
    np.testing.assert_allclose(O.block_ell_matmul(x, values, col), x @ W.T, atol=1e-10)


def test_matmul_brute_force_with_sentinel():
    g = rng(6)
    R, C, K, B = 3, 4, 3, 4
    values = g.standard_normal((R, K, B, B))
    col = O.random_topology(R, C, K, g)
    col[1, 2] = -1
    col[2, :] = -1
    x = g.standard_normal((5, C * B))
    y = O.block_ell_matmul(x, values, col, chunk=2)
    np.testing.assert_allclose(y, brute_matmul(x, values, col), atol=1e-10)
    assert np.all(y[:, 2 * B:3 * B] == 0)


def test_matmul_identity_tiles_gather():
    B, C = 4, 3
    values = np.tile(np.eye(B)[None, None], (2, 1, 1, 1))
    col = np.array([[2], [0]], dtype=np.int32)
    x = np.arange(2 * C * B, dtype=np.float64).reshape(2, C * B)
    y = O.block_ell_matmul(x, values, col)
    np.testing.assert_array_equal(y[:, :B], x[:, 2 * B:3 * B])
    np.testing.assert_array_equal(y[:, B:], x[:, :B])


def test_matmul_linearity():
    g = rng(7)
    values = g.standard_normal((4, 2, 8, 8))
    col = O.random_topology(4, 3, 2, g)
    x1, x2 = g.standard_normal((3, 24)), g.standard_normal((3, 24))
    a = O.block_ell_matmul(2.0 * x1 - 3.0 * x2, values, col)
    b = 2.0 * O.block_ell_matmul(x1, values, col) - 3.0 * O.block_ell_matmul(x2, values, col)
    np.testing.assert_allclose(a, b, atol=1e-10)


# ---------------------------------------------------------------- SwiGLU / norm / loop

def test_silu_closed_forms():
    assert O.silu(np.array(0.0)) == 0.0
    z = np.linspace(-8, 8, 33)
    np.testing.assert_allclose(O.silu(z) - O.silu(-z), z, atol=1e-12)
    np.testing.assert_allclose(O.silu(np.array([1.0])), [1.0 / (1.0 + math.exp(-1.0))], rtol=1e-15)


def test_swiglu_brute_dense():
    g = rng(8)
    B, dm, dff = 4, 12, 16
    Cm, Cf = dm // B, dff // B
    Rf, Rm = dff // B, dm // B
    gate = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, Cm, 2, g))
    up = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, Cm, 2, g))
    down = (g.standard_normal((Rm, 3, B, B)), O.random_topology(Rm, Cf, 3, g))
    x = g.standard_normal((5, dm))
    Wg = O.block_ell_to_dense(*gate, dff, dm)
    Wu = O.block_ell_to_dense(*up, dff, dm)
    Wd = O.block_ell_to_dense(*down, dm, dff)
    a, b = x @ Wg.T, x @ Wu.T
    h = a / (1 + np.exp(-a)) * b
    out, h2, g2, u2 = O.swiglu_fwd(x, gate, up, down, add_residual=True)
    np.testing.assert_allclose(out, h @ Wd.T + x, atol=1e-10)
    np.testing.assert_allclose(h2, h, atol=1e-12)
    out0, *_ = O.swiglu_fwd(x, gate, up, down, add_residual=False)
    np.testing.assert_allclose(out - out0, x, atol=1e-12)


def test_swiglu_biases_brute_dense():
    """The biased SwiGLU (each projection adds its bias, reference mlp.py:82) against dense math;
    a planted mistake (the up bias added after the product) is caught."""
    g = rng(81)
    B, dm, dff = 4, 12, 16
    Cm, Cf, Rf, Rm = dm // B, dff // B, dff // B, dm // B
    gate = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, Cm, 2, g))
    up = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, Cm, 2, g))
    down = (g.standard_normal((Rm, 3, B, B)), O.random_topology(Rm, Cf, 3, g))
    bg, bu, bd = g.standard_normal(dff), g.standard_normal(dff), g.standard_normal(dm)
    x = g.standard_normal((5, dm))
    Wg, Wu, Wd = (O.block_ell_to_dense(*gate, dff, dm), O.block_ell_to_dense(*up, dff, dm),
                  O.block_ell_to_dense(*down, dm, dff))
    a, b = x @ Wg.T + bg, x @ Wu.T + bu
    h = a / (1 + np.exp(-a)) * b
    out, h2, g2, u2 = O.swiglu_fwd(x, gate, up, down, add_residual=True, biases=(bg, bu, bd))
    np.testing.assert_allclose(out, h @ Wd.T + bd + x, atol=1e-10)
    np.testing.assert_allclose(g2, a, atol=1e-12)
    np.testing.assert_allclose(u2, b, atol=1e-12)
    wrong = (a / (1 + np.exp(-a)) * (x @ Wu.T) + bu) @ Wd.T + bd + x
    assert np.abs(wrong - out).max() > 1e-3
    # only some biases
    out_g, *_ = O.swiglu_fwd(x, gate, up, down, biases=(bg, None, None))
    np.testing.assert_allclose(out_g, (a / (1 + np.exp(-a)) * (x @ Wu.T)) @ Wd.T, atol=1e-10)


def test_gelu_tanh_closed_forms_and_torch():
    torch = pytest.importorskip("torch")
    assert O.gelu_tanh(np.array(0.0)) == 0.0
    z = np.linspace(-6, 6, 49)
    np.testing.assert_allclose(O.gelu_tanh(z) - O.gelu_tanh(-z), z, atol=1e-12)   # odd part is z/2
    np.testing.assert_allclose(O.gelu_tanh(np.array([30.0, -30.0])), [30.0, 0.0], atol=1e-12)
    ref = torch.nn.functional.gelu(torch.tensor(z, dtype=torch.float64), approximate="tanh").numpy()
    np.testing.assert_allclose(O.gelu_tanh(z), ref, atol=1e-14)
    exact = torch.nn.functional.gelu(torch.tensor(z, dtype=torch.float64)).numpy()
    assert np.abs(O.gelu_tanh(z) - exact).max() > 1e-5          # the tanh form, not the erf form


def test_gelu_mlp_brute_dense():
    g = rng(82)
    B, dm, dff = 4, 8, 16
    fc1 = (g.standard_normal((dff // B, 2, B, B)), O.random_topology(dff // B, dm // B, 2, g))
    fc2 = (g.standard_normal((dm // B, 3, B, B)), O.random_topology(dm // B, dff // B, 3, g))
    b1, b2 = g.standard_normal(dff), g.standard_normal(dm)
    x = g.standard_normal((3, dm))
    W1, W2 = O.block_ell_to_dense(*fc1, dff, dm), O.block_ell_to_dense(*fc2, dm, dff)
    a = x @ W1.T + b1
    gel = 0.5 * a * (1 + np.tanh(math.sqrt(2 / math.pi) * (a + 0.044715 * a ** 3)))
    np.testing.assert_allclose(O.gelu_mlp_fwd(x, fc1, fc2, b1, b2), gel @ W2.T + b2, atol=1e-10)


def test_rmsnorm_bwd_matches_autograd_and_fd():
    torch = pytest.importorskip("torch")
    g = rng(83)
    x = g.standard_normal((6, 16))
    s = 1.0 + 0.3 * g.standard_normal(16)
    dy = g.standard_normal((6, 16))
    xt = torch.tensor(x, requires_grad=True)
    st = torch.tensor(s, requires_grad=True)
    y = xt / torch.sqrt((xt * xt).mean(-1, keepdim=True) + 1e-5) * st
    (y * torch.tensor(dy)).sum().backward()
    dx, ds = O.rmsnorm_bwd(x, s, dy, eps=1e-5)
    np.testing.assert_allclose(dx, xt.grad.numpy(), atol=1e-12)
    np.testing.assert_allclose(ds, st.grad.numpy(), atol=1e-12)
    e = 1e-6
    xp, xm = x.copy(), x.copy()
    xp[2, 5] += e
    xm[2, 5] -= e
    fd = (np.sum(O.rmsnorm(xp, s) * dy) - np.sum(O.rmsnorm(xm, s) * dy)) / (2 * e)
    assert abs(fd - dx[2, 5]) < 1e-6


def test_swiglu_bias_grads_match_autograd():
    torch = pytest.importorskip("torch")
    B, dm, dff = 4, 12, 16
    gate, up, down, x, dy = _bwd_case(84, B, dm, dff)
    g = rng(85)
    bg, bu, bd = g.standard_normal(dff), g.standard_normal(dff), g.standard_normal(dm)
    T = lambda a, grad=False: torch.tensor(a, dtype=torch.float64, requires_grad=grad)
    xt = T(x)
    bgt, but, bdt = T(bg, True), T(bu, True), T(bd, True)
    a = xt @ T(_dense_sum(*gate, dff, dm)).T + bgt
    b = xt @ T(_dense_sum(*up, dff, dm)).T + but
    out = (torch.nn.functional.silu(a) * b) @ T(_dense_sum(*down, dm, dff)).T + bdt + xt
    (out * T(dy)).sum().backward()
    dbg, dbu, dbd = O.swiglu_bias_grads(dy, a.detach().numpy(), b.detach().numpy(), down)
    np.testing.assert_allclose(dbg, bgt.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dbu, but.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dbd, bdt.grad.numpy(), atol=1e-10)


def test_rmsnorm_closed_forms():
    x = np.full((2, 8), 3.0)
    np.testing.assert_allclose(O.rmsnorm(x, np.ones(8), eps=0.0), np.ones((2, 8)), atol=1e-15)
    x = np.array([[3.0, 4.0]])   # mean square 12.5
    np.testing.assert_allclose(O.rmsnorm(x, np.array([1.0, 2.0]), eps=0.0),
                               [[3 / math.sqrt(12.5), 8 / math.sqrt(12.5)]], rtol=1e-15)
    x = rng(9).standard_normal((3, 16))
    s = rng(10).standard_normal(16)
    np.testing.assert_allclose(O.rmsnorm(10 * x, s, eps=0.0), O.rmsnorm(x, s, eps=0.0), rtol=1e-12)


def test_looped_composition():
    g = rng(11)
    B, dm, dff = 4, 8, 16
    gate = (0.1 * g.standard_normal((4, 1, B, B)), O.random_topology(4, 2, 1, g))
    up = (0.1 * g.standard_normal((4, 1, B, B)), O.random_topology(4, 2, 1, g))
    down = (0.1 * g.standard_normal((2, 2, B, B)), O.random_topology(2, 4, 2, g))
    h = g.standard_normal((3, dm))
    s = np.ones(dm)
    np.testing.assert_array_equal(O.looped_swiglu(h, s, gate, up, down, L=0), h)
    one = h + O.swiglu_fwd(O.rmsnorm(h, s), gate, up, down)[0]
    np.testing.assert_allclose(O.looped_swiglu(h, s, gate, up, down, L=1), one, atol=1e-12)
    two = one + O.swiglu_fwd(O.rmsnorm(one, s), gate, up, down)[0]
    np.testing.assert_allclose(O.looped_swiglu(h, s, gate, up, down, L=2), two, atol=1e-12)


def _core_blocks(g, n_core, B=4, dm=8, dff=16, bias=False):
    out = []
    for _ in range(n_core):
        gate = (0.3 * g.standard_normal((dff // B, 1, B, B)), O.random_topology(dff // B, dm // B, 1, g))
        up = (0.3 * g.standard_normal((dff // B, 1, B, B)), O.random_topology(dff // B, dm // B, 1, g))
        down = (0.3 * g.standard_normal((dm // B, 2, B, B)), O.random_topology(dm // B, dff // B, 2, g))
        bs = tuple(0.1 * g.standard_normal(n) for n in (dff, dff, dm)) if bias else None
        out.append((1.0 + 0.2 * g.standard_normal(dm), gate, up, down, bs))
    return out


def test_looped_core_reduces_to_looped_swiglu_and_mlp_step():
    g = rng(12)
    dm = 8
    h = g.standard_normal((5, dm))
    blk = _core_blocks(g, 1)
    s, gate, up, down, _ = blk[0]
    # one block, no injection, no depths: the shared-weight looped block
    np.testing.assert_allclose(O.looped_core(h, None, None, None, blk, L=3),
                               O.looped_swiglu(h, s, gate, up, down, L=3), atol=1e-12)
    # one iteration: the injection, then every core block in order (persistent_mlp_step)
    blks = _core_blocks(g, 3, bias=True)
    e = g.standard_normal((5, dm))
    la, ld = g.standard_normal(dm), g.standard_normal(dm)
    want = O.diagonal_injection(h, e, la, ld)
    for (sc, gt, u, d, bs) in blks:
        want = want + O.swiglu_fwd(O.rmsnorm(want, sc), gt, u, d, biases=bs)[0]
    np.testing.assert_allclose(O.looped_core(h, e, la, ld, blks, L=1), want, atol=1e-12)
    # two iterations: the injection again at the start of the second
    two = O.diagonal_injection(want, e, la, ld)
    for (sc, gt, u, d, bs) in blks:
        two = two + O.swiglu_fwd(O.rmsnorm(two, sc), gt, u, d, biases=bs)[0]
    np.testing.assert_allclose(O.looped_core(h, e, la, ld, blks, L=2), two, atol=1e-12)
    np.testing.assert_array_equal(O.looped_core(h, e, la, ld, blks, L=0), h)


def test_looped_core_depth_freeze_and_planted_mistakes():
    g = rng(13)
    dm, S = 8, 3
    depths = np.array([0, 1, 4, 2, 7])
    h = g.standard_normal((len(depths) * S, dm))
    e = g.standard_normal(h.shape)
    la, ld = g.standard_normal(dm), g.standard_normal(dm)
    blks = _core_blocks(g, 2)
    L = 4
    got = O.looped_core(h, e, la, ld, blks, L=L, depths=depths, seq_len=S)
    # each sequence equals the loop run for exactly min(depth, L) iterations on its rows
    for b, dep in enumerate(depths):
        rows = slice(b * S, (b + 1) * S)
        want = O.looped_core(h[rows], e[rows], la, ld, blks, L=min(dep, L))
        np.testing.assert_allclose(got[rows], want, atol=1e-12)
    np.testing.assert_array_equal(got[0:S], h[0:S])          # depth 0 keeps h
    # a ragged last sequence (depths cover N rows in runs of seq_len)
    got2 = O.looped_core(h[:-1], e[:-1], la, ld, blks, L=L, depths=depths, seq_len=S)
    np.testing.assert_allclose(got2, got[:-1], atol=1e-12)

    # planted mistakes are caught: the injection applied only once, the freeze at t <= depth,
    # the blocks in reverse order
    def once(h0):
        x = O.diagonal_injection(h0, e, la, ld)
        return O.looped_core(x, None, None, None, blks, L=L, depths=depths, seq_len=S)
    assert np.abs(once(h) - got).max() > 1e-3
    late = O.looped_core(h, e, la, ld, blks, L=L, depths=depths + 1, seq_len=S)
    assert np.abs(late - got).max() > 1e-3
    rev = O.looped_core(h, e, la, ld, blks[::-1], L=L, depths=depths, seq_len=S)
    assert np.abs(rev - got).max() > 1e-3


# ---------------------------------------------------------------- ternary

def test_ternary_quantize_hand_block():
    # mean|w| = (0.4+0.2+0.1+0.3)/4 = 0.25 (exact in float32 via the chosen values)
    w = np.array([0.5, -0.25, 0.125, 0.125], dtype=np.float32).reshape(1, 1, 2, 2)
    t, s = O.ternary_quantize_blocks(w)
    assert s[0, 0] == np.float32(0.25)
    # w/s = 2, -1, 0.5, 0.5 -> round-half-even: 2 -> clamp 1, -1, 0, 0
    np.testing.assert_array_equal(t.reshape(-1), [1, -1, 0, 0])
    t0, s0 = O.ternary_quantize_blocks(np.zeros((1, 1, 2, 2), np.float32))
    assert s0[0, 0] == np.float32(1e-8) and np.all(t0 == 0)


def test_activation_quantize_hand_rows():
    x = np.array([[1.0, -1.0, 0.5, 0.25],
                  [2.0, 1.0 / 256 * 2, -3 / 256 * 2, 0.0]], dtype=np.float32)
    q, sx = O.activation_quantize_int8(x)
    # row 0: absmax 1, scale 128: 128 -> clamp 127, -128, 64, 32
    np.testing.assert_array_equal(q[0], [127, -128, 64, 32])
    # row 1: absmax 2, scale 64: 128->127, 0.5 -> 0 (half to even), -1.5 -> -2, 0
    np.testing.assert_array_equal(q[1], [127, 0, -2, 0])
    np.testing.assert_array_equal(sx, np.array([1.0 / 128, 2.0 / 128], np.float32))
    qz, sz = O.activation_quantize_int8(np.zeros((1, 4), np.float32))
    assert np.all(qz == 0) and sz[0] == np.float32(1e-8 / 128)


def test_activation_quantize_matches_bitlinear_dequant():
    # bonsai-test/bitlinear.py:58-69 returns x_q / scale; our (q, sx) must give q * (absmax/128)
    x = rng(12).standard_normal((6, 32)).astype(np.float32)
    q, sx = O.activation_quantize_int8(x)
    absmax = np.abs(x).max(axis=1)
    scale = np.float32(128) / absmax.astype(np.float32)
    deq_ref = np.clip(np.rint(x * scale[:, None]), -128, 127) / scale[:, None]
    np.testing.assert_allclose(q * sx[:, None], deq_ref, rtol=1e-6)


def test_pack_known_words():
    t = np.zeros((1, 1, 16, 1), dtype=np.int8)
    t[0, 0, 0, 0] = 1      # i=0 -> bit 0, code 01
    t[0, 0, 5, 0] = -1     # i=5 -> bit 8*1 + 2*1 = 10, code 11
    t[0, 0, 15, 0] = 1     # i=15 -> bit 8*3 + 2*3 = 30, code 01
    w = O.pack_ternary(t)
    assert w.shape == (1, 1, 1, 1)
    assert int(w[0, 0, 0, 0]) == (1 << 0) | (3 << 10) | (1 << 30)
    # byte-extraction property used by the kernels
    word = int(w[0, 0, 0, 0])
    for qd in range(4):
        b = (word >> (2 * qd)) & 0x03030303
        for lane in range(4):
            code = (b >> (8 * lane)) & 3
            assert [0, 1, 0, -1][code] == t[0, 0, 4 * qd + lane, 0]


def test_pack_round_trip_all_codes():
    t = rng(13).integers(-1, 2, size=(3, 2, 64, 64)).astype(np.int8)
    np.testing.assert_array_equal(O.unpack_ternary(O.pack_ternary(t)), t)
    with pytest.raises(ValueError):
        O.pack_ternary(np.full((1, 1, 16, 16), 2, np.int8))


def test_partials_brute_force_and_extreme():
    g = rng(14)
    R, C, K, B = 2, 3, 2, 16
    t = g.integers(-1, 2, size=(R, K, B, B)).astype(np.int8)
    col = O.random_topology(R, C, K, g)
    col[1, 1] = -1
    q = g.integers(-128, 128, size=(3, C * B)).astype(np.int8)
    P = O.ternary_block_partials(q, t, col)
    for n in range(3):
        for r in range(R):
            for k in range(K):
                for j in range(B):
                    c = col[r, k]
                    ref = 0 if c < 0 else sum(int(q[n, c * B + i]) * int(t[r, k, i, j]) for i in range(B))
                    assert P[n, r, k, j] == ref
    # extreme: all -128 against all -1 gives B*128
    tq = -np.ones((1, 1, 64, 64), np.int8)
    qq = np.full((1, 64), -128, np.int8)
    assert O.ternary_block_partials(qq, tq, np.zeros((1, 1), np.int32)).max() == 64 * 128


def test_fixed_point_scales_bounds():
    g = rng(15)
    for K, B in ((4, 64), (16, 64), (8, 32), (32, 16)):
        s = np.abs(g.standard_normal((5, K))).astype(np.float32) * 0.02 + 1e-3
        col = np.zeros((5, K), np.int32)
        m, e = O.ternary_fixed_point(s, col, B)
        approx = m * np.ldexp(1.0, -e)[:, None]
        rel = np.abs(approx - s) / s.max(axis=1, keepdims=True)
        assert rel.max() <= 2.0 ** -13
        assert (m.max(axis=1) * K * B * 128 < 2 ** 31).all()


def test_ternary_matmul_dense_equivalence():
    g = rng(16)
    R, C, K, B = 3, 4, 2, 16
    t = g.integers(-1, 2, size=(R, K, B, B)).astype(np.int8)
    s = (np.abs(g.standard_normal((R, K))) * 0.02 + 0.01).astype(np.float32)
    col = O.random_topology(R, C, K, g)
    x = g.standard_normal((4, C * B)).astype(np.float32)
    q, sq = O.activation_quantize_int8(x)
    y, _ = O.ternary_matmul(q, sq, t, s, col, exact_scales=True)
    W = O.block_ell_to_dense(t.astype(np.float64) * s[:, :, None, None], col, R * B, C * B)
    np.testing.assert_allclose(y, (q.astype(np.float64) * sq[:, None]) @ W.T, rtol=1e-12, atol=1e-12)
    yf, acc = O.ternary_matmul(q, sq, t, s, col, exact_scales=False)
    assert np.abs(yf - y).max() <= 2.0 ** -12 * np.abs(y).max()


# ---------------------------------------------------------------- planted mistakes

def test_planted_transposed_tile_is_caught():
    g = rng(17)
    values = g.standard_normal((3, 2, 8, 8))
    col = O.random_topology(3, 4, 2, g)
    x = g.standard_normal((4, 32))
    wrong = O.block_ell_matmul(x, values.transpose(0, 1, 3, 2), col)
    W = O.block_ell_to_dense(values, col, 24, 32)
    assert np.abs(wrong - x @ W.T).max() > 1e-3


def test_planted_dropped_block_is_caught():
    g = rng(18)
    values = g.standard_normal((3, 2, 8, 8))
    col = O.random_topology(3, 4, 2, g)
    x = g.standard_normal((4, 32))
    c2 = col.copy()
    c2[0, 1] = -1
    assert np.abs(O.block_ell_matmul(x, values, c2) - brute_matmul(x, values, col)).max() > 1e-3


def test_planted_round_half_away_is_caught():
    x = np.array([[2.0, 0.5 / 64.0, 2.5 / 64.0]], dtype=np.float32)
    q, _ = O.activation_quantize_int8(x)            # scale 64: 0.5 -> 0 and 2.5 -> 2
    np.testing.assert_array_equal(q[0, 1:], [0, 2])
    away = np.sign(x * 64) * np.floor(np.abs(x * 64) + 0.5)
    assert not np.array_equal(q[0, 1:], away[0, 1:].astype(np.int8))


def test_bf16_round():
    a = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.14159], np.float32)
    r = O.bf16_round(a)
    np.testing.assert_array_equal(r[:4], np.array([1.0, 1.0, 1.0 + 2 ** -6, -2.5], np.float32))
    assert abs(r[4] - 3.140625) < 1e-7


# ---------------------------------------------------------------- backward

def _tile_grads_from_dense(gW, col, R, B):
    """Gather a dense [out, in] weight gradient into [R, K, B_in, B_out] tiles (dead -> 0)."""
    K = col.shape[1]
    C = gW.shape[1] // B
    out = np.zeros((R, K, B, B))
    for r in range(R):
        for k in range(K):
            c = int(col[r, k])
            if 0 <= c < C:
                out[r, k] = gW[r * B:(r + 1) * B, c * B:(c + 1) * B].T
    return out


def test_matmul_t_dense_adjoint_and_sentinel():
    g = rng(21)
    R, C, K, B = 5, 4, 3, 4
    values = g.standard_normal((R, K, B, B))
    col = O.random_topology(R, C, K, g)
    col[2, 1] = -1
    W = O.block_ell_to_dense(values, col, R * B, C * B)
    dy = g.standard_normal((6, R * B))
    x = g.standard_normal((6, C * B))
    dx = O.block_ell_matmul_t(dy, values, col, C)
    np.testing.assert_allclose(dx, dy @ W, atol=1e-10)
    # adjoint identity <A x, y> = <x, A^T y>
    lhs = np.sum(O.block_ell_matmul(x, values, col) * dy)
    np.testing.assert_allclose(lhs, np.sum(x * dx), rtol=1e-12)
    # a dead slot contributes nothing: changing its tile leaves the result unchanged
    v2 = values.copy()
    v2[2, 1] += 5.0
    np.testing.assert_array_equal(O.block_ell_matmul_t(dy, v2, col, C), dx)


def test_weight_grad_matches_autograd():
    torch = pytest.importorskip("torch")
    g = rng(22)
    R, C, K, B = 4, 5, 2, 4
    values = g.standard_normal((R, K, B, B))
    col = O.random_topology(R, C, K, g)
    col[1, 0] = col[1, 1]          # duplicate column in one row
    col[3, 1] = -1                 # dead slot
    x = g.standard_normal((7, C * B))
    dy = g.standard_normal((7, R * B))
    W = torch.tensor(O.block_ell_to_dense(values, col, R * B, C * B), requires_grad=True)
    (torch.tensor(x) @ W.T * torch.tensor(dy)).sum().backward()
    ref = _tile_grads_from_dense(W.grad.numpy(), col, R, B)
    np.testing.assert_allclose(O.block_ell_weight_grad(x, dy, col, B), ref, atol=1e-10)


def _dense_sum(values, col, out_f, in_f):
    """Dense [out, in] weight of a Block-ELL matrix with duplicate slots summed (the forward's
    semantics; the checkpoint bridge overwrites instead)."""
    R, K, B, _ = values.shape
    W = np.zeros((out_f, in_f))
    for r in range(R):
        for k in range(K):
            c = int(col[r, k])
            if 0 <= c < in_f // B:
                W[r * B:(r + 1) * B, c * B:(c + 1) * B] += values[r, k].T
    return W


def _bwd_case(seed, B=4, dm=12, dff=16, N=5):
    g = rng(seed)
    Cm, Cf, Rf, Rm = dm // B, dff // B, dff // B, dm // B
    gate = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, Cm, 2, g))
    up = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, Cm, 2, g))
    down = (g.standard_normal((Rm, 3, B, B)), O.random_topology(Rm, Cf, 3, g))
    gate[1][0, 1] = -1             # dead slot
    down[1][1, 2] = down[1][1, 0]  # duplicate column
    x = g.standard_normal((N, dm))
    dy = g.standard_normal((N, dm))
    return gate, up, down, x, dy


def test_swiglu_bwd_matches_autograd():
    torch = pytest.importorskip("torch")
    B, dm, dff = 4, 12, 16
    gate, up, down, x, dy = _bwd_case(23, B, dm, dff)
    T = lambda a, grad=False: torch.tensor(a, dtype=torch.float64, requires_grad=grad)
    xt = T(x, True)
    Wg = T(_dense_sum(*gate, dff, dm), True)
    Wu = T(_dense_sum(*up, dff, dm), True)
    Wd = T(_dense_sum(*down, dm, dff), True)
    a, b = xt @ Wg.T, xt @ Wu.T
    hh = torch.nn.functional.silu(a) * b
    out = hh @ Wd.T + xt
    (out * T(dy)).sum().backward()
    gx = a.detach().numpy()
    ux = b.detach().numpy()
    dx, dgv, duv, ddv = O.swiglu_bwd(dy, x, gx, ux, hh.detach().numpy(), gate, up, down)
    np.testing.assert_allclose(dx, xt.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dgv, _tile_grads_from_dense(Wg.grad.numpy(), gate[1], dff // B, B), atol=1e-10)
    np.testing.assert_allclose(duv, _tile_grads_from_dense(Wu.grad.numpy(), up[1], dff // B, B), atol=1e-10)
    np.testing.assert_allclose(ddv, _tile_grads_from_dense(Wd.grad.numpy(), down[1], dm // B, B), atol=1e-10)
    assert np.all(dgv[0, 1] == 0)


def test_swiglu_bwd_finite_differences():
    B, dm, dff = 4, 12, 16
    gate, up, down, x, dy = _bwd_case(24, B, dm, dff, N=3)

    def loss(xx, gv, uv, dv):
        out, *_ = O.swiglu_fwd(xx, (gv, gate[1]), (uv, up[1]), (dv, down[1]), add_residual=True)
        return float(np.sum(out * dy))

    _, h, gx, ux = O.swiglu_fwd(x, gate, up, down)
    dx, dgv, duv, ddv = O.swiglu_bwd(dy, x, gx, ux, h, gate, up, down)
    eps = 1e-6
    for (n, f) in [(0, 0), (2, 7), (1, 11)]:
        xp, xm = x.copy(), x.copy()
        xp[n, f] += eps
        xm[n, f] -= eps
        fd = (loss(xp, gate[0], up[0], down[0]) - loss(xm, gate[0], up[0], down[0])) / (2 * eps)
        assert abs(fd - dx[n, f]) < 1e-6 * max(1.0, abs(fd))
    for name, idx in [("g", (1, 0, 2, 3)), ("u", (3, 1, 0, 1)), ("d", (2, 2, 3, 0))]:
        vals = {"g": gate[0], "u": up[0], "d": down[0]}
        grads = {"g": dgv, "u": duv, "d": ddv}
        vp = {k: v.copy() for k, v in vals.items()}
        vm = {k: v.copy() for k, v in vals.items()}
        vp[name][idx] += eps
        vm[name][idx] -= eps
        fd = (loss(x, vp["g"], vp["u"], vp["d"]) - loss(x, vm["g"], vm["u"], vm["d"])) / (2 * eps)
        assert abs(fd - grads[name][idx]) < 1e-6 * max(1.0, abs(fd))


def test_planted_untransposed_tile_in_backward_is_caught():
    g = rng(25)
    values = g.standard_normal((3, 2, 4, 4))
    col = O.random_topology(3, 4, 2, g)
    dy = g.standard_normal((4, 12))
    W = O.block_ell_to_dense(values, col, 12, 16)
    wrong = O.block_ell_matmul_t(dy, values.transpose(0, 1, 3, 2), col, 4)
    assert np.abs(wrong - dy @ W).max() > 1e-3


# ---------------------------------------------------------------- topology transforms

def test_alive_slots_hand_rows():
    col = np.array([[0, -1, 3, 4], [2, 2, -1, 1]], np.int32)
    alive = np.array([[1, 1, 1, 0], [1, 0, 1, 1]], bool)
    np.testing.assert_array_equal(O.alive_slots(col, alive, 4),
                                  [[True, False, True, False], [True, False, False, True]])


def test_compact_topology_hand_rows():
    B = 2
    vals = np.arange(3 * 4 * B * B, dtype=np.float32).reshape(3, 4, B, B)
    col = np.array([[5, 6, 7, 8], [1, 2, 3, 4], [9, 9, 9, 9]], np.int32)
    alive = np.array([[0, 1, 0, 1], [1, 1, 1, 0], [0, 0, 0, 0]], bool)
    v2, c2, a2, K_new = O.compact_topology(vals, col, alive)
    assert K_new == 3
    np.testing.assert_array_equal(c2, [[6, 8, 5], [1, 2, 3], [9, 9, 9]])     # alive first, order kept
    np.testing.assert_array_equal(a2, [[1, 1, 0], [1, 1, 1], [0, 0, 0]])
    np.testing.assert_array_equal(v2[0, 0], vals[0, 1])
    np.testing.assert_array_equal(v2[0, 2], vals[0, 0])
    # compaction keeps the product: dead slots (sentinel) contribute nothing either way
    g = rng(31)
    R, C, K, B = 4, 6, 5, 4
    values = g.standard_normal((R, K, B, B))
    c = O.random_topology(R, C, K, g)
    al = g.random((R, K)) < 0.6
    x = g.standard_normal((3, C * B))
    eff = np.where(al, c, -1)
    v3, c3, a3, _ = O.compact_topology(values, c, al)
    np.testing.assert_allclose(O.block_ell_matmul(x, v3, np.where(a3, c3, -1)),
                               O.block_ell_matmul(x, values, eff), atol=1e-12)
    _, _, _, K1 = O.compact_topology(values, c, np.zeros((R, K), bool))
    assert K1 == 1                                                     # at least one slot


def test_column_importance_reference_and_brute():
    # reference tests/test_column_reorder.py:16-29: shape and non-negativity
    g = rng(32)
    R_model, K1, C_ff, K2 = 4, 8, 12, 6
    fc1_cols = g.integers(0, C_ff, (R_model, K1)).astype(np.int32)
    fc1_cols[0, 3] = -1
    fc1_alive = g.random((R_model, K1)) < 0.7
    fc2_alive = g.random((C_ff, K2)) < 0.5
    imp = O.column_importance(fc1_alive, fc2_alive, fc1_cols, C_ff)
    assert imp.shape == (C_ff,) and np.all(imp >= 0)
    brute = np.zeros(C_ff)
    for r in range(R_model):
        for k in range(K1):
            if fc1_cols[r, k] >= 0 and fc1_alive[r, k]:
                brute[fc1_cols[r, k]] += 1
    for c in range(C_ff):
        brute[c] += fc2_alive[c].sum()
    np.testing.assert_array_equal(imp, brute)


def test_column_permutation_known_answer_and_ties():
    perm = O.column_permutation(np.array([1.0, 5.0, 3.0, 0.0, 2.0]))   # reference :31-35
    assert perm[0] == 1 and perm[-1] == 3
    np.testing.assert_array_equal(O.column_permutation(np.array([2.0, 7.0, 2.0, 7.0])), [1, 3, 0, 2])


def test_apply_permutation_reference_cases_and_invariance():
    # reference :38-55 (column dim, reversed order)
    col = np.array([[0, 2, 4, 5], [1, 3, 4, 5]], np.int32)
    alive = np.ones((2, 4), bool)
    perm = np.array([5, 4, 3, 2, 1, 0], np.int32)
    _, c2, _ = O.apply_permutation(np.ones((2, 4, 16, 16)), col, alive, perm, True)
    np.testing.assert_array_equal(c2[0], np.argsort(perm)[col[0]])
    # reference :57-69 (row dim)
    g = rng(33)
    vals = g.standard_normal((4, 3, 16, 16))
    v2, _, _ = O.apply_permutation(vals, np.arange(12).reshape(4, 3), np.ones((4, 3), bool),
                                   np.array([3, 1, 0, 2]), False)
    np.testing.assert_array_equal(v2[0], vals[3])
    np.testing.assert_array_equal(v2[1], vals[1])
    # reference :99-113 (sentinels stay -1)
    cs = np.array([[0, 2, -1, -1], [1, 3, -1, -1]], np.int32)
    _, c3, _ = O.apply_permutation(None, cs, None, np.arange(8), True)
    assert np.all(c3[:, 2:] == -1)
    # permuting d_ff consistently (gate/up rows, down columns) leaves the SwiGLU FFN unchanged
    B, dm, dff = 4, 8, 16
    Rf, Cf = dff // B, dff // B
    gate = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, dm // B, 2, g))
    up = (g.standard_normal((Rf, 2, B, B)), O.random_topology(Rf, dm // B, 2, g))
    down = (g.standard_normal((dm // B, 3, B, B)), O.random_topology(dm // B, Cf, 3, g))
    x = g.standard_normal((3, dm))
    p = g.permutation(Cf).astype(np.int32)
    al = lambda w: np.ones(w[1].shape, bool)
    gv, gc, _ = O.apply_permutation(gate[0], gate[1], al(gate), p, False)
    uv, uc, _ = O.apply_permutation(up[0], up[1], al(up), p, False)
    _, dc, _ = O.apply_permutation(down[0], down[1], al(down), p, True)
    ref, *_ = O.swiglu_fwd(x, gate, up, down)
    got, *_ = O.swiglu_fwd(x, (gv, gc), (uv, uc), (down[0], dc))
    np.testing.assert_allclose(got, ref, atol=1e-12)


def test_k_active_macros_reference_cases():
    alive = np.ones((4, 8), bool)
    col = np.tile(np.arange(8, dtype=np.int32), (4, 1))
    assert O.k_active_macros(alive, col, 4) == 2                       # reference :71-82
    alive2 = np.zeros((2, 8), bool)
    alive2[:, :2] = True
    col2 = np.full((2, 8), -1, np.int32)
    col2[:, :2] = [0, 1]
    assert O.k_active_macros(alive2, col2, 4) == 1                     # reference :84-96
    assert O.k_active_macros(np.zeros((2, 3), bool), np.zeros((2, 3), np.int32), 4) == 0


def test_permute_optimizer_rows_hand_tree():
    perm = np.array([2, 0, 1], np.int32)
    mu = np.arange(3 * 2, dtype=np.float32).reshape(3, 2)
    other = np.arange(4, dtype=np.float32)                      # first dim != C_ff: untouched
    state = {"count": 7, "mu": mu, "nested": [mu * 10, other], "t": (mu,)}
    out = O.permute_optimizer_rows(state, perm, is_column_dim=False)
    np.testing.assert_array_equal(out["mu"], [[4, 5], [0, 1], [2, 3]])
    np.testing.assert_array_equal(out["nested"][0], [[40, 50], [0, 10], [20, 30]])
    assert out["nested"][1] is other and out["count"] == 7 and isinstance(out["t"], tuple)
    same = O.permute_optimizer_rows(state, perm, is_column_dim=True)
    assert same["mu"] is mu                                      # column mode: moments stay put


def _csc_brute(col, C):
    flat = col.reshape(-1)
    lists = [[e for e in range(flat.size) if flat[e] == c] for c in range(C)]
    ptr = np.cumsum([0] + [len(l) for l in lists])
    return ptr, [e for l in lists for e in l]


def test_transposed_index_brute_force():
    rng = np.random.default_rng(3)
    for R, K, C in [(1, 1, 1), (3, 4, 5), (7, 3, 2), (10, 9, 40)]:
        col = rng.integers(-1, C + 2, size=(R, K)).astype(np.int32)
        ptr, ent = O.transposed_index(col, C)
        bp, be = _csc_brute(col, C)
        np.testing.assert_array_equal(ptr, bp)
        np.testing.assert_array_equal(ent, be)
        valid = ((col >= 0) & (col < C)).sum()
        assert ptr[-1] == valid and len(set(ent.tolist())) == valid
    ptr, ent = O.transposed_index(np.full((2, 3), -1, np.int32), 4)
    assert ptr.tolist() == [0, 0, 0, 0, 0] and ent.size == 0


# ---------------------------------------------------------------- PyTorch CPU restatement (the CPU baseline)

def _tw(r, R, C, K, B, sentinel=False):
    v = (r.standard_normal((R, K, B, B)) * 0.05).astype(np.float32)
    col = O.random_topology(R, C, K, r)
    if sentinel:
        col[0, -1] = -1
    return v, col


def test_torch_cpu_swiglu_and_loop_match_oracle():
    import torch
    from oracle import torch_cpu as TC
    r = rng(41)
    B, dm, dff = 16, 64, 256
    g, u, d = _tw(r, dff // B, dm // B, 2, B, True), _tw(r, dff // B, dm // B, 2, B), _tw(r, dm // B, dff // B, 4, B)
    x = r.standard_normal((2 * TC.CHUNK + 37, dm)).astype(np.float32)     # several chunks, ragged tail
    tt = lambda w: (torch.from_numpy(w[0]), torch.from_numpy(w[1]))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    got = TC.swiglu_fwd(torch.from_numpy(x), tt(g), tt(u), tt(d), add_residual=True).numpy()
    want, *_ = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    scale = (1 + 0.1 * r.standard_normal(dm)).astype(np.float32)
    h = x[:300]
    got = TC.looped_swiglu(torch.from_numpy(h), torch.from_numpy(scale), tt(g), tt(u), tt(d), L=3).numpy()
    want = O.looped_swiglu(h.astype(np.float64), scale.astype(np.float64), f64(g), f64(u), f64(d), L=3)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_torch_cpu_ternary_matches_oracle():
    import torch
    from oracle import torch_cpu as TC
    r = rng(42)
    B, dm, dff, n = 64, 256, 512, 70
    def tw(R, C, K, sentinel=False):
        t = r.integers(-1, 2, size=(R, K, B, B)).astype(np.int8)
        s = (0.01 + 0.01 * r.random((R, K))).astype(np.float32)
        col = O.random_topology(R, C, K, r)
        if sentinel:
            col[1, 0] = -1
        return t, s, col
    g, u, d = tw(dff // B, dm // B, 2, True), tw(dff // B, dm // B, 2), tw(dm // B, dff // B, 4)
    tt = lambda w: (torch.from_numpy(w[0].astype(np.float32)), torch.from_numpy(w[1]), torch.from_numpy(w[2]))
    x = r.standard_normal((n, dm)).astype(np.float32)
    q, sx = TC.activation_quantize_int8(torch.from_numpy(x))
    q_ref, sx_ref = O.activation_quantize_int8(x)
    assert np.array_equal(q.numpy().astype(np.int8), q_ref) and np.array_equal(sx.numpy(), sx_ref)
    got = TC.ternary_matmul(q, sx, *tt(g)).numpy()
    want, _ = O.ternary_matmul(q_ref, sx_ref, *g)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    got = TC.ternary_swiglu_fwd(torch.from_numpy(x), tt(g), tt(u), tt(d)).numpy()
    res = O.ternary_swiglu_fwd(x, g, u, d)
    # h is re-quantised: a float32 vs float64 h can flip a rounding of hq, which moves the output by
    # one int8 step of one token's hidden value times a weight, far below the tolerance used here
    assert np.abs(got - res["out"]).max() <= 1e-3 * np.abs(res["out"]).max()


# ---------------------------------------------------------------- diagonal injection

def test_diagonal_injection_closed_forms_and_torch():
    import torch
    r = rng(51)
    n, d = 7, 12
    h, e = r.standard_normal((n, d)), r.standard_normal((n, d))
    la, ld = 0.3 * r.standard_normal(d), 0.5 * r.standard_normal(d)
    # log_A -> -inf: A -> 0, decay -> 1; log_dt = log(e - 1): dt = 1 exactly
    out = O.diagonal_injection(h, e, np.full(d, -np.inf), np.full(d, math.log(math.e - 1)))
    np.testing.assert_allclose(out, h + e, rtol=1e-12, atol=1e-12)
    # the reference's PyTorch formula (interop/pt_model.py:931-935), in float64
    tl, td = torch.tensor(la), torch.tensor(ld)
    A = -torch.exp(tl)
    dt = torch.nn.functional.softplus(td)
    ref = (torch.exp(dt * A) * torch.tensor(h) + dt * torch.tensor(e)).numpy()
    np.testing.assert_allclose(O.diagonal_injection(h, e, la, ld), ref, rtol=1e-12, atol=1e-12)


def test_diagonal_injection_bwd_autograd_and_finite_differences():
    import torch
    r = rng(52)
    n, d = 9, 10
    h, e, dy = r.standard_normal((n, d)), r.standard_normal((n, d)), r.standard_normal((n, d))
    la, ld = 0.3 * r.standard_normal(d), 0.5 * r.standard_normal(d)
    th, te, tla, tld = (torch.tensor(a, requires_grad=True) for a in (h, e, la, ld))
    A = -torch.exp(tla)
    dt = torch.nn.functional.softplus(tld)
    out = torch.exp(dt * A) * th + dt * te
    out.backward(torch.tensor(dy))
    got = O.diagonal_injection_bwd(h, e, la, ld, dy)
    for g, t in zip(got, (th, te, tla, tld)):
        np.testing.assert_allclose(g, t.grad.numpy(), rtol=1e-10, atol=1e-12)
    eps = 1e-6
    for j in (0, 4, 9):
        for which in (2, 3):
            p = [la.copy(), ld.copy()]
            p[which - 2][j] += eps
            up = np.sum(dy * O.diagonal_injection(h, e, *p))
            p[which - 2][j] -= 2 * eps
            dn = np.sum(dy * O.diagonal_injection(h, e, *p))
            assert abs((up - dn) / (2 * eps) - got[which][j]) < 1e-6
