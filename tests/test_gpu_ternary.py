"""GPU parity of the int8 / ternary kernels against the CPU oracle.

Bars: activation quantisation (xq, sx) bit-exact; packing bit-exact; the int32
block partials bit-exact; the fixed-point scaled products bit-exact against the
oracle's restatement of the same fixed-point arithmetic; single products within
1e-2 * max|ref| of the exact-scale (float64) oracle; whole FFNs (with the int8
re-quantisation of h) within the bounds of ffn_vs_exact.
"""

import ctypes as C

import numpy as np
import pytest

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _say(msg):
    print(msg, flush=True)


def ffn_vs_exact(out, ref, hq=None, sh=None, down=None, resid=None):
    """A whole ternary FFN against the exact-scale oracle.

    The int8 re-quantisation of h turns a last-ulp difference of an h value near a rounding
    boundary into a whole quantum (amax / 128) of the down input.  On the CPU the oracle's own
    fixed-point and exact-scale pipelines differ by 0.94 % of the output RMS and 1.25 % of
    max|ref| at d_model 2048, d_ff 8192, 64 tokens (1.6 % of the hq values flipped), so that
    difference is quantisation noise of the reference semantics, not scaling error.  Hence two
    checks: given the kernel's own hq (and sh), the exact-scale down product must agree to 2^-8
    of max|y| (this isolates the fixed-point scaling, <= 2^-12 relative, beside the bf16
    rounding of the output, <= 2^-9); and the whole FFN must agree to 1.5e-2 in relative RMS and
    3e-2 of max|ref| per element (the noise allowance).  The exact bars are the int32
    accumulators and the down product given hq, checked bit for bit elsewhere."""
    out = np.asarray(out, np.float64)
    if hq is not None:
        yd, _ = O.ternary_matmul(hq, sh, *down, exact_scales=True)
        if resid is not None:
            yd = yd + np.asarray(resid, np.float64)
        rel_d, ab_d = T.rel_err(out, yd)
        assert rel_d <= 2.0 ** -8, f"down given hq: rel {rel_d} abs {ab_d}"
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean((out - ref) ** 2)) / max(np.sqrt(np.mean(ref ** 2)), 1e-30))
    rel, ab = T.rel_err(out, ref)
    assert rms <= 1.5 * TOL and rel <= 3 * TOL, f"relative rms {rms}, max {rel} (abs {ab})"


def tern_weight(rng, R, C_, K, B, sentinel_frac=0.0):
    t = rng.integers(-1, 2, size=(R, K, B, B)).astype(np.int8)
    lat = rng.standard_normal((R, K, B, B)).astype(np.float32) * 0.02
    s = np.maximum(np.mean(np.abs(lat.reshape(R, K, -1)), axis=2), 1e-8).astype(np.float32)
    col = O.random_topology(R, C_, K, rng)
    if sentinel_frac:
        col[rng.random(col.shape) < sentinel_frac] = -1
    return t, s, col


def check_accumulators(res, xq, sx, g, u, d, rows=None):
    """Bit-exact checks of the exported accumulators of ternary_swiglu_fwd_accumulators: the int32
    sums sum_k m*P of gate and up given xq, their fp32 pre-activations, the down sums given the
    kernel's own hq; h within TOL of silu(g)*u.  Only ``rows`` are copied back when given."""
    import torch
    if rows is not None:
        idx = torch.as_tensor(rows, device=res[0].device)
        res = [t[idx] for t in res]
    out, h, hq, sh, ag, au, ad, gp, up = (T.to_np(t) for t in res)
    n = xq.shape[0]
    gf, acc_g = O.ternary_matmul(xq, sx, *g, exact_scales=False)
    uf, acc_u = O.ternary_matmul(xq, sx, *u, exact_scales=False)
    assert np.array_equal(ag, acc_g.reshape(n, -1)), "gate int32 accumulators"
    assert np.array_equal(au, acc_u.reshape(n, -1)), "up int32 accumulators"
    assert np.array_equal(gp.view(np.uint32), gf.astype(np.float32).view(np.uint32)), "gate pre-activations"
    assert np.array_equal(up.view(np.uint32), uf.astype(np.float32).view(np.uint32)), "up pre-activations"
    assert np.abs(acc_g).max() > 0 and np.abs(acc_u).max() > 0
    yd, acc_d = O.ternary_matmul(hq, sh, *d, exact_scales=False)
    assert np.array_equal(ad, acc_d.reshape(n, -1)), "down int32 accumulators"
    # h = silu(g) * u from the kernel's own (bit-exact) pre-activations, device exp / rcp
    href = O.bf16_round(O.silu(gp.astype(np.float64)) * up)
    assert T.rel_err(h, href)[0] <= TOL
    return out, h, hq, sh, yd


def gpu_tern(w):
    import torch
    t, s, col = w
    packed = O.pack_ternary(t).view(np.int32)
    return T.to_gpu(packed), T.to_gpu(s), T.to_gpu(col.astype(np.int32))


def test_quantize_act_bit_exact(gpu):
    from looped_blockell import kernels
    rng = np.random.default_rng(1)
    x = T.act(rng, 300, 2048)
    x[0] = 0.0                                   # absmax clamp row
    x[1, :4] = [2.0, 1.0 / 64, -3.0 / 64, 0.0]   # ties at scale 64
    x[1, 4:] = 0.0
    q, s = kernels.quantize_act_int8(T.to_gpu_bf16(x))
    q_ref, s_ref = O.activation_quantize_int8(x)
    assert np.array_equal(T.to_np(q), q_ref)
    assert np.array_equal(T.to_np(s), s_ref)


def test_pack_bit_exact(gpu):
    from looped_blockell import kernels
    rng = np.random.default_rng(2)
    for B in (16, 32, 64):
        t = rng.integers(-1, 2, size=(3, 2, B, B)).astype(np.int8)
        p = T.to_np(kernels.pack_ternary(T.to_gpu(t))).view(np.uint32)
        assert np.array_equal(p, O.pack_ternary(t)), B


def test_ternary_quantize_weights(gpu):
    from looped_blockell import kernels
    rng = np.random.default_rng(3)
    v = T.act(rng, 4 * 3 * 64, 64).reshape(4, 3, 64, 64) * 0.02
    v = O.bf16_round(v)
    p, s = kernels.ternary_quantize_weights(T.to_gpu_bf16(v))
    s = T.to_np(s)
    t_ref, s_ref = O.ternary_quantize_blocks(v)
    np.testing.assert_allclose(s, s_ref, rtol=1e-6)
    # codes bit-exact given the kernel's own scale
    t_given = np.clip(np.rint(v.reshape(12, -1) / s.reshape(12, 1)), -1, 1).astype(np.int8).reshape(v.shape)
    assert np.array_equal(O.unpack_ternary(T.to_np(p).view(np.uint32)), t_given)


@pytest.mark.parametrize("B", [16, 32, 64])
@pytest.mark.parametrize("N", [1, 37, 128])
def test_ternary_matmul_partials_and_scaling(gpu, B, N):
    from looped_blockell import kernels
    _say(f"ternary matmul B={B} N={N}")
    rng = np.random.default_rng(10 + B + N)
    R, C_, K = 4, 6, 3
    w = tern_weight(rng, R, C_, K, B, sentinel_frac=0.15)
    x = T.act(rng, N, C_ * B)
    xq, sx = O.activation_quantize_int8(x)
    y, part = kernels.ternary_matmul(T.to_gpu(xq), T.to_gpu(sx), *gpu_tern(w), want_partials=True)
    P_ref = O.ternary_block_partials(xq, w[0], w[2])
    assert np.array_equal(T.to_np(part).astype(np.int64), P_ref)
    # fixed-point scaled product: bit-exact before the bf16 output rounding
    y_fix, _ = O.ternary_matmul(xq, sx, w[0], w[1], w[2], exact_scales=False)
    assert np.array_equal(T.to_np(y), O.bf16_round(y_fix))
    y_exact, _ = O.ternary_matmul(xq, sx, w[0], w[1], w[2], exact_scales=True)
    assert T.rel_err(T.to_np(y), y_exact)[0] <= TOL


def test_ternary_extreme_partials(gpu):
    """All-(-128) activations against all-(-1) tiles: P = B*128 per block, no overflow."""
    from looped_blockell import kernels
    B, K, R, C_ = 64, 16, 2, 16
    t = -np.ones((R, K, B, B), np.int8)
    s = np.full((R, K), 0.02, np.float32)
    col = np.tile(np.arange(K, dtype=np.int32), (R, 1))
    xq = np.full((3, C_ * B), -128, np.int8)
    sx = np.ones(3, np.float32)
    y, part = kernels.ternary_matmul(T.to_gpu(xq), T.to_gpu(sx), *gpu_tern((t, s, col)), want_partials=True)
    assert (T.to_np(part) == B * 128).all()
    y_fix, acc = O.ternary_matmul(xq, sx, t, s, col, exact_scales=False)
    assert np.array_equal(T.to_np(y), O.bf16_round(y_fix))


TERN_CASES = [
    # (d_model, d_ff, B, density, N)
    (512, 2048, 64, 0.125, 100),
    (256, 1024, 32, 0.25, 65),
    (128, 512, 16, 0.25, 33),
    (2048, 8192, 64, 0.125, 64),    # the ternary headline geometry, small N
]


@pytest.mark.parametrize("case", TERN_CASES)
@pytest.mark.parametrize("resid", [False, True])
def test_ternary_swiglu(gpu, case, resid):
    from looped_blockell import kernels
    d_model, d_ff, B, dens, N = case
    _say(f"ternary swiglu {case} resid={resid}")
    rng = np.random.default_rng(hash(case) % 2 ** 31)
    Kg, Kd = O.k_for_density(d_model // B, dens), O.k_for_density(d_ff // B, dens)
    g = tern_weight(rng, d_ff // B, d_model // B, Kg, B)
    u = tern_weight(rng, d_ff // B, d_model // B, Kg, B)
    d = tern_weight(rng, d_model // B, d_ff // B, Kd, B)
    x = T.act(rng, N, d_model)
    xq, sx = O.activation_quantize_int8(x)
    xg = T.to_gpu_bf16(x)
    res = kernels.ternary_swiglu_fwd_accumulators(
        T.to_gpu(xq), T.to_gpu(sx), gpu_tern(g), gpu_tern(u), gpu_tern(d), xg if resid else None)
    out, h, hq, sh, _ = check_accumulators(res, xq, sx, g, u, d)
    # h re-quantisation is bit-exact given the kernel's h
    hq_ref, sh_ref = O.activation_quantize_int8(h)
    assert np.array_equal(hq, hq_ref) and np.array_equal(sh, sh_ref)
    # gate/up: fixed-point products are bit-exact; h within tolerance (SiLU uses the device exp)
    gf, _ = O.ternary_matmul(xq, sx, *g, exact_scales=False)
    uf, _ = O.ternary_matmul(xq, sx, *u, exact_scales=False)
    assert T.rel_err(h, O.bf16_round(O.silu(gf.astype(np.float64)) * uf))[0] <= TOL
    # down: bit-exact given the kernel's hq (plus the residual in fp32)
    yd, _ = O.ternary_matmul(hq, sh, *d, exact_scales=False)
    if resid:
        yd = (yd + x).astype(np.float32)
    assert np.array_equal(out, O.bf16_round(yd))
    # whole FFN against the exact-scale oracle
    ref = O.ternary_swiglu_fwd(x, g, u, d, add_residual=resid, exact_scales=True, h_round=O.bf16_round)
    ffn_vs_exact(out, ref["out"], hq, sh, d, x if resid else None)


# B = 64 geometries served by the two-kernel path (gate/up kernel + down kernel with
# on-the-fly re-quantisation): ragged N, every slice count (N >= 16384 -> 1 slice,
# 8192 -> 2, fewer -> 4), slot counts that are not multiples of the ring depths (2 and 8),
# dead slots, down rows fewer than the 8 waves, and a fully dead gate row.
SPLIT_CASES = [
    # (d_model, d_ff, Kg, Kd, N, sentinel_frac)
    (256, 1024, 3, 5, 1, 0.0),
    (256, 1024, 3, 5, 65, 0.2),
    (512, 2048, 2, 7, 8192 + 3, 0.1),
    (256, 512, 4, 8, 16384 + 37, 0.0),
    (2048, 4096, 5, 3, 200, 0.3),
    (1024, 6144, 4, 12, 300, 0.1),    # 384 panel units per token row: 1024 threads in 2 whole row groups
    (512, 9216, 2, 9, 70, 0.0),       # 576 units: one row group, 448 threads idle in the fill
]


@pytest.mark.parametrize("case", SPLIT_CASES)
def test_ternary_swiglu_split(gpu, case):
    from looped_blockell import kernels
    d_model, d_ff, Kg, Kd, N, frac = case
    B = 64
    _say(f"ternary swiglu split {case}")
    rng = np.random.default_rng(abs(hash(case)) % 2 ** 31)
    g = tern_weight(rng, d_ff // B, d_model // B, Kg, B, sentinel_frac=frac)
    u = tern_weight(rng, d_ff // B, d_model // B, Kg, B, sentinel_frac=frac)
    d = tern_weight(rng, d_model // B, d_ff // B, Kd, B, sentinel_frac=frac)
    if frac:
        g[2][0, :] = -1                                  # a gate row with no live block
    x = T.act(rng, N, d_model)
    xq, sx = O.activation_quantize_int8(x)
    xg = T.to_gpu_bf16(x)
    args = (T.to_gpu(xq), T.to_gpu(sx), gpu_tern(g), gpu_tern(u), gpu_tern(d), xg)
    assert kernels.ternary_prepare(*args[2:5]).numel() > 0, "geometry outside the two-kernel path"
    out, h, hq, sh = kernels.ternary_swiglu_fwd_with_intermediate(*args)
    out_ws = kernels.ternary_swiglu_fwd(*args)
    out, h, hq, sh, out_ws = T.to_np(out), T.to_np(h), T.to_np(hq), T.to_np(sh), T.to_np(out_ws)
    assert np.array_equal(out, out_ws)
    # the same kernels with the accumulator exports: identical outputs, bit-exact accumulators
    res = kernels.ternary_swiglu_fwd_accumulators(*args)
    out_a, h_a, hq_a, sh_a, _ = check_accumulators(res, xq, sx, g, u, d)
    assert np.array_equal(out_a, out) and np.array_equal(h_a, h) and np.array_equal(hq_a, hq)
    hq_ref, sh_ref = O.activation_quantize_int8(h)
    assert np.array_equal(hq, hq_ref) and np.array_equal(sh, sh_ref)
    gf, _ = O.ternary_matmul(xq, sx, *g, exact_scales=False)
    uf, _ = O.ternary_matmul(xq, sx, *u, exact_scales=False)
    href = O.bf16_round(O.silu(gf.astype(np.float64)) * uf)
    assert T.rel_err(h, href)[0] <= TOL
    if frac:
        assert (h[:, :B] == 0).all()
    yd, _ = O.ternary_matmul(hq, sh, *d, exact_scales=False)
    assert np.array_equal(out, O.bf16_round((yd + x).astype(np.float32)))
    ref = O.ternary_swiglu_fwd(x, g, u, d, add_residual=True, exact_scales=True, h_round=O.bf16_round)
    ffn_vs_exact(out, ref["out"], hq, sh, d, x)


def test_ternary_swiglu_split_extreme(gpu):
    """All-(-128) activations against all-(-1) tiles with equal scales: accumulators
    K * m * 64 * 128 within 1% of the int32 limit the fixed point is sized for, bit-exact."""
    _say("ternary swiglu split extreme accumulators")
    from looped_blockell import kernels
    B, d_model, d_ff, K, N = 64, 2048, 2048, 32, 70
    t = -np.ones((d_ff // B, K, B, B), np.int8)
    s = np.full((d_ff // B, K), 127 / 128, np.float32)
    col = np.tile(np.arange(K, dtype=np.int32), (d_ff // B, 1))
    td = -np.ones((d_model // B, K, B, B), np.int8)
    sd = np.full((d_model // B, K), 127 / 128, np.float32)
    xq = np.full((N, d_model), -128, np.int8)
    sx = np.full(N, 1.0 / 128, np.float32)
    out, h, hq, sh = kernels.ternary_swiglu_fwd_with_intermediate(
        T.to_gpu(xq), T.to_gpu(sx), gpu_tern((t, s, col)), gpu_tern((t, s, col)), gpu_tern((td, sd, col)), None)
    h = T.to_np(h)
    gf, acc = O.ternary_matmul(xq, sx, t, s, col, exact_scales=False)
    m, _ = O.ternary_fixed_point(s, col, B)
    assert acc.max() == K * m.max() * B * 128 and acc.max() > 0.99 * 2 ** 31
    assert T.rel_err(h, O.bf16_round(O.silu(gf.astype(np.float64)) * gf))[0] <= TOL
    yd, _ = O.ternary_matmul(T.to_np(hq), T.to_np(sh), td, sd, col, exact_scales=False)
    assert np.array_equal(T.to_np(out), O.bf16_round(yd))


def test_ternary_full_size_sampled_rows(gpu):
    """The ternary FFN at full size (8192 tokens, d_model 2048, d_ff 8192, B 64); bit-exact checks on
    sampled rows."""
    from looped_blockell import kernels
    _say("ternary d2048 ff8192 B64 N8192 full size")
    rng = np.random.default_rng(1003)
    d_model, d_ff, B, N = 2048, 8192, 64, 8192
    g = tern_weight(rng, d_ff // B, d_model // B, 4, B)
    u = tern_weight(rng, d_ff // B, d_model // B, 4, B)
    d = tern_weight(rng, d_model // B, d_ff // B, 16, B)
    x = T.act(rng, N, d_model)
    xg = T.to_gpu_bf16(x)
    xq_t, sx_t = kernels.quantize_act_int8(xg)
    res = kernels.ternary_swiglu_fwd_accumulators(xq_t, sx_t, gpu_tern(g), gpu_tern(u), gpu_tern(d))
    out_plain = kernels.ternary_swiglu_fwd(xq_t, sx_t, gpu_tern(g), gpu_tern(u), gpu_tern(d))
    import torch
    assert torch.equal(out_plain, res[0])
    rows = np.sort(rng.choice(N, 256, replace=False))
    xq, sx = O.activation_quantize_int8(x[rows])
    assert np.array_equal(T.to_np(xq_t)[rows], xq) and np.array_equal(T.to_np(sx_t)[rows], sx)
    # int32 accumulators of gate, up (given xq) and down (given the kernel's hq) bit-exact, the fp32
    # pre-activations bit-exact, on the sampled rows
    out, h, hq_r, sh_r, yd = check_accumulators(res, xq, sx, g, u, d, rows=rows)
    assert np.array_equal(out, O.bf16_round(yd))
    hq_ref, sh_ref = O.activation_quantize_int8(h)
    assert np.array_equal(hq_r, hq_ref) and np.array_equal(sh_r, sh_ref)
    ref = O.ternary_swiglu_fwd(x[rows], g, u, d, exact_scales=True, h_round=O.bf16_round)
    ffn_vs_exact(out, ref["out"], hq_r, sh_r, d)


# Large B = 64 geometries on sampled rows: several thousand tokens (row groups dealt over the down
# rows where the 16-token blocks number fewer than 256), a ragged last block, dead slots, down rows
# with 9-30 slots, d_ff from 2048 to 8192, with and without the residual.
LARGE_CASES = [
    # (d_model, d_ff, Kg, Kd, N, sentinel_frac, residual)
    (2048, 8192, 3, 13, 4096 + 5, 0.2, True),
    (1024, 4096, 4, 9, 6000, 0.0, False),
    (512, 6144, 2, 30, 8192 + 33, 0.1, True),
    (2048, 2048, 4, 16, 9000, 0.0, True),
]


@pytest.mark.parametrize("case", LARGE_CASES)
def test_ternary_swiglu_large_sampled(gpu, case):
    """Sampled rows (the last rows of the ragged block among them): int32 accumulators of gate/up
    (given xq) and down (given the kernel's hq) bit-exact, hq the oracle's quantisation of the
    kernel's h, outputs bit-exact given hq; the plain and accumulator-exporting launches agree."""
    import torch
    from looped_blockell import kernels
    d_model, d_ff, Kg, Kd, N, frac, resid = case
    B = 64
    _say(f"ternary large sampled {case}")
    rng = np.random.default_rng(abs(hash(case)) % 2 ** 31)
    g = tern_weight(rng, d_ff // B, d_model // B, Kg, B, sentinel_frac=frac)
    u = tern_weight(rng, d_ff // B, d_model // B, Kg, B, sentinel_frac=frac)
    d = tern_weight(rng, d_model // B, d_ff // B, Kd, B, sentinel_frac=frac)
    x = T.act(rng, N, d_model)
    xg = T.to_gpu_bf16(x)
    xq_t, sx_t = kernels.quantize_act_int8(xg)
    args = (xq_t, sx_t, gpu_tern(g), gpu_tern(u), gpu_tern(d), xg if resid else None)
    res = kernels.ternary_swiglu_fwd_accumulators(*args)
    out_plain = kernels.ternary_swiglu_fwd(*args)
    assert torch.equal(out_plain, res[0])
    rows = np.unique(np.concatenate([rng.choice(N, 96, replace=False), np.arange(N - 8, N)]))
    xq, sx = O.activation_quantize_int8(x[rows])
    out, h, hq, sh, yd = check_accumulators(res, xq, sx, g, u, d, rows=rows)
    hq_ref, sh_ref = O.activation_quantize_int8(h)
    assert np.array_equal(hq, hq_ref) and np.array_equal(sh, sh_ref)
    if resid:
        yd = (yd + x[rows]).astype(np.float32)
    assert np.array_equal(out, O.bf16_round(yd))


@pytest.mark.parametrize("case", [
    # (d_model, d_ff, B, Kg, Kd, token counts, sentinel_frac)
    (512, 2048, 64, 2, 7, (300, 17), 0.1),      # the B = 64 two-kernel path: prepared weights
    (256, 1024, 32, 2, 8, (77, 5), 0.0),         # row-block path: no prepared form
])
def test_ternary_prepared_matches_per_call_preparation(gpu, case):
    """lbk_ternary_prepare + lbk_swiglu_fwd_ternary_prepared against lbk_swiglu_fwd_ternary_acc (the
    same kernels, bit-identical outputs and accumulators) on two calls in a row reusing one prepared
    buffer; then the operator pair and TernaryMLPBlock's cache."""
    import torch
    from looped_blockell import kernels
    d_model, d_ff, B, Kg, Kd, ns, frac = case
    _say(f"ternary prepared {case}")
    A = T.abi()
    lib = A.load()
    rng = np.random.default_rng(900 + B)
    g = tern_weight(rng, d_ff // B, d_model // B, Kg, B, sentinel_frac=frac)
    u = tern_weight(rng, d_ff // B, d_model // B, Kg, B, sentinel_frac=frac)
    d = tern_weight(rng, d_model // B, d_ff // B, Kd, B, sentinel_frac=frac)
    tw = [gpu_tern(w) for w in (g, u, d)]
    gs, us, ds = (T.tern_struct(*w) for w in tw)
    pb = lib.lbk_ternary_prepared_bytes(d_model, C.byref(gs), C.byref(us), C.byref(ds))
    assert (pb > 0) == (B == 64)
    prep = torch.empty(max(pb, 1), dtype=torch.uint8, device="cuda")
    A.check(lib.lbk_ternary_prepare(d_model, C.byref(gs), C.byref(us), C.byref(ds), T.ptr(prep), pb, T.stream()),
            "ternary_prepare")
    for n in ns:
        x = T.act(rng, n, d_model)
        xq, sx = O.activation_quantize_int8(x)
        txq, tsx, txr = T.to_gpu(xq), T.to_gpu(sx), T.to_gpu_bf16(x)
        outs = []
        for prepared in (False, True):
            o = torch.empty(n, d_model, dtype=torch.bfloat16, device="cuda")
            h = torch.empty(n, d_ff, dtype=torch.bfloat16, device="cuda")
            accs = [torch.empty(n, f, dtype=dt, device="cuda") for f, dt in
                    ((d_ff, torch.int32), (d_ff, torch.int32), (d_model, torch.int32), (d_ff, torch.float32),
                     (d_ff, torch.float32))]
            acc = A.TernaryAcc(*(T.ptr(t) for t in accs))
            if prepared:
                wsb = lib.lbk_ternary_prepared_workspace_bytes(n, d_model, C.byref(gs), C.byref(us), C.byref(ds))
                ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
                st = lib.lbk_swiglu_fwd_ternary_prepared(T.ptr(txq), T.ptr(tsx), n, d_model, C.byref(gs), C.byref(us),
                                                         C.byref(ds), T.ptr(prep) if pb else None, pb, T.ptr(txr),
                                                         T.ptr(o), T.ptr(h), None, None, C.byref(acc), T.ptr(ws), wsb,
                                                         T.stream())
            else:
                wsb = lib.lbk_ternary_swiglu_workspace_bytes(n, d_model, C.byref(gs), C.byref(us), C.byref(ds))
                ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
                st = lib.lbk_swiglu_fwd_ternary_acc(T.ptr(txq), T.ptr(tsx), n, d_model, C.byref(gs), C.byref(us),
                                                    C.byref(ds), T.ptr(txr), T.ptr(o), T.ptr(h), None, None,
                                                    C.byref(acc), T.ptr(ws), wsb, T.stream())
            A.check(st, "ternary forward")
            torch.cuda.synchronize()
            outs.append([o, h] + accs)
        for a, b in zip(*outs):
            assert torch.equal(a, b)
        ref = O.ternary_swiglu_fwd(x, g, u, d, add_residual=True, exact_scales=True, h_round=O.bf16_round)
        ffn_vs_exact(T.to_np(outs[1][0]), ref["out"])
    if pb:
        small = torch.empty(pb - 256, dtype=torch.uint8, device="cuda")
        assert lib.lbk_ternary_prepare(d_model, C.byref(gs), C.byref(us), C.byref(ds), T.ptr(small), small.numel(),
                                       T.stream()) == A.LBK_ERR_WORKSPACE
    # operators and the layer cache
    from looped_blockell.layers.ternary import TernaryBlockELLWeight, TernaryMLPBlock
    wts = [TernaryBlockELLWeight(*w) for w in tw]
    m = TernaryMLPBlock(*wts)
    x = T.to_gpu_bf16(T.act(rng, 40, d_model))
    xq, sx = kernels.quantize_act_int8(x)
    y = m(x)
    assert torch.equal(y, kernels.ternary_swiglu_fwd(xq, sx, *[w.triple() for w in wts]))
    with torch.no_grad():
        wts[2].scales.mul_(2.0)                      # new version: the cache is rebuilt
    y2 = m(x)
    assert torch.equal(y2, kernels.ternary_swiglu_fwd(xq, sx, *[w.triple() for w in wts]))
    assert not torch.equal(y2, y)
