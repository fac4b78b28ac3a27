"""Parity of the prune-time topology transforms (looped_blockell.opt over the C ABI) against the
oracle.  All of it is integer, index and copy work, so the bar is bit-exact equality.

Edge cases follow the reference's column-reorder and compaction tests: sentinel columns (-1),
columns past C_ff, all-dead rows and layers, ties and NaNs in the importance, rows longer than
one 64-slot wave chunk.  A size-independent property closes it: permuting d_ff consistently
(gate/up rows gathered, down column indices remapped) leaves the FFN forward unchanged.
"""

import ctypes as C

import numpy as np
import pytest

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[topo] {msg}", flush=True)


def _opt():
    from looped_blockell import opt
    return opt


def _np(t):
    return T.to_np(t)


def _layer(rng, R, C_, K, B, p_alive, sentinel_frac=0.0, over_frac=0.0):
    vals = O.bf16_round(rng.standard_normal((R, K, B, B)).astype(np.float32))
    col = rng.integers(0, C_, size=(R, K)).astype(np.int32)
    col[rng.random((R, K)) < sentinel_frac] = -1
    over = rng.random((R, K)) < over_frac
    col[over] = C_ + rng.integers(0, 3, size=int(over.sum()))
    alive = rng.random((R, K)) < p_alive
    return vals, col, alive


def _gpu_layer(vals, col, alive):
    import torch
    return T.to_gpu_bf16(vals), T.to_gpu(col.astype(np.int32)), T.to_gpu(alive.astype(np.bool_))


COMPACT_CASES = [
    # (R, K, B, p_alive, dead_rows)
    (48, 20, 32, 0.6, (3,)),
    (16, 130, 16, 0.3, (0, 15)),        # K spans three 64-slot chunks
    (8, 12, 64, 0.9, ()),
    (6, 9, 16, 0.0, ()),                # nothing alive: K_new = 1
    (5, 64, 32, 1.0, ()),               # everything alive: order unchanged
]


@pytest.mark.parametrize("case", COMPACT_CASES)
def test_compact_parity(gpu, case):
    R, K, B, p, dead = case
    _say(f"compact {case}")
    rng = np.random.default_rng(R * 1000 + K)
    vals, col, alive = _layer(rng, R, 2 * K, K, B, p, sentinel_frac=0.1)
    for r in dead:
        alive[r] = False
    ov, oc, oa, kn = _opt().compact_single_layer(*_gpu_layer(vals, col, alive))
    rv, rc, ra, rk = O.compact_topology(vals, col, alive)
    assert kn == rk
    np.testing.assert_array_equal(_np(oc), rc)
    np.testing.assert_array_equal(_np(oa), ra)
    np.testing.assert_array_equal(_np(ov), rv)


IMP_CASES = [
    # (R1, K1, C_ff, R2, K2)
    (32, 16, 128, 128, 24),
    (64, 40, 256, 200, 8),              # fc2 rows past C_ff are ignored
    (16, 70, 512, 300, 16),             # fc2 shorter than C_ff
    (1, 1, 1, 1, 1),
]


@pytest.mark.parametrize("case", IMP_CASES)
def test_column_importance_parity(gpu, case):
    R1, K1, C_ff, R2, K2 = case
    _say(f"importance {case}")
    rng = np.random.default_rng(R1 + 7 * K1 + C_ff)
    c1 = rng.integers(0, C_ff, size=(R1, K1)).astype(np.int32)
    c1[rng.random((R1, K1)) < 0.1] = -1
    over = rng.random((R1, K1)) < 0.05
    c1[over] = C_ff + 1
    a1 = rng.random((R1, K1)) < 0.7
    a2 = rng.random((R2, K2)) < 0.5
    c2 = rng.integers(0, 8, size=(R2, K2)).astype(np.int32)
    got = _opt().compute_column_importance(T.to_gpu(a1), T.to_gpu(a2), T.to_gpu(c1), T.to_gpu(c2), C_ff)
    np.testing.assert_array_equal(_np(got), O.column_importance(a1, a2, c1, C_ff))


def _importance(name):
    rng = np.random.default_rng(11)
    if name == "ties":
        return rng.integers(0, 5, size=300).astype(np.float32)
    if name == "special":
        return np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.0, np.nan, 3.0, -1.0, 0.0], np.float32)
    if name == "wide":
        wide = rng.standard_normal(5000).astype(np.float32)
        wide[::7] = 1.5
        return wide
    if name == "one":
        return np.array([2.0], np.float32)
    return rng.integers(0, 50, size=16384).astype(np.float32)      # the largest C_ff accepted


@pytest.mark.parametrize("name", ["ties", "special", "wide", "one", "max"])
def test_column_permutation_parity(gpu, name):
    imp = _importance(name)
    _say(f"permutation {name} C={imp.shape[0]}")
    got = _np(_opt().compute_permutation(T.to_gpu(imp)))
    np.testing.assert_array_equal(got, O.column_permutation(imp))


@pytest.mark.parametrize("is_column_dim", [True, False])
def test_apply_permutation_parity(gpu, is_column_dim):
    _say(f"apply permutation column={is_column_dim}")
    rng = np.random.default_rng(5 if is_column_dim else 6)
    C_ff, K, B = 96, 70, 16
    R = 40 if is_column_dim else C_ff
    vals, col, alive = _layer(rng, R, C_ff, K, B, 0.6, sentinel_frac=0.1, over_frac=0.05 if is_column_dim else 0.0)
    perm = rng.permutation(C_ff).astype(np.int32)
    inp = _gpu_layer(vals, col, alive)
    ov, oc, oa = _opt().apply_permutation_to_block_ell(*inp, T.to_gpu(perm), is_column_dim=is_column_dim)
    if is_column_dim:                  # the tiles keep their slots: the same tensors come back
        assert ov is inp[0] and oa is inp[2]
    rv, rc, ra = O.apply_permutation(vals, col, alive, perm, is_column_dim)
    np.testing.assert_array_equal(_np(oc), rc)
    np.testing.assert_array_equal(_np(oa), ra)
    np.testing.assert_array_equal(_np(ov), rv)


@pytest.mark.parametrize("tpm", [1, 4, 16])
def test_k_active_macros_parity(gpu, tpm):
    _say(f"k_active tpm={tpm}")
    rng = np.random.default_rng(tpm)
    R, K, C_ff = 64, 33, 200
    col = rng.integers(-1, C_ff, size=(R, K)).astype(np.int32)
    alive = rng.random((R, K)) < 0.3
    # the largest column sits in a dead slot: it must not count
    col[0, 0], alive[0, 0] = C_ff + 50, False
    got = int(_np(_opt().compute_k_active_macros(T.to_gpu(alive), T.to_gpu(col), tpm, C_ff)))
    assert got == O.k_active_macros(alive, col, tpm)
    none = np.zeros_like(alive)
    assert int(_np(_opt().compute_k_active_macros(T.to_gpu(none), T.to_gpu(col), tpm, C_ff))) == 0


def test_reorder_pipeline_and_forward_invariance(gpu):
    """Importance -> permutation -> gate/up rows gathered and down columns remapped, as the
    reference's reorder step does for one FFN; the forward output must not change.  The down
    projection sums its tiles in the order of their d_ff columns (it stages h through LDS by
    column range), so the permutation reorders that float32 sum: outputs may differ by one bf16
    ulp after rounding, and by no more."""
    import torch
    _say("pipeline d_model=256 d_ff=1024 B=32")
    rng = np.random.default_rng(21)
    d_model, d_ff, B, N = 256, 1024, 32, 96
    g, u, d = T.ffn_weights(rng, d_model, d_ff, B, 0.25)
    C_ff = d_ff // B
    # the reference scores d_ff columns from the down projection's column indices (fc1 role) and
    # the up/gate rows (fc2 role); all slots alive here except the sentinels
    d_alive = d[1] >= 0
    g_alive = g[1] >= 0
    opt = _opt()
    imp = opt.compute_column_importance(T.to_gpu(d_alive), T.to_gpu(g_alive), T.to_gpu(d[1]), T.to_gpu(g[1]),
                                        C_ff)
    perm = opt.compute_permutation(imp)
    ref_perm = O.column_permutation(O.column_importance(d_alive, g_alive, d[1], C_ff))
    np.testing.assert_array_equal(_np(perm), ref_perm)

    def gathered(w, alive):
        v, c, _ = opt.apply_permutation_to_block_ell(*_gpu_layer(w[0], w[1], alive), perm, is_column_dim=False)
        return v, c

    g2, u2 = gathered(g, g_alive), gathered(u, u[1] >= 0)
    dv, dc, _ = opt.apply_permutation_to_block_ell(*_gpu_layer(d[0], d[1], d_alive), perm, is_column_dim=True)
    x = T.to_gpu_bf16(T.act(rng, N, d_model))
    y0 = T.abi_swiglu(x, T.gpu_weight(g), T.gpu_weight(u), T.gpu_weight(d))[0]
    y1 = T.abi_swiglu(x, g2, u2, (dv, dc))[0]
    torch.cuda.synchronize()
    a, b = _np(y0).astype(np.float64), _np(y1).astype(np.float64)
    ulp = 2.0 ** -7 * np.maximum(np.abs(a), np.abs(b))          # one bf16 ulp bounds the rounding flip
    assert np.all(np.abs(a - b) <= ulp + 1e-5 * np.abs(a).max())
    assert np.mean(a != b) < 0.05


def test_abi_argument_errors(gpu):
    import torch
    A = T.abi()
    lib = A.load()
    v = torch.zeros(4, 3, 16, 16, dtype=torch.bfloat16, device="cuda")
    c = torch.zeros(4, 3, dtype=torch.int32, device="cuda")
    a = torch.ones(4, 3, dtype=torch.uint8, device="cuda")
    ov, oc, oa = torch.empty_like(v), torch.empty_like(c), torch.empty_like(a)
    P = T.ptr
    # K_new beyond K
    assert lib.lbk_topology_compact_bf16(P(v), P(c), P(a), 4, 3, 16, 4, P(ov), P(oc), P(oa), T.stream()) == A.LBK_ERR_ARG
    # row mode needs one row per permutation entry
    perm = torch.arange(8, dtype=torch.int32, device="cuda")
    assert lib.lbk_apply_permutation_bf16(P(v), P(c), P(a), 4, 3, 16, P(perm), 8, 0, P(ov), P(oc), P(oa),
                                          T.stream()) == A.LBK_ERR_SHAPE
    # unsupported tile size
    assert lib.lbk_topology_compact_bf16(P(v), P(c), P(a), 4, 3, 24, 2, P(ov), P(oc), P(oa), T.stream()) == A.LBK_ERR_TILE
    assert lib.lbk_k_active_macros(P(c), P(a), 4, 3, 0, P(oc), T.stream()) == A.LBK_ERR_ARG
    with pytest.raises(RuntimeError):
        _opt().compute_permutation(torch.zeros(4))


def test_optimizer_rows_parity(gpu):
    import torch
    _say("optimizer rows")
    rng = np.random.default_rng(8)
    C_ff, K, B = 48, 6, 16
    perm = rng.permutation(C_ff).astype(np.int32)
    mu = rng.standard_normal((C_ff, K, B, B)).astype(np.float32)
    nu = rng.random((C_ff, K, B, B)).astype(np.float32)
    odd = rng.integers(0, 255, size=(C_ff, 5)).astype(np.uint8)      # 5-byte rows: the byte path
    other = rng.standard_normal((7, 3)).astype(np.float32)
    state = {"step": torch.tensor(3.0), "exp_avg": T.to_gpu(mu), "exp_avg_sq": T.to_gpu(nu),
             "extra": [T.to_gpu(odd), T.to_gpu(other)]}
    out = _opt().apply_permutation_to_optimizer(state, T.to_gpu(perm), "fc2_values", is_column_dim=False)
    ref = O.permute_optimizer_rows({"exp_avg": mu, "exp_avg_sq": nu, "extra": [odd, other]}, perm, False)
    np.testing.assert_array_equal(_np(out["exp_avg"]), ref["exp_avg"])
    np.testing.assert_array_equal(_np(out["exp_avg_sq"]), ref["exp_avg_sq"])
    np.testing.assert_array_equal(_np(out["extra"][0]), ref["extra"][0])
    assert out["extra"][1] is state["extra"][1] and out["step"] is state["step"]
    same = _opt().apply_permutation_to_optimizer(state, T.to_gpu(perm), "fc1_values", is_column_dim=True)
    assert same["exp_avg"] is state["exp_avg"]


def test_full_reorder_step_parity(gpu):
    _say("full reorder step")
    rng = np.random.default_rng(9)
    C_ff, R_model, K1, K2, B, tpm = 64, 12, 20, 10, 16, 8
    v1, c1, a1 = _layer(rng, R_model, C_ff, K1, B, 0.5, sentinel_frac=0.1)
    v2, c2, a2 = _layer(rng, C_ff, 24, K2, B, 0.5)
    mu = rng.standard_normal((C_ff, K2, B, B)).astype(np.float32)
    got = _opt().full_reorder_step(*_gpu_layer(v1, c1, a1), *_gpu_layer(v2, c2, a2), {"exp_avg": T.to_gpu(mu)},
                                   C_ff, tpm)
    perm = O.column_permutation(O.column_importance(a1, a2, c1, C_ff))
    r1 = O.apply_permutation(v1, c1, a1, perm, True)
    r2 = O.apply_permutation(v2, c2, a2, perm, False)
    for g_, r_ in zip(got[:6], r1 + r2):
        np.testing.assert_array_equal(_np(g_), r_)
    np.testing.assert_array_equal(_np(got[6]["exp_avg"]), mu[perm])
    assert int(_np(got[7])) == O.k_active_macros(r1[2], r1[1], tpm)


CSC_CASES = [
    # (R, K, C, sentinel_frac)
    (32, 32, 128, 0.1),
    (128, 8, 32, 0.0),
    (5, 300, 700, 0.3),
    (64, 64, 16384, 0.05),             # the largest C accepted: scan over 16 chunks
    (3, 4, 10, 1.0),                   # every slot dead: empty index
]


@pytest.mark.parametrize("case", CSC_CASES)
def test_transposed_index_parity(gpu, case):
    R, K, C_, sf = case
    _say(f"transposed index {case}")
    rng = np.random.default_rng(R + K + C_)
    col = rng.integers(0, C_ + 2, size=(R, K)).astype(np.int32)      # a few columns past C
    col[rng.random((R, K)) < sf] = -1
    ptr, ent = _opt().transposed_index(T.to_gpu(col), C_)
    rp, re_ = O.transposed_index(col, C_)
    np.testing.assert_array_equal(_np(ptr), rp)
    np.testing.assert_array_equal(_np(ent), re_)
