"""GPU tests of the looped core (lbk_looped_core_bf16 / lbk_looped_core_persistent_bf16,
titan::looped_core, looped_blockell.layers.LoopedCore): per iteration the diagonal injection,
n_core distinct pre-norm SwiGLU blocks and the per-sequence depth freeze
(reference looped_blockell/looping/looped_model.py:293-340, interop/pt_model.py:1441-1509),
against the float64 oracle (oracle.looped_core), with the bf16 tolerance
max|y - ref| <= 1e-2 * max|ref|; and exact properties: rows of depth 0 keep h_in bit for bit, a
row of depth d equals the same call with L = d, and with one block, no injection and no depths
the core equals the looped block (titan::looped_swiglu) bit for bit."""

import numpy as np
import pytest
import torch

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _say(msg):
    print(msg, flush=True)


def _f64_blocks(blocks):
    f = lambda w: (w[0].astype(np.float64), w[1])
    return [(s.astype(np.float64), f(g), f(u), f(d), None if bs is None else tuple(b.astype(np.float64) for b in bs))
            for (s, g, u, d, bs) in blocks]


def _inputs(rng, N, d_model, n_seq):
    h = T.act(rng, N, d_model)
    e = T.act(rng, N, d_model)
    la = (0.3 * rng.standard_normal(d_model)).astype(np.float32)
    ld = (0.5 * rng.standard_normal(d_model)).astype(np.float32)
    return h, e, la, ld


CORE_CASES = [
    # (d_model, d_ff, B, density, N, seq_len, n_core, L, bias, shared, path)
    (256, 1024, 32, 0.25, 200, 25, 2, 3, True, False, "split"),
    (512, 1024, 16, 0.25, 260, 20, 3, 4, False, True, "split"),
    (256, 512, 32, 0.5, 40, 8, 2, 3, True, False, "decode"),
    (128, 512, 64, 0.5, 100, 10, 2, 3, True, False, "rowblock"),
]


# the persistent launch takes the two-kernel shapes only (its refusal of the others is tested below)
@pytest.mark.parametrize("case,persistent", [(c, False) for c in CORE_CASES] +
                         [(c, True) for c in CORE_CASES if c[-1] == "split"])
def test_looped_core_parity(gpu, case, persistent):
    d_model, d_ff, B, dens, N, S, n_core, L, bias, shared, path = case
    _say(f"looped core {case} persistent={persistent}")
    rng = np.random.default_rng(abs(hash(case[:10])) % 2 ** 31)
    blocks = T.core_blocks(rng, n_core, d_model, d_ff, B, dens, bias=bias, shared=shared, sentinel_frac=0.05)
    n_seq = (N + S - 1) // S
    depths = rng.integers(0, L + 2, size=n_seq).astype(np.int32)
    depths[0], depths[-1] = 0, L + 3          # a sequence that never runs, one deeper than L
    h, e, la, ld = _inputs(rng, N, d_model, n_seq)
    bt = T.core_blocks_gpu(blocks)
    ht, et = T.to_gpu_bf16(h), T.to_gpu_bf16(e)
    lat, ldt, dt = T.to_gpu(la), T.to_gpu(ld), T.to_gpu(depths)
    out = T.abi_looped_core(ht, bt, L, e_t=et, log_A_t=lat, log_dt_t=ldt, depths_t=dt, seq_len=S,
                            persistent=persistent)
    torch.cuda.synchronize()
    got = T.to_np(out)
    ref = O.looped_core(h.astype(np.float64), e.astype(np.float64), la, ld, _f64_blocks(blocks), L, depths=depths,
                        seq_len=S)
    rel, ab = T.rel_err(got, ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
    # depth 0: h_in bit for bit
    assert np.array_equal(got[:S], h[:S])
    # the torch operator gives the same bits
    ws = [(b[1][0], b[1][1], b[2][0], b[2][1], b[3][0], b[3][1]) for b in bt]
    from looped_blockell import kernels
    op = kernels.looped_core(ht, et, lat, ldt, [b[0] for b in bt], [w[0] for w in ws], [w[1] for w in ws],
                             [w[2] for w in ws], [w[3] for w in ws], [w[4] for w in ws], [w[5] for w in ws], L,
                             biases=[b[4] if b[4] is not None else (None, None, None) for b in bt], depths=dt,
                             seq_len=S, persistent=persistent)
    assert torch.equal(op, out)


@pytest.mark.parametrize("persistent", [False, True])
def test_looped_core_depth_equals_shorter_loop(gpu, persistent):
    """A sequence of depth d inside an L-iteration call equals an L = d call on its rows, bit for bit
    (every row runs the same arithmetic; frozen rows only stop being updated)."""
    rng = np.random.default_rng(4242)
    d_model, d_ff, B, N, S, L = 256, 1024, 32, 192, 32, 4
    _say(f"looped core depth == shorter loop persistent={persistent}")
    blocks = T.core_blocks(rng, 2, d_model, d_ff, B, 0.25)
    bt = T.core_blocks_gpu(blocks)
    h, e, la, ld = _inputs(rng, N, d_model, N // S)
    ht, et, lat, ldt = T.to_gpu_bf16(h), T.to_gpu_bf16(e), T.to_gpu(la), T.to_gpu(ld)
    depths = np.array([0, 1, 2, 3, 4, 9], np.int32)
    full = T.to_np(T.abi_looped_core(ht, bt, L, e_t=et, log_A_t=lat, log_dt_t=ldt, depths_t=T.to_gpu(depths),
                                     seq_len=S, persistent=persistent))
    for dep in range(0, L + 1):
        short = T.to_np(T.abi_looped_core(ht, bt, dep, e_t=et, log_A_t=lat, log_dt_t=ldt, persistent=persistent))
        for b in np.nonzero(np.minimum(depths, L) == dep)[0]:
            rows = slice(b * S, (b + 1) * S)
            assert np.array_equal(full[rows], short[rows]), f"sequence {b} (depth {depths[b]})"


def test_looped_core_one_block_equals_looped_swiglu(gpu):
    """One block, no injection, no depths: the looped block's operators bit for bit (launches and the
    persistent launch)."""
    rng = np.random.default_rng(77)
    d_model, d_ff, B, N, L = 512, 2048, 32, 300, 3
    _say("looped core n_core=1 == looped_swiglu")
    blocks = T.core_blocks(rng, 1, d_model, d_ff, B, 0.25)
    bt = T.core_blocks_gpu(blocks)
    ht = T.to_gpu_bf16(T.act(rng, N, d_model))
    sc, g, u, d, _ = bt[0]
    for persistent in (False, True):
        core = T.abi_looped_core(ht, bt, L, persistent=persistent)
        ref = T.abi_looped(ht, sc, g, u, d, L, 1e-5, persistent=persistent, launches=not persistent)
        torch.cuda.synchronize()
        assert torch.equal(core, ref), f"persistent={persistent}"


@pytest.mark.parametrize("persistent", [False, True])
def test_looped_core_full_size_sampled_rows(gpu, persistent):
    """The looped-block geometry at full size (d_model 1024, d_ff 4096, B 32, 25 %, 32 x 512 tokens) with
    n_core = 2 distinct blocks, L = 3, the injection and per-sequence depths 0..4; sampled rows of
    sampled sequences against the oracle."""
    rng = np.random.default_rng(2048)
    d_model, d_ff, B, S, nb, L = 1024, 4096, 32, 512, 32, 3
    N = S * nb
    _say(f"looped core full size n_core=2 L=3 persistent={persistent}")
    blocks = T.core_blocks(rng, 2, d_model, d_ff, B, 0.25)
    bt = T.core_blocks_gpu(blocks)
    h, e, la, ld = _inputs(rng, N, d_model, nb)
    depths = (np.arange(nb) % 5).astype(np.int32)
    out = T.abi_looped_core(T.to_gpu_bf16(h), bt, L, e_t=T.to_gpu_bf16(e), log_A_t=T.to_gpu(la),
                            log_dt_t=T.to_gpu(ld), depths_t=T.to_gpu(depths), seq_len=S, persistent=persistent)
    got = T.to_np(out)
    seqs = [0, 1, 2, 3, 4, 17, 31]
    rows = np.concatenate([b * S + np.sort(rng.choice(S, 12, replace=False)) for b in seqs])
    ref = O.looped_core(h[rows].astype(np.float64), e[rows].astype(np.float64), la, ld, _f64_blocks(blocks), L,
                        depths=np.repeat(depths[seqs], 12), seq_len=1)
    rel, ab = T.rel_err(got[rows], ref)
    assert rel <= TOL, f"rel {rel} abs {ab}"
    assert np.array_equal(got[:S], h[:S])   # depth 0


def test_looped_core_errors(gpu):
    A = T.abi()
    rng = np.random.default_rng(5)
    d_model, d_ff = 256, 512
    h = T.to_gpu_bf16(T.act(rng, 70, d_model))
    bt = T.core_blocks_gpu(T.core_blocks(rng, 2, d_model, d_ff, 32, 0.25))
    assert T.abi_looped_core(h, [], 2, expect=A.LBK_ERR_ARG) == A.LBK_ERR_ARG
    assert T.abi_looped_core(h, bt * 5, 2, expect=A.LBK_ERR_ARG) == A.LBK_ERR_ARG          # 10 > 8 blocks
    assert T.abi_looped_core(h, bt, 2, e_t=h, expect=A.LBK_ERR_NULL) == A.LBK_ERR_NULL      # no log_A / log_dt
    assert T.abi_looped_core(h, bt, 2, depths_t=T.to_gpu(np.ones(70, np.int32)), seq_len=0,
                             expect=A.LBK_ERR_ARG) == A.LBK_ERR_ARG
    b64 = T.core_blocks_gpu(T.core_blocks(rng, 1, d_model, d_ff, 64, 0.5))
    assert T.abi_looped_core(h, b64, 2, persistent=True, expect=A.LBK_ERR_SHAPE) == A.LBK_ERR_SHAPE
    mixed = T.core_blocks_gpu(T.core_blocks(rng, 1, d_model, d_ff, 32, 0.25, shared=True)) + bt[:1]
    assert T.abi_looped_core(h, mixed, 2, persistent=True, expect=A.LBK_ERR_SHAPE) == A.LBK_ERR_SHAPE
    # L = 0 copies h
    assert torch.equal(T.abi_looped_core(h, bt, 0), h)


def test_looped_core_layer_inference_and_training(gpu):
    """LoopedCore: the operator path (no gradients) against the differentiable composition (with
    gradients) on the same parameters, and gradients reaching every parameter."""
    from looped_blockell.layers import LoopedCore
    torch.manual_seed(11)
    m = LoopedCore(256, 1024, n_core=2, tile_size=32, density=0.25, device="cuda")
    with torch.no_grad():
        for mlp in m.mlps:
            for lin in (mlp.w_gate, mlp.w_up, mlp.w_down):
                lin.bias.copy_(0.05 * torch.randn_like(lin.bias))
        m.log_A.copy_(0.2 * torch.randn_like(m.log_A))
    h = torch.randn(4, 24, 256, device="cuda").to(torch.bfloat16)
    e = torch.randn(4, 24, 256, device="cuda").to(torch.bfloat16)
    depths = torch.tensor([0, 3, 1, 2], device="cuda", dtype=torch.int32)
    with torch.no_grad():
        inf = m(h, e, depths, L=3)
    hg = h.clone().requires_grad_(True)
    tr = m(hg, e, depths, L=3)
    assert T.rel_err(T.to_np(tr), T.to_np(inf))[0] <= TOL
    assert torch.equal(inf[0], h[0])
    tr.float().sum().backward()
    assert hg.grad is not None and m.log_A.grad is not None and m.log_dt.grad is not None
    assert m.mlps[1].w_down.values.grad is not None and m.norms[0].scale.grad is not None
