"""Parity of the storage-format bridges against the oracle (bit-exact: copies and integer
selection), through looped_blockell.interop over the C ABI, and the packed ternary file round
trip.  Cases cover B in {16, 32, 64}, bf16 and fp32 weights, the -1 sentinel, duplicate
columns in a row (the last slot wins, as in the reference's scatter loop), equal-norm blocks
(ties go to the smaller column) and corrupted or mismatched ternary files.
"""

import numpy as np
import pytest

import lbk_testlib as T
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[format] {msg}", flush=True)


def _ix():
    from looped_blockell import interop
    return interop


def _torch_dtype(name):
    import torch
    return {"bf16": torch.bfloat16, "fp32": torch.float32}[name]


def _dense(rng, out_f, in_f, dt):
    w = rng.standard_normal((out_f, in_f)).astype(np.float32)
    return O.bf16_round(w) if dt == "bf16" else w


CASES = [(16, "bf16", 64, 128), (32, "fp32", 96, 256), (64, "bf16", 128, 192), (32, "bf16", 32, 64)]


@pytest.mark.parametrize("B,dt,out_f,in_f", CASES)
def test_dense_to_block_ell_parity(gpu, B, dt, out_f, in_f):
    _say(f"dense_to_block_ell B={B} {dt} {out_f}x{in_f}")
    w = _dense(np.random.default_rng(B + out_f), out_f, in_f, dt)
    vals, cols = _ix().dense_to_block_ell(T.to_gpu(w, _torch_dtype(dt)), tile_size=B)
    rv, rc = O.dense_to_block_ell(w, tile_size=B)
    np.testing.assert_array_equal(T.to_np(cols), rc)
    np.testing.assert_array_equal(T.to_np(vals), rv)


@pytest.mark.parametrize("B,dt,out_f,in_f", CASES)
def test_block_ell_to_dense_parity(gpu, B, dt, out_f, in_f):
    _say(f"block_ell_to_dense B={B} {dt} {out_f}x{in_f}")
    rng = np.random.default_rng(7 * B + in_f)
    R, Cb = out_f // B, in_f // B
    K = max(2, Cb // 2)
    vals = rng.standard_normal((R, K, B, B)).astype(np.float32)
    vals = O.bf16_round(vals) if dt == "bf16" else vals
    col = rng.integers(0, Cb, size=(R, K)).astype(np.int32)        # duplicates within a row happen
    col[0, :2] = col[0, 2] if K > 2 else 0                            # ... and one is forced
    col[rng.random((R, K)) < 0.15] = -1
    got = _ix().block_ell_to_dense(T.to_gpu(vals, _torch_dtype(dt)), T.to_gpu(col), out_f, in_f)
    np.testing.assert_array_equal(T.to_np(got), O.block_ell_to_dense(vals, col, out_f, in_f))


def test_gather_tiles_sentinel_and_range(gpu):
    _say("gather_tiles")
    rng = np.random.default_rng(2)
    B, out_f, in_f = 16, 64, 96
    w = rng.standard_normal((out_f, in_f)).astype(np.float32)
    col = np.array([[0, 5, -1], [2, 2, 1], [6, 3, 4], [-1, -1, 0]], np.int32)     # 6 is past C = 6
    got = T.to_np(_ix().gather_tiles(T.to_gpu(w), T.to_gpu(col), B))
    blocks = w.reshape(4, B, 6, B).transpose(0, 2, 3, 1)
    for r in range(4):
        for k in range(3):
            c = col[r, k]
            ref = blocks[r, c] if 0 <= c < 6 else np.zeros((B, B), np.float32)
            np.testing.assert_array_equal(got[r, k], ref)


@pytest.mark.parametrize("dt,density,B", [("bf16", 0.5, 32), ("fp32", 0.25, 32), ("bf16", 1.0, 32),
                                          ("bf16", 0.25, 16), ("fp32", 0.5, 64)])
def test_create_block_ell_from_dense_parity(gpu, dt, density, B):
    from looped_blockell.layers import block_ell_to_dense, create_block_ell_from_dense
    _say(f"create_block_ell_from_dense {dt} density={density} B={B}")
    rng = np.random.default_rng(int(density * 100) + B)
    out_f, in_f = 4 * B, 16 * B
    w = _dense(rng, out_f, in_f, dt)
    # equal-norm blocks: row 0 holds copies of one block (ties go to the smaller column)
    w[:B, B:2 * B] = w[:B, 3 * B:4 * B] = w[:B, 5 * B:6 * B] = w[:B, 0:B]
    e = create_block_ell_from_dense(T.to_gpu(w, _torch_dtype(dt)), tile_size=B, density=density)
    rv, rc, cfg = O.create_block_ell_from_dense(w, tile_size=B, density=density)
    assert e.config.K == cfg.K
    np.testing.assert_array_equal(T.to_np(e.col_indices), rc)
    np.testing.assert_array_equal(T.to_np(e.values), rv)
    np.testing.assert_array_equal(T.to_np(block_ell_to_dense(e)), O.block_ell_to_dense(rv, rc, out_f, in_f))


def test_dense_checkpoint_bridge_through_mlp(gpu):
    """A dense PyTorch checkpoint of an MLP loads into MLPBlock (tiles gathered at the layer's
    topology) and the forward equals the oracle on those tiles; dense_state_dict gives back the
    dense weights with dead tiles zero."""
    import torch
    from looped_blockell.layers import MLPBlock
    _say("dense checkpoint bridge d_model=256 d_ff=512 B=32")
    rng = np.random.default_rng(12)
    d_model, d_ff, B, N = 256, 512, 32, 48
    m = MLPBlock(d_model, d_ff, use_swiglu=True, tile_size=B, density=0.5, device="cuda")
    dense = {f"{n}.weight": O.bf16_round((rng.standard_normal(s) * 0.05).astype(np.float32))
             for n, s in (("w_gate", (d_ff, d_model)), ("w_up", (d_ff, d_model)), ("w_down", (d_model, d_ff)))}
    sd = {k: T.to_gpu(v) for k, v in dense.items()}
    done = _ix().load_dense_state_dict(m, sd)
    assert sorted(done) == ["w_down", "w_gate", "w_up"]
    m.w_down.alive_mask[0, 0] = False                       # one pruned tile: dense export writes zeros
    x = T.act(rng, N, d_model)
    with torch.no_grad():
        y = T.to_np(m(T.to_gpu_bf16(x)))
    tiles = {}
    for n in ("w_gate", "w_up", "w_down"):
        lin = getattr(m, n)
        cols = T.to_np(lin.col_indices)
        all_tiles, _ = O.dense_to_block_ell(dense[f"{n}.weight"], B)          # [R, C, B_in, B_out]
        np.testing.assert_array_equal(T.to_np(lin.values), np.take_along_axis(all_tiles, cols[:, :, None, None], 1))
        tiles[n] = (T.to_np(lin.values).astype(np.float64), T.to_np(lin.effective_col_indices()))
    ref = O.swiglu_fwd(x.astype(np.float64), tiles["w_gate"], tiles["w_up"], tiles["w_down"])[0]
    err, _ = T.rel_err(y, ref)
    assert err <= 1e-2
    back = _ix().dense_state_dict(m)
    for n in ("w_gate", "w_up", "w_down"):
        lin = getattr(m, n)
        v, c = T.to_np(lin.values), T.to_np(lin.effective_col_indices())
        np.testing.assert_array_equal(T.to_np(back[f"{n}.weight"]),
                                      O.block_ell_to_dense(v, c, lin.out_features, lin.in_features))


def _ternary_triple(rng, R, K, B, Cb):
    import torch
    from looped_blockell.layers import TernaryBlockELLWeight
    t = rng.integers(-1, 2, size=(R, K, B, B)).astype(np.int8)
    s = (rng.random((R, K)) * 0.05 + 0.01).astype(np.float32)
    c = np.stack([rng.choice(Cb, size=K, replace=False) for _ in range(R)]).astype(np.int32)
    w = TernaryBlockELLWeight.from_codes(T.to_gpu(t), T.to_gpu(s), T.to_gpu(c))
    return w, t


def test_ternary_file_round_trip_and_forward(gpu, tmp_path):
    import torch
    from looped_blockell.layers import TernaryMLPBlock
    _say("ternary file round trip d_model=256 d_ff=512 B=32")
    rng = np.random.default_rng(5)
    d_model, d_ff, B = 256, 512, 32
    g, tg = _ternary_triple(rng, d_ff // B, 4, B, d_model // B)
    u, _ = _ternary_triple(rng, d_ff // B, 4, B, d_model // B)
    d, _ = _ternary_triple(rng, d_model // B, 8, B, d_ff // B)
    np.testing.assert_array_equal(T.to_np(g.packed).view(np.uint32), O.pack_ternary(tg))   # the file's words
    path = str(tmp_path / "ffn.safetensors")
    ix = _ix()
    ix.save_ternary(path, {"w_gate": g, "w_up": u, "w_down": d},
                    in_features={"w_gate": d_model, "w_up": d_model, "w_down": d_ff}, metadata={"step": 3})
    ws, meta = ix.load_ternary(path)
    assert meta == {"step": "3"}
    for n, w in (("w_gate", g), ("w_up", u), ("w_down", d)):
        for a, b in zip(ws[n].triple(), w.triple()):
            assert torch.equal(a, b)
    x = T.to_gpu_bf16(T.act(rng, 40, d_model))
    with torch.no_grad():
        y0 = TernaryMLPBlock(g, u, d)(x)
        y1 = TernaryMLPBlock(ws["w_gate"], ws["w_up"], ws["w_down"])(x)
    assert torch.equal(y0, y1)


def test_ternary_file_rejects_bad_content(gpu, tmp_path):
    import torch
    _say("ternary file rejections")
    rng = np.random.default_rng(6)
    ix = _ix()
    w, _ = _ternary_triple(rng, 4, 3, 16, 8)
    packed = w.packed.clone()
    words = T.to_np(packed).view(np.uint32).copy()
    words[1, 2, 3, 0] = (words[1, 2, 3, 0] & ~np.uint32(0b11 << 10)) | np.uint32(0b10 << 10)   # one 0b10 field
    words[3, 0, 0, 0] = np.uint32(0xAAAAAAAA)                                                # sixteen more
    bad = torch.from_numpy(words.view(np.int32)).cuda()
    assert ix.check_ternary_codes(bad) == 17
    assert ix.check_ternary_codes(w.packed) == 0
    p1 = str(tmp_path / "bad.safetensors")
    ix.save_ternary(p1, {"w": (bad, w.scales, w.col_indices)})
    with pytest.raises(ValueError, match="17 invalid"):
        ix.load_ternary(p1)
    p2 = str(tmp_path / "range.safetensors")
    ix.save_ternary(p2, {"w": w}, in_features={"w": 16 * 4})           # columns up to 7 exceed C = 4
    with pytest.raises(ValueError, match="column index"):
        ix.load_ternary(p2)
    from safetensors.torch import save_file
    p3 = str(tmp_path / "version.safetensors")
    save_file({"w.packed": w.packed.cpu(), "w.scales": w.scales.cpu(), "w.col_indices": w.col_indices.cpu()}, p3,
              metadata={"format": ix.TERNARY_FORMAT, "version": "99", "weights": '["w"]', "B": '{"w": 16}'})
    with pytest.raises(ValueError, match="version"):
        ix.load_ternary(p3)


def test_format_abi_argument_errors(gpu):
    import torch
    A = T.abi()
    lib = A.load()
    P = T.ptr
    d = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda")
    c = torch.zeros(4, 2, dtype=torch.int32, device="cuda")
    v = torch.zeros(4, 2, 16, 16, dtype=torch.bfloat16, device="cuda")
    assert lib.lbk_dense_to_block_ell(P(d), 64, 3, 4, 4, 16, P(c), 2, P(v), T.stream()) == A.LBK_ERR_ALIGN
    assert lib.lbk_dense_to_block_ell(P(d), 32, 2, 4, 4, 16, P(c), 2, P(v), T.stream()) == A.LBK_ERR_ARG   # ld < C*B
    assert lib.lbk_block_ell_to_dense(P(v), P(c), 4, 2, 24, 4, 2, P(d), 64, T.stream()) == A.LBK_ERR_TILE
    assert lib.lbk_block_ell_topk_columns(P(d), 64, 2, 4, 4, 16, 5, P(c), T.stream()) == A.LBK_ERR_ARG    # K > C
    with pytest.raises(RuntimeError, match="GPU"):
        _ix().dense_to_block_ell(torch.zeros(32, 32), 16)
