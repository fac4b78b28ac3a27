"""CPU-side tests: the C ABI library's exports and host validation, the torch
operator registrations (shape functions), and the layer API's host logic.
No kernel is launched here."""

import ctypes as C
import os
import re

import numpy as np
import pytest
import torch

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lbk.h")
PKG = os.path.join(ROOT, "looped-blockell-tpu_amd", "looped_blockell")
LIB = os.path.join(PKG, "liblbk.so")
EXT = os.path.join(PKG, "_titan_ext.so")

needs_lib = pytest.mark.skipif(not os.path.exists(LIB), reason="liblbk.so not built")
needs_ext = pytest.mark.skipif(not os.path.exists(EXT), reason="_titan_ext.so not built")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lbk_[a-z0-9_]+)\s*\(", text)))


@needs_lib
def test_library_exports_every_header_symbol():
    from looped_blockell import abi
    lib = abi.load()
    declared = header_functions()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in lbk.h but not exported"
    assert sorted(abi.exported_symbols()) == declared


@needs_lib
def test_status_strings_and_version():
    from looped_blockell import abi
    lib = abi.load()
    assert lib.lbk_version() == 1
    assert abi.status_string(0) == "ok"
    for code in range(1, 9):
        assert abi.status_string(code) != "unknown status"
    assert abi.status_string(99) == "unknown status"


def _bell(R=4, K=2, B=32, values=0x1000, col=0x2000):
    from looped_blockell import abi
    return abi.Bell(values, col, R, K, B)


@needs_lib
def test_abi_validation_codes_without_gpu():
    """Every check below returns before any HIP call (host-side validation only)."""
    from looped_blockell import abi as A
    lib = A.load()
    s = C.c_void_p(0)
    y, x = C.c_void_p(0x10000), C.c_void_p(0x20000)
    # bad tile size
    w = _bell(B=24)
    assert lib.lbk_block_ell_matmul_bf16(x, 8, 96, 96, C.byref(w), None, y, 96, s) == A.LBK_ERR_TILE
    # in_features not a multiple of B
    w = _bell(B=32)
    assert lib.lbk_block_ell_matmul_bf16(x, 8, 100, 100, C.byref(w), None, y, 128, s) == A.LBK_ERR_SHAPE
    # negative N
    assert lib.lbk_block_ell_matmul_bf16(x, -1, 64, 64, C.byref(w), None, y, 128, s) == A.LBK_ERR_ARG
    # N = 0 is a no-op even with NULL buffers
    assert lib.lbk_block_ell_matmul_bf16(None, 0, 64, 64, C.byref(w), None, None, 128, s) == A.LBK_OK
    # NULL activations
    assert lib.lbk_block_ell_matmul_bf16(None, 4, 64, 64, C.byref(w), None, y, 128, s) == A.LBK_ERR_NULL
    # misaligned activations
    assert lib.lbk_block_ell_matmul_bf16(C.c_void_p(0x20002), 4, 64, 64, C.byref(w), None, y, 128, s) == A.LBK_ERR_ALIGN
    # NULL values with live blocks
    wnull = A.Bell(0, 0x2000, 4, 2, 32)
    assert lib.lbk_block_ell_matmul_bf16(x, 4, 64, 64, C.byref(wnull), None, y, 128, s) == A.LBK_ERR_NULL


@needs_lib
def test_abi_swiglu_shape_and_workspace_checks():
    from looped_blockell import abi as A
    lib = A.load()
    s = C.c_void_p(0)
    x, out = C.c_void_p(0x10000), C.c_void_p(0x40000)
    g, u = _bell(R=8, K=2, B=32), _bell(R=8, K=2, B=32)
    d = _bell(R=2, K=4, B=32)                              # d_model = 64, d_ff = 256
    # mismatched gate/up R
    u_bad = _bell(R=6, K=2, B=32)
    assert lib.lbk_swiglu_fwd_bf16(x, 4, 64, C.byref(g), C.byref(u_bad), C.byref(d), 0, out, None, None, None,
                                   None, 0, s) == A.LBK_ERR_SHAPE
    # down R inconsistent with d_model
    assert lib.lbk_swiglu_fwd_bf16(x, 4, 96, C.byref(g), C.byref(u), C.byref(d), 0, out, None, None, None,
                                   None, 0, s) == A.LBK_ERR_SHAPE
    # mixed tile sizes
    d16 = _bell(R=4, K=4, B=16)
    assert lib.lbk_swiglu_fwd_bf16(x, 4, 64, C.byref(g), C.byref(u), C.byref(d16), 0, out, None, None, None,
                                   None, 0, s) == A.LBK_ERR_TILE
    # B = 64 uses the general two-kernel path: needs a workspace for h
    g64, u64, d64 = _bell(R=4, K=1, B=64), _bell(R=4, K=1, B=64), _bell(R=1, K=2, B=64)
    need = lib.lbk_swiglu_workspace_bytes(4, 64, C.byref(g64), C.byref(u64), C.byref(d64), 0)
    assert need >= 4 * 256 * 2
    assert lib.lbk_swiglu_fwd_bf16(x, 4, 64, C.byref(g64), C.byref(u64), C.byref(d64), 0, out, None, None, None,
                                   None, 0, s) == A.LBK_ERR_WORKSPACE
    # every path stages h in the workspace unless intermediates go to the caller's h_out
    assert lib.lbk_swiglu_workspace_bytes(4, 64, C.byref(g), C.byref(u), C.byref(d), 0) >= 4 * 256 * 2
    assert lib.lbk_swiglu_workspace_bytes(4, 64, C.byref(g), C.byref(u), C.byref(d), 1) == 0
    assert lib.lbk_looped_workspace_bytes(4, 64, C.byref(g), C.byref(u), C.byref(d)) >= 4 * 64 * 4 + 4 * 256 * 2
    # looped: negative L / eps
    assert lib.lbk_looped_swiglu_bf16(x, 4, 64, C.c_void_p(0x5000), C.c_float(1e-5), -1, C.byref(g), C.byref(u),
                                      C.byref(d), out, None, 0, s) == A.LBK_ERR_ARG
    assert lib.lbk_looped_swiglu_bf16(x, 4, 64, C.c_void_p(0x5000), C.c_float(-1.0), 2, C.byref(g), C.byref(u),
                                      C.byref(d), out, None, 0, s) == A.LBK_ERR_ARG


@needs_lib
def test_abi_ternary_checks():
    from looped_blockell import abi as A
    lib = A.load()
    s = C.c_void_p(0)
    w = A.BellTernary(0x1000, 0x2000, 0x3000, 4, 2, 48)
    assert lib.lbk_ternary_matmul(C.c_void_p(0x10000), C.c_void_p(0x20000), 4, 96, C.byref(w), C.c_void_p(0x30000),
                                  None, s) == A.LBK_ERR_TILE
    w = A.BellTernary(0x1000, 0x2000, 0x3000, 4, 2, 64)
    assert lib.lbk_ternary_matmul(C.c_void_p(0x10000), C.c_void_p(0x20000), 4, 100, C.byref(w),
                                  C.c_void_p(0x30000), None, s) == A.LBK_ERR_SHAPE
    assert lib.lbk_quantize_act_int8(C.c_void_p(0x10000), 4, 12, 12, C.c_void_p(0x20000), C.c_void_p(0x30000),
                                     s) == A.LBK_ERR_ALIGN
    assert lib.lbk_pack_ternary(C.c_void_p(0x1000), 2, 2, 40, C.c_void_p(0x2000), s) == A.LBK_ERR_TILE
    w = A.BellTernary(0x1000, 0x2000, 0x3000, 4, 2, 64)          # d_ff 256
    wd = A.BellTernary(0x1000, 0x2000, 0x3000, 2, 2, 64)         # d_model 128
    assert lib.lbk_ternary_swiglu_workspace_bytes(8, 128, C.byref(w), C.byref(w), C.byref(wd)) >= 8 * 256 * 3
    assert lib.lbk_ternary_swiglu_workspace_bytes(8, 96, C.byref(w), C.byref(w), C.byref(wd)) == 0


# ------------------------------------------------------------------ torch operator registrations

@needs_ext
def test_torch_ops_registered_with_meta_shapes():
    from looped_blockell import kernels
    ops = kernels.ops()
    m = dict(device="meta")
    x = torch.empty(10, 64, dtype=torch.bfloat16, **m)
    vg = torch.empty(8, 2, 32, 32, dtype=torch.bfloat16, **m)
    cg = torch.empty(8, 2, dtype=torch.int32, **m)
    vd = torch.empty(2, 4, 32, 32, dtype=torch.bfloat16, **m)
    cd = torch.empty(2, 4, dtype=torch.int32, **m)
    assert ops.block_ell_swiglu_fwd(x, vg, cg, vg, cg, vd, cd, True).shape == (10, 64)
    r = ops.block_ell_swiglu_fwd_with_intermediate(x, vg, cg, vg, cg, vd, cd, False)
    assert [tuple(t.shape) for t in r] == [(10, 64), (10, 256), (10, 256), (10, 256)]
    assert ops.block_ell_matmul(x, vg, cg).shape == (10, 256)
    assert ops.looped_swiglu(x, torch.empty(64, **m), vg, cg, vg, cg, vd, cd, 8).shape == (10, 64)
    q, s = ops.quantize_act_int8(x)
    assert q.dtype == torch.int8 and s.shape == (10,)
    assert ops.pack_ternary(torch.empty(3, 2, 64, 64, dtype=torch.int8, **m)).shape == (3, 2, 64, 4)
    p = torch.empty(8, 2, 64, 4, dtype=torch.int32, **m)
    sc = torch.empty(8, 2, **m)
    xq = torch.empty(5, 128, dtype=torch.int8, **m)
    y, part = ops.ternary_matmul(xq, torch.empty(5, **m), p, sc, cg, True)
    assert y.shape == (5, 512) and part.shape == (5, 8, 2, 64)
    h = torch.empty(10, 64, dtype=torch.bfloat16, **m)
    assert ops.persistent_mlp_step(h, h, torch.empty(64, **m), torch.empty(64, **m), [torch.empty(64, **m)],
                                   [vg], [cg], [vg], [cg], [vd], [cd]).shape == (10, 64)


@needs_ext
def test_ops_fail_loudly_on_cpu_tensors():
    from looped_blockell import kernels
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    v = torch.zeros(2, 2, 32, 32, dtype=torch.bfloat16)
    c = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError):
        kernels.block_ell_matmul(x, v, c)
    with pytest.raises((RuntimeError, NotImplementedError)):
        kernels.ops().block_ell_matmul(x, v, c)


# ------------------------------------------------------------------ layer API host logic

def test_layer_config_and_topology():
    from looped_blockell.layers import BlockELLConfig, create_random_topology
    cfg = BlockELLConfig(R=4, C=8, K=3, B=16)
    assert (cfg.out_features, cfg.in_features, cfg.density, cfg.total_blocks) == (64, 128, 0.375, 12)
    with pytest.raises(ValueError):
        BlockELLConfig(R=1, C=2, K=3)
    col = create_random_topology(16, 8, 3, 0)
    assert col.dtype == torch.int32 and col.shape == (16, 3)
    for r in range(16):
        assert len(set(col[r].tolist())) == 3
    assert torch.equal(col, create_random_topology(16, 8, 3, 0))


def test_layer_dense_conversions_refuse_cpu_tensors():
    """The dense bridge runs on the HIP kernels only: CPU tensors are refused, never converted
    by a CPU fallback (the GPU parity lives in test_gpu_format.py)."""
    from looped_blockell.layers import block_ell_to_dense, create_block_ell_from_dense
    from looped_blockell.layers.block_ell import BlockELLConfig, BlockELLTensor
    w = torch.randn(64, 128, generator=torch.Generator().manual_seed(3))
    with pytest.raises(RuntimeError, match="GPU"):
        create_block_ell_from_dense(w, tile_size=16, density=1.0)
    e = BlockELLTensor(torch.zeros(4, 8, 16, 16), torch.zeros(4, 8, dtype=torch.int32), BlockELLConfig(4, 8, 8, 16))
    with pytest.raises(RuntimeError, match="GPU"):
        block_ell_to_dense(e)


def test_ternary_file_layout_on_host(tmp_path):
    """save_ternary writes the documented header and the packed words unchanged: the words of
    the oracle's packing round-trip through the file and unpack to the same codes."""
    import json
    from safetensors import safe_open
    from looped_blockell.interop import TERNARY_FORMAT, save_ternary
    rng = np.random.default_rng(4)
    t = rng.integers(-1, 2, size=(3, 2, 32, 32)).astype(np.int8)
    words = O.pack_ternary(t).view(np.int32)
    scales = rng.random((3, 2)).astype(np.float32)
    cols = np.array([[0, 2], [1, -1], [3, 0]], np.int32)
    path = str(tmp_path / "w.safetensors")
    save_ternary(path, {"core.0.w_gate": (torch.from_numpy(words), torch.from_numpy(scales), torch.from_numpy(cols))},
                 in_features={"core.0.w_gate": 128}, metadata={"step": 7})
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata()
        assert meta["format"] == TERNARY_FORMAT and meta["version"] == "1" and meta["user.step"] == "7"
        assert json.loads(meta["weights"]) == ["core.0.w_gate"] and json.loads(meta["B"]) == {"core.0.w_gate": 32}
        back = f.get_tensor("core.0.w_gate.packed").numpy()
        np.testing.assert_array_equal(f.get_tensor("core.0.w_gate.col_indices").numpy(), cols)
        np.testing.assert_array_equal(f.get_tensor("core.0.w_gate.scales").numpy(), scales)
    np.testing.assert_array_equal(O.unpack_ternary(back.view(np.uint32)), t)


def test_blockell_linear_topology_rules():
    from looped_blockell.layers import BlockELLLinear, MLPBlock
    lin = BlockELLLinear(64, 128, tile_size=16, density=1.0)
    assert torch.equal(lin.col_indices, torch.arange(8, dtype=torch.int32).repeat(4, 1))
    m = MLPBlock(256, 1024, use_swiglu=True, tile_size=16, density=0.25)
    assert m.w_gate.K == 4 and m.w_down.K == 16          # K = max(1, int(C * density))
    assert torch.equal(m.w_gate.col_indices, m.w_up.col_indices)   # same shape -> same seed
    m.w_gate.alive_mask[0, 1] = False
    eff = m.w_gate.effective_col_indices()
    assert eff[0, 1].item() == -1 and eff[0, 0].item() == m.w_gate.col_indices[0, 0].item()
    m.w_gate.alive_mask[0, 1] = True
    assert m.w_gate.effective_col_indices()[0, 1].item() == m.w_gate.col_indices[0, 1].item()
