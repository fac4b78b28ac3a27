"""The HIP kernels against the committed golden fixtures (tests/golden/), through the C ABI; the
expectations come from the files, not from a run of the oracle.  bf16 SwiGLU: max-abs error
<= 1e-2 of max |expected|; ternary: int32 block partials and the bf16 outputs bit-exact."""

import os

import numpy as np
import pytest

import lbk_testlib as T

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-2


def _f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _cases(z, prefix):
    return sorted({k.split("_")[0] for k in z.files if k.startswith(prefix)})


def test_swiglu_tiny_golden(gpu):
    z = np.load(os.path.join(HERE, "swiglu_tiny.npz"))
    for case in _cases(z, "swiglu"):
        print(f"[golden] {case}", flush=True)
        f = lambda k: z[f"{case}_{k}"]
        x = T.to_gpu_bf16(_f32(f("x")))
        w = [(T.to_gpu_bf16(_f32(f("v" + n))), T.to_gpu(f("c" + n).astype(np.int32))) for n in "gud"]
        out = T.abi_swiglu(x, *w, add_residual=True)[0]
        rel, ab = T.rel_err(T.to_np(out), f("out"))
        assert rel <= TOL, f"{case}: rel {rel} abs {ab}"


def test_ternary_tiny_golden(gpu):
    from looped_blockell import kernels
    z = np.load(os.path.join(HERE, "ternary_tiny.npz"))
    for case in _cases(z, "ternary"):
        print(f"[golden] {case}", flush=True)
        f = lambda k: z[f"{case}_{k}"]
        packed = kernels.pack_ternary(T.to_gpu(f("t")))
        y, part = kernels.ternary_matmul(T.to_gpu(f("xq")), T.to_gpu(f("sx")), packed, T.to_gpu(f("s")),
                                         T.to_gpu(f("col").astype(np.int32)), want_partials=True)
        assert np.array_equal(T.to_np(part), f("partials")), case
        assert np.array_equal(T.to_np(y), f("y")), case
