"""The committed golden fixtures (tests/golden/) are reproduced by the oracle: integers and the
bf16-rounded ternary outputs bit for bit, float64-derived outputs to 1e-12 relative.  A change
to the oracle that moves any of them fails here; the GPU kernels are checked against the same
fixtures in test_gpu_golden.py."""

import json
import os
import sys

import numpy as np

from oracle import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import make_fixtures as MF  # noqa: E402


def test_swiglu_tiny_fixtures_reproduced():
    z = np.load(os.path.join(HERE, "swiglu_tiny.npz"))
    for n, case in enumerate(MF.SWIGLU_TINY):
        got = MF.swiglu_case(1000 + n, *case)
        for k, v in got.items():
            ref = z[f"swiglu{n}_{k}"]
            if k == "out":
                np.testing.assert_allclose(v, ref, rtol=1e-6, atol=1e-7)
            else:
                np.testing.assert_array_equal(v, ref)


def test_ternary_tiny_fixtures_reproduced():
    z = np.load(os.path.join(HERE, "ternary_tiny.npz"))
    for n, case in enumerate(MF.TERNARY_TINY):
        got = MF.ternary_case(2000 + n, *case)
        for k, v in got.items():
            np.testing.assert_array_equal(v, z[f"ternary{n}_{k}"])


def test_small_geometry_summary_reproduced():
    with open(os.path.join(HERE, "small_geometry_summary.json")) as f:
        ref = json.load(f)
    rng = np.random.default_rng(ref["seed"])
    g, u, d = (O.random_topology(R, C, 4, rng) for R, C in ((64, 16), (64, 16), (16, 64)))
    vals = [(rng.standard_normal((R, 4, 16, 16)) * 0.02).astype(np.float32) for R in (64, 64, 16)]
    x = rng.standard_normal((512, 256)).astype(np.float32)
    out = O.swiglu_fwd(x.astype(np.float64), (vals[0].astype(np.float64), g), (vals[1].astype(np.float64), u),
                       (vals[2].astype(np.float64), d))[0]
    assert list(out.shape) == ref["shape"]
    np.testing.assert_allclose(out.sum(), ref["sum"], rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(np.abs(out).sum(), ref["abs_sum"], rtol=1e-12)
    np.testing.assert_allclose(out[0, :8], ref["row0_head"], rtol=1e-12)
    np.testing.assert_allclose(out[511, -8:], ref["row511_tail"], rtol=1e-12)
