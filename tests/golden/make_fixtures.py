"""Writes the golden fixtures of this directory from the oracle (tests/golden/*.npz, *.json).

The reference repository ships no numeric golden vectors, so these fixtures are the oracle's
outputs on small seeded inputs, frozen: tests/test_golden.py checks that the oracle still
reproduces them bit for bit (a change to the oracle shows up there), and
tests/test_gpu_golden.py checks the HIP kernels against the stored expectations without
running the oracle.  Run from the repository root:  python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402

# (B, K, N, sentinel, m): tiny SwiGLU FFNs, d_model = m*B, d_ff = 2*d_model, gate/up/down all with
# K slots; weights and activations are bf16 values (stored as their 16-bit patterns)
SWIGLU_TINY = [(16, 1, 1, False, 4), (16, 2, 5, True, 4), (32, 3, 33, True, 4), (64, 2, 5, False, 2),
               (32, 1, 1, True, 4)]
# (B, K, N): ternary products, in_features = 4B, 3 block rows
TERNARY_TINY = [(16, 2, 5), (32, 3, 33), (64, 1, 1)]


def bf16(a):
    return O.bf16_round(np.asarray(a, np.float32))


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32).__rshift__(16).astype(np.uint16)


def swiglu_case(seed, B, K, N, sentinel, mult):
    rng = np.random.default_rng(seed)
    d_model = mult * B
    d_ff = 2 * d_model

    def weight(R, C):
        v = bf16(rng.standard_normal((R, K, B, B)) * 0.05)
        c = O.random_topology(R, C, K, rng)
        if sentinel:
            c[0, 0] = -1
        return v, c

    g, u, d = weight(d_ff // B, d_model // B), weight(d_ff // B, d_model // B), weight(d_model // B, d_ff // B)
    x = bf16(rng.standard_normal((N, d_model)))
    f64 = lambda w: (w[0].astype(np.float64), w[1])
    out = O.swiglu_fwd(x.astype(np.float64), f64(g), f64(u), f64(d), add_residual=True)[0]
    return dict(x=bits(x), vg=bits(g[0]), cg=g[1], vu=bits(u[0]), cu=u[1], vd=bits(d[0]), cd=d[1],
                out=out.astype(np.float32))


def ternary_case(seed, B, K, N):
    rng = np.random.default_rng(seed)
    R, C = 3, 4
    t = rng.integers(-1, 2, size=(R, K, B, B)).astype(np.int8)
    s = (rng.random((R, K)) * 0.05 + 0.01).astype(np.float32)
    col = O.random_topology(R, C, K, rng)
    x = rng.standard_normal((N, C * B)).astype(np.float32)
    xq, sx = O.activation_quantize_int8(x)
    P = O.ternary_block_partials(xq, t, col).astype(np.int32)
    y_fix, _ = O.ternary_matmul(xq, sx, t, s, col, exact_scales=False)
    return dict(xq=xq, sx=sx, t=t, s=s, col=col, partials=P, y=bf16(y_fix))


def main():
    arrays = {}
    for n, (B, K, N, sen, mult) in enumerate(SWIGLU_TINY):
        for k, v in swiglu_case(1000 + n, B, K, N, sen, mult).items():
            arrays[f"swiglu{n}_{k}"] = v
    np.savez_compressed(os.path.join(HERE, "swiglu_tiny.npz"), **arrays)
    arrays = {}
    for n, (B, K, N) in enumerate(TERNARY_TINY):
        for k, v in ternary_case(2000 + n, B, K, N).items():
            arrays[f"ternary{n}_{k}"] = v
    np.savez_compressed(os.path.join(HERE, "ternary_tiny.npz"), **arrays)
    # the small CPU-runnable geometry (d_model 256, d_ff 1024, B 16, K 4, 512 tokens): seed,
    # checksums and slices of the output
    rng = np.random.default_rng(7)
    g, u, d = (O.random_topology(R, C, 4, rng) for R, C in ((64, 16), (64, 16), (16, 64)))
    vals = [(rng.standard_normal((R, 4, 16, 16)) * 0.02).astype(np.float32) for R in (64, 64, 16)]
    x = rng.standard_normal((512, 256)).astype(np.float32)
    out = O.swiglu_fwd(x.astype(np.float64), (vals[0].astype(np.float64), g), (vals[1].astype(np.float64), u),
                       (vals[2].astype(np.float64), d))[0]
    summary = {"seed": 7, "shape": [512, 256], "sum": float(out.sum()), "abs_sum": float(np.abs(out).sum()),
               "row0_head": [float(v) for v in out[0, :8]], "row511_tail": [float(v) for v in out[511, -8:]]}
    with open(os.path.join(HERE, "small_geometry_summary.json"), "w") as f:
        json.dump(summary, f, indent=1)


if __name__ == "__main__":
    main()
