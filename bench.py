#!/usr/bin/env python3
"""Benchmark of the Block-ELL SwiGLU FFN forward on one MI355X.

Headline (one JSON line on stdout): the bf16 Block-ELL SwiGLU FFN at
d_model=1024, d_ff=4096, B=32, 25% density, 16384 tokens — effective TFLOP/s
over nonzero blocks (plus tokens/s), inputs resident in HBM, one step = one
forward pass.  The line also carries:
  roofline      the dominant kernel's achieved vs peak, timed with HIP events
                on the stream the kernel runs on;
  cpu_baseline  a PyTorch CPU float32 restatement of the reference layer (its
                gather + einsum, chunked over tokens), median of 3 runs on the
                host cores, on the same workload (bounded token samples for the
                ternary and looped lines, each named in its "sample");
  extra         the other workloads (shared gate/up topology, the backward of the
                headline workload, the plain Block-ELL product and its backward, ternary FFN, looped block
                L=8, decode, and the prune-time topology transforms on the headline weights).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only-main | --skip-main]
                      [--only shared,backward,...] [--copy-calibration]
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "looped-blockell-tpu_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "effective TFLOP/s (nonzero blocks) + tokens/s, Block-ELL SwiGLU FFN"
TRAFFIC_PROFILE_BF16 = os.path.join(ROOT, "profiles", "swiglu_bf16_gu_dn_N16384_d1024_ff4096_B32.txt")


def profiled_traffic(path):
    """HBM bytes per step recorded by the committed rocprofv3 counter summary, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_step"):
                    return float(line.split("=", 1)[1])
    except OSError:
        pass
    return None
WARMUP_S = 0.3
FEWER_TOKENS = [64, 1024, 4096]   # token counts of the headline and looped workloads' fewer-token runs
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_INT8_TOPS = 5000.0       # MI355X dense int8 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E

WORKLOADS = {
    "bf16": dict(d_model=1024, d_ff=4096, B=32, density=0.25, N=16384, seed=1002),
    "ternary": dict(d_model=2048, d_ff=8192, B=64, density=0.125, N=8192, seed=1003),
    "looped": dict(d_model=1024, d_ff=4096, B=32, density=0.25, N=32 * 512, L=8, seed=1004),
    "decode": dict(d_model=4096, d_ff=14336, B=64, density=0.10, N=16, seed=1005, copies=12),
}


def geometry(w):
    B = w["B"]
    Cm, Cf = w["d_model"] // B, w["d_ff"] // B
    Kg = max(1, int(Cm * w["density"]))
    Kd = max(1, int(Cf * w["density"]))
    Rf, Rm = w["d_ff"] // B, w["d_model"] // B
    return Rf, Rm, Cm, Cf, Kg, Kd


def nonzero_flops(w):
    Rf, Rm, _, _, Kg, Kd = geometry(w)
    B = w["B"]
    return 2.0 * w["N"] * B * B * (Rf * 2 * Kg + Rm * Kd) * w.get("L", 1)


def algorithmic_bytes(w, ternary=False):
    """Weights + indices (+ scales) + input read once + output written once; h excluded."""
    Rf, Rm, _, _, Kg, Kd = geometry(w)
    B = w["B"]
    blocks = Rf * 2 * Kg + Rm * Kd
    if ternary:
        return blocks * (B * B // 4 + 4 + 4) + w["N"] * w["d_model"] * (1 + 2) + w["N"] * 4
    return blocks * (B * B * 2 + 4) + w["N"] * w["d_model"] * 2 * 2


# ---------------------------------------------------------------------------------------------

def make_bell(R, C, K, B, gen, device, std=0.02):
    import torch
    vals = (torch.randn(R, K, B, B, generator=gen, device=device) * std).to(torch.bfloat16)
    cols = torch.argsort(torch.rand(R, C, generator=gen, device=device), dim=1)[:, :K].to(torch.int32).contiguous()
    return vals, cols


def make_ffn(w, device, gen):
    Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
    B = w["B"]
    g = make_bell(Rf, Cm, Kg, B, gen, device)
    u = make_bell(Rf, Cm, Kg, B, gen, device)
    d = make_bell(Rm, Cf, Kd, B, gen, device)
    return g, u, d


def make_ternary(R, C, K, B, gen, device):
    import torch
    from looped_blockell import kernels
    t = torch.randint(-1, 2, (R, K, B, B), generator=gen, device=device, dtype=torch.int8)
    lat = torch.randn(R, K, B * B, generator=gen, device=device) * 0.02
    s = lat.abs().mean(dim=2).clamp_min(1e-8).float().contiguous()
    cols = torch.argsort(torch.rand(R, C, generator=gen, device=device), dim=1)[:, :K].to(torch.int32).contiguous()
    return kernels.pack_ternary(t), s, cols


def time_steps(step, steps, warmup, step_events=False):
    """Run `warmup` untimed steps (more if they take under WARMUP_S), then exactly `steps` timed ones.

    Returns (ms_per_step from the host clock between two synchronisations,
    list of per-step durations from HIP events on the current stream).  The
    timed steps run back to back with no event between them (a recorded event
    separates two launches on the GPU, which costs a short kernel several
    microseconds), and the per-step durations come from a second, untimed pass
    of the same steps with an event pair around each; with step_events=True
    the timed pass itself carries the events.
    """
    import torch
    # untimed warm-up: `warmup` steps, continued until the GPU has been busy for WARMUP_S (its
    # clocks ramp up under load: the first ~100 ms of a fresh process run up to 10 % slower)
    t_w = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t_w < WARMUP_S:
        step(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def with_events():
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            ev[i][0].record(stream)
            step(i)
            ev[i][1].record(stream)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3, [a.elapsed_time(b) for a, b in ev]

    if step_events:
        wall_ms, per = with_events()
        return wall_ms / steps, per
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    _, per = with_events()
    return wall_ms / steps, per


def median(xs):
    s = sorted(xs)
    n = len(s)
    return s[n // 2] if n % 2 else 0.5 * (s[n // 2 - 1] + s[n // 2])


# ---------------------------------------------------------------------------------------------

def bench_bf16(steps, warmup, device):
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["bf16"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    g, u, d = make_ffn(w, device, gen)
    x = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    args = (*g, *u, *d)
    out = {}
    # The weights are fixed across forwards (inference, as MLPBlock runs it without gradients):
    # their packed copy is built once, outside the timed steps, and each step is the gate/up and
    # down launches.
    packed = kernels.swiglu_prepack(*args)

    def step(i):
        out["y"] = kernels.swiglu_fwd_prepacked(x, packed, *args, add_residual=False)

    ms, per = time_steps(step, steps, warmup)
    flops = nonzero_flops(w)
    kern_ms = sum(per) / len(per)
    achieved = flops / (kern_ms * 1e-3) / 1e12

    def step_pack(i):
        out["y2"] = kernels.swiglu_fwd(x, *args, add_residual=False)

    ms_p, per_p = time_steps(step_pack, steps, warmup)

    # the same forward on fewer tokens (the first N rows of x): fewer token blocks than CUs, so
    # the gate/up rows are split over workgroups and the down kernel takes smaller workgroups
    by_tokens = {}
    for n in FEWER_TOKENS:
        xs = x[:n].contiguous()
        ms_n, _ = time_steps(lambda i: kernels.swiglu_fwd_prepacked(xs, packed, *args, add_residual=False),
                             steps, warmup)
        by_tokens[str(n)] = dict(ms_per_step=ms_n, value=nonzero_flops(dict(w, N=n)) / (ms_n * 1e-3) / 1e12)
    res = dict(
        ms_per_step=ms, value=flops / (ms * 1e-3) / 1e12, tokens_per_s=w["N"] / (ms * 1e-3),
        kernel_ms_avg=kern_ms, kernel_ms_median=median(per),
        roofline=dict(bound="mfma", achieved=achieved, peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                      frac=achieved / PEAK_BF16_TFLOPS, traffic=profiled_traffic(TRAFFIC_PROFILE_BF16),
                      traffic_source=os.path.relpath(TRAFFIC_PROFILE_BF16, ROOT) + " (2 x FETCH_SIZE + WRITE_SIZE "
                                     "of the two launches, the factors a copy of known size reads)",
                      kernel="SwiGLU forward launch pair gu_kernel_w12<32,4,false> + "
                             "dnf_kernel<32,4,false>, timed together with HIP events around each step",
                      algorithmic_flops_per_launch=flops,
                      algorithmic_bytes_per_launch=algorithmic_bytes(w)),
        fewer_tokens=dict(workload="the same forward (weights packed once) on the first N tokens", unit="TFLOP/s",
                          by_tokens=by_tokens),
        with_pack=dict(workload="the same forward packing the weights on every call (titan::block_ell_swiglu_fwd: "
                                "pack_bf16_multi_kernel + gu_kernel_w12 + dnf_kernel)",
                       ms_per_step=ms_p, value=flops / (ms_p * 1e-3) / 1e12, unit="TFLOP/s",
                       kernel_ms_avg=sum(per_p) / len(per_p)),
    )
    assert torch.isfinite(out["y"].float()).all() and torch.equal(out["y"], out["y2"])
    return res


def bench_bf16_shared(steps, warmup, device):
    """The headline workload with gate and up sharing one topology (the reference layer's
    initialisation: both are seeded from the same hash, ``looped_blockell/layers/mlp.py:94``)."""
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["bf16"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    g, u, d = make_ffn(w, device, gen)
    x = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    args = (g[0], g[1], u[0], g[1], *d)   # up reads gate's column indices
    packed = kernels.swiglu_prepack(*args)

    def step(i):
        kernels.swiglu_fwd_prepacked(x, packed, *args, add_residual=False)

    ms, per = time_steps(step, steps, warmup)
    flops = nonzero_flops(w)
    return dict(workload="bf16 SwiGLU FFN as the headline workload, gate and up sharing one topology "
                         "(weights packed once)",
                ms_per_step=ms, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s",
                tokens_per_s=w["N"] / (ms * 1e-3), frac_of_bf16_peak=flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                kernel_ms_avg=sum(per) / len(per))


def bench_bf16_backward(steps, warmup, device):
    """Backward of the headline workload (titan::block_ell_swiglu_bwd) from the forward's saved
    tensors: dh, dx and the three tile gradients, twice the forward's nonzero-block FLOPs."""
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["bf16"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    g, u, d = make_ffn(w, device, gen)
    x = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    dy = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    _, h, gp, uo = kernels.swiglu_fwd_with_intermediate(x, *g, *u, *d, add_residual=True)
    out = {}

    def step(i):
        out["r"] = kernels.swiglu_bwd(dy, x, gp, uo, h, *g, *u, *d)

    ms, per = time_steps(step, steps, warmup)
    flops = 2 * nonzero_flops(w)
    assert all(torch.isfinite(t.float()).all() for t in out["r"])
    # the same backward on the first N tokens
    by_tokens = {}
    for n in FEWER_TOKENS:
        sl = [t[:n].contiguous() for t in (dy, x, gp, uo, h)]
        ms_n, _ = time_steps(lambda i: kernels.swiglu_bwd(*sl, *g, *u, *d), steps, warmup)
        by_tokens[str(n)] = dict(ms_per_step=ms_n, value=2 * nonzero_flops(dict(w, N=n)) / (ms_n * 1e-3) / 1e12)
    # the same geometry at B = 16 (the reference's default tile)
    w16 = dict(w, B=16)
    g16, u16, d16 = make_ffn(w16, device, gen)
    _, h16, gp16, uo16 = kernels.swiglu_fwd_with_intermediate(x, *g16, *u16, *d16, add_residual=True)
    ms16, per16 = time_steps(lambda i: kernels.swiglu_bwd(dy, x, gp16, uo16, h16, *g16, *u16, *d16), steps, warmup)
    f16 = 2 * nonzero_flops(w16)
    return dict(workload="backward of the headline workload (dx and the gate/up/down tile gradients)",
                ms_per_step=ms, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s",
                frac_of_bf16_peak=flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, kernel_ms_avg=sum(per) / len(per),
                fewer_tokens=dict(workload="the same backward on the first N tokens", unit="TFLOP/s",
                                  by_tokens=by_tokens),
                b16=dict(workload="the same geometry at B = 16", ms_per_step=ms16,
                         value=f16 / (ms16 * 1e-3) / 1e12, unit="TFLOP/s",
                         frac_of_bf16_peak=f16 / (ms16 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         kernel_ms_avg=sum(per16) / len(per16)))


def bench_topology(steps, warmup, device):
    """Prune-time topology transforms on the headline weights (60% of slots alive): the full
    column reorder (importance, permutation, down column remap, gate rows and their Adam moments
    gathered), the same row gather for up, then compaction of all three weights.  Copy-bound;
    two host reads per compaction (K_new) and one for the index are part of the step."""
    import torch
    from looped_blockell import opt
    w = WORKLOADS["bf16"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    g, u, d = make_ffn(w, device, gen)
    alive = [torch.rand(t[1].shape, generator=gen, device=device) < 0.6 for t in (g, u, d)]
    C_ff = w["d_ff"] // w["B"]
    moments = {"exp_avg": torch.zeros(g[0].shape, dtype=torch.float32, device=device),
               "exp_avg_sq": torch.zeros(g[0].shape, dtype=torch.float32, device=device)}
    out = {}

    def step(i):
        r = opt.full_reorder_step(d[0], d[1], alive[2], g[0], g[1], alive[0], moments, C_ff, 4)
        uv, uc, ua = opt.apply_permutation_to_block_ell(u[0], u[1], alive[1], opt.compute_permutation(
            opt.compute_column_importance(alive[2], alive[0], d[1], g[1], C_ff)), is_column_dim=False)
        out["k"] = [opt.compact_single_layer(r[3], r[4], r[5])[3], opt.compact_single_layer(uv, uc, ua)[3],
                    opt.compact_single_layer(r[0], r[1], r[2])[3]]

    ms, per = time_steps(step, steps, warmup)
    vb = lambda t: t[0].numel() * 2
    kn = out["k"]
    byts = (2 * vb(g) + 2 * 2 * g[0].numel() * 4 + 2 * vb(u)                  # row gathers (values, moments)
            + sum(2 * vb(t) * k // t[0].shape[1] for t, k in zip((g, u, d), kn)))   # compaction copies
    return dict(workload="topology transforms on the headline weights: full column reorder (with Adam "
                         "moments), up-row gather, compaction of gate/up/down",
                ms_per_step=ms, value=byts / (ms * 1e-3) / 1e9, unit="GB/s",
                frac_of_hbm_peak=byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, algorithmic_bytes=byts,
                k_new=kn, kernel_ms_avg=sum(per) / len(per))


def bench_formats(steps, warmup, device):
    """The dense <-> Block-ELL bridge at the headline shapes: dense bf16 gate/up [4096, 1024] and
    down [1024, 4096] -> top-25 % blocks per row by Frobenius norm + tile gather (the layer API's
    create_block_ell_from_dense), then back to dense.  Copy-bound."""
    import torch
    from looped_blockell.layers import block_ell_to_dense, create_block_ell_from_dense
    w = WORKLOADS["bf16"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    dm, dff, B = w["d_model"], w["d_ff"], w["B"]
    dense = [torch.randn(s, generator=gen, device=device).to(torch.bfloat16) for s in ((dff, dm), (dff, dm), (dm, dff))]
    out = {}

    def step(i):
        es = [create_block_ell_from_dense(d, tile_size=B, density=w["density"]) for d in dense]
        out["d"] = [block_ell_to_dense(e) for e in es]

    ms, per = time_steps(step, steps, warmup)
    full = sum(d.numel() * 2 for d in dense)
    # norms read every dense block; the gather reads and writes the kept quarter; to-dense
    # reads the tiles and writes every dense block
    byts = full + 2 * w["density"] * full + w["density"] * full + full
    assert all(torch.isfinite(d.float()).all() for d in out["d"])
    return dict(workload="dense <-> Block-ELL bridge: top-25% block selection + gather, and back to dense, for "
                         "gate/up [4096,1024] and down [1024,4096] bf16",
                ms_per_step=ms, value=byts / (ms * 1e-3) / 1e9, unit="GB/s",
                frac_of_hbm_peak=byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, algorithmic_bytes=byts,
                kernel_ms_avg=sum(per) / len(per))


def bench_matmul(steps, warmup, device):
    """The layer API's plain Block-ELL product (block_ell_matmul / BlockELLLinear, with a bias) at
    the headline workload's gate shape [16384, 1024] -> [16384, 4096] and down shape
    [16384, 4096] -> [16384, 1024], B=32, density 0.25."""
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["bf16"]
    gen = torch.Generator(device=device).manual_seed(w["seed"] + 7)
    Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
    B, N = w["B"], w["N"]
    res = {}
    for name, (R, C, K, fin) in dict(gate_shape=(Rf, Cm, Kg, w["d_model"]), down_shape=(Rm, Cf, Kd, w["d_ff"])).items():
        v, c = make_bell(R, C, K, B, gen, device)
        x = torch.randn(N, fin, generator=gen, device=device).to(torch.bfloat16)
        bias = torch.randn(R * B, generator=gen, device=device) * 0.01
        ms, per = time_steps(lambda i: kernels.block_ell_matmul(x, v, c, bias), steps, warmup)
        flops = 2.0 * N * B * B * R * K
        res[name] = dict(ms_per_step=ms, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s",
                         frac_of_bf16_peak=flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         kernel_ms_avg=sum(per) / len(per))
    g = res["gate_shape"]
    return dict(workload="block_ell_matmul forward with bias (weights packed per call), gate shape 1024 -> 4096 "
                         "and down shape 4096 -> 1024, 16384 tokens, B=32, density 0.25",
                ms_per_step=g["ms_per_step"], value=g["value"], unit="TFLOP/s",
                frac_of_bf16_peak=g["frac_of_bf16_peak"], kernel_ms_avg=g["kernel_ms_avg"],
                down_shape=res["down_shape"])


def bench_default_layer(steps, warmup, device):
    """The reference's default tile-16 SwiGLU layer (biases zero-initialised as in its MLPBlock; gate
    and up with one shared topology, as its init seeds both from one hash) at its two model
    geometries, 16384 tokens each, weights packed once as MLPBlock keeps them: configs/ablation.yaml
    (d_model 512, d_ff 2048, initial density 1.0: K_gate 32, K_down 128) and configs/large.yaml
    pruned to 25 % (d_model 2048, d_ff 8192: K_gate 32, K_down 128)."""
    import torch
    from looped_blockell import kernels
    res = {}
    for name, (dm, dff, dens) in dict(ablation=(512, 2048, 1.0), large_25pct=(2048, 8192, 0.25)).items():
        w = dict(d_model=dm, d_ff=dff, B=16, density=dens, N=16384)
        gen = torch.Generator(device=device).manual_seed(2000 + dm)
        (vg, cg), (vu, _), (vd, cd) = make_ffn(w, device, gen)
        bg = torch.zeros(dff, device=device)
        bu = torch.zeros(dff, device=device)
        bd = torch.zeros(dm, device=device)
        x = torch.randn(w["N"], dm, generator=gen, device=device).to(torch.bfloat16)
        packed = kernels.swiglu_prepack(vg, cg, vu, cg, vd, cd)
        ms, per = time_steps(lambda i: kernels.swiglu_fwd_prepacked(x, packed, vg, cg, vu, cg, vd, cd, False,
                                                                    bg, bu, bd), steps, warmup)
        flops = nonzero_flops(w)
        res[name] = dict(workload=f"d_model={dm} d_ff={dff} B=16 density={dens} N=16384, biases, shared gate/up "
                                  f"topology, prepacked", ms_per_step=ms, value=flops / (ms * 1e-3) / 1e12,
                         unit="TFLOP/s", frac_of_bf16_peak=flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         tokens_per_s=w["N"] / (ms * 1e-3), kernel_ms_avg=sum(per) / len(per))
    a = res["ablation"]
    return dict(workload="the reference's default tile-16 SwiGLU layer at its ablation geometry (value) and its "
                         "large geometry at 25 % density (large_25pct)",
                ms_per_step=a["ms_per_step"], value=a["value"], unit="TFLOP/s",
                frac_of_bf16_peak=a["frac_of_bf16_peak"], **res)


def bench_matmul_backward(steps, warmup, device):
    """Backward of one Block-ELL product at the headline gate shape (x [16384, 1024] -> [16384, 4096],
    B=32, 25 %): dx = dy W and the tile gradients (titan::block_ell_matmul_bwd), 2x the product's
    nonzero-block FLOPs."""
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["bf16"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
    vals, cols = make_bell(Rf, Cm, Kg, w["B"], gen, device)
    x = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    dy = torch.randn(w["N"], w["d_ff"], generator=gen, device=device).to(torch.bfloat16)
    out = {}

    def step(i):
        out["r"] = kernels.block_ell_matmul_bwd(dy, x, vals, cols)

    ms, per = time_steps(step, steps, warmup)
    flops = 2 * 2 * w["N"] * w["B"] ** 2 * Rf * Kg
    assert all(torch.isfinite(t.float()).all() for t in out["r"])
    return dict(workload="backward of one Block-ELL product, x [16384,1024] -> [16384,4096], B=32, density 0.25",
                ms_per_step=ms, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s",
                frac_of_bf16_peak=flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, kernel_ms_avg=sum(per) / len(per))


def bench_ternary(steps, warmup, device):
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["ternary"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
    B = w["B"]
    g = make_ternary(Rf, Cm, Kg, B, gen, device)
    u = make_ternary(Rf, Cm, Kg, B, gen, device)
    d = make_ternary(Rm, Cf, Kd, B, gen, device)
    x = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    # weights prepared once, as TernaryMLPBlock keeps them
    prep = kernels.ternary_prepare(g, u, d)

    def step(i):
        # TernaryMLPBlock.forward: per-token int8 quantisation of x, then the ternary FFN
        xq, sx = kernels.quantize_act_int8(x)
        kernels.ternary_swiglu_fwd_prepared(xq, sx, prep, g, u, d)

    ms, per = time_steps(step, steps, warmup)
    ops = nonzero_flops(w)
    tops = ops / (ms * 1e-3) / 1e12
    xq, sx = kernels.quantize_act_int8(x)

    def step_q(i):
        kernels.ternary_swiglu_fwd_prepared(xq, sx, prep, g, u, d)

    ms_q, per_q = time_steps(step_q, steps, warmup)

    def step_p(i):
        xq2, sx2 = kernels.quantize_act_int8(x)
        kernels.ternary_swiglu_fwd(xq2, sx2, g, u, d)

    ms_p, per_p = time_steps(step_p, steps, warmup)
    return dict(workload="ternary 2-bit weights / int8 activations SwiGLU FFN, d_model=2048 d_ff=8192 B=64 "
                         "density=0.125 N=8192 (forward from bf16 x: activation quantisation + FFN on weights "
                         "prepared once)",
                ms_per_step=ms, value=tops, unit="TOP/s", tokens_per_s=w["N"] / (ms * 1e-3),
                frac_of_int8_peak=tops / PEAK_INT8_TOPS, algorithmic_ops=ops,
                algorithmic_bytes=algorithmic_bytes(w, ternary=True), kernel_ms_avg=sum(per) / len(per),
                from_quantized=dict(workload="the same FFN from already-quantised xq, sx",
                                    ms_per_step=ms_q, value=ops / (ms_q * 1e-3) / 1e12, unit="TOP/s",
                                    kernel_ms_avg=sum(per_q) / len(per_q)),
                per_call_prepare=dict(workload="from bf16 x, preparing the weights on every call "
                                               "(titan::block_ell_swiglu_fwd_ternary)",
                                      ms_per_step=ms_p, value=ops / (ms_p * 1e-3) / 1e12, unit="TOP/s",
                                      kernel_ms_avg=sum(per_p) / len(per_p)))


def bench_looped(steps, warmup, device):
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["looped"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    g, u, d = make_ffn(w, device, gen)
    h = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    scale = torch.ones(w["d_model"], device=device)

    def step(i):
        kernels.looped_swiglu_persistent(h, scale, *g, *u, *d, L=w["L"], eps=1e-5)

    ms, per = time_steps(step, steps, warmup)
    flops = nonzero_flops(w)
    tf = flops / (ms * 1e-3) / 1e12

    def step_l(i):
        kernels.looped_swiglu_launches(h, scale, *g, *u, *d, L=w["L"], eps=1e-5)

    ms_l, per_l = time_steps(step_l, steps, warmup)
    tf_l = flops / (ms_l * 1e-3) / 1e12

    # fewer tokens: the persistent launch has one workgroup per 64 tokens, the per-iteration
    # kernels split the weight rows over many
    small = {}
    for n in FEWER_TOKENS:
        hs = h[:n].contiguous()
        ms_p, _ = time_steps(lambda i: kernels.looped_swiglu_persistent(hs, scale, *g, *u, *d, L=w["L"], eps=1e-5),
                             steps, warmup)
        ms_s, _ = time_steps(lambda i: kernels.looped_swiglu_launches(hs, scale, *g, *u, *d, L=w["L"], eps=1e-5),
                             steps, warmup)
        small[str(n)] = dict(persistent_ms=ms_p, launches_ms=ms_s)
    persistent = dict(workload="weight packing + one persistent launch: a workgroup owns a 64-token block for all "
                               "L iterations (titan::looped_swiglu_persistent)",
                      ms_per_step=ms, value=tf, unit="TFLOP/s", frac_of_bf16_peak=tf / PEAK_BF16_TFLOPS,
                      kernel_ms_avg=sum(per) / len(per))
    launches = dict(workload="weight packing + an fp32 copy + 2L launches (gate/up and down per iteration; the "
                             "default of titan::looped_swiglu)",
                    ms_per_step=ms_l, value=tf_l, unit="TFLOP/s", frac_of_bf16_peak=tf_l / PEAK_BF16_TFLOPS,
                    kernel_ms_avg=sum(per_l) / len(per_l))
    # the line's value is the faster of the two forms, named in "mode"; both are reported
    best, mode = (persistent, "persistent") if ms <= ms_l else (launches, "launches")
    return dict(workload="looped RMSNorm -> SwiGLU -> residual, L=8 shared weights, d_model=1024 d_ff=4096 B=32 "
                         "density=0.25 N=32x512 (value: the faster of the persistent launch and the per-iteration "
                         "launches, named in mode)",
                mode=mode, ms_per_step=best["ms_per_step"], value=best["value"], unit="TFLOP/s",
                tokens_per_s=w["N"] / (best["ms_per_step"] * 1e-3),
                token_iterations_per_s=w["N"] * w["L"] / (best["ms_per_step"] * 1e-3),
                frac_of_bf16_peak=best["frac_of_bf16_peak"], kernel_ms_avg=best["kernel_ms_avg"],
                persistent=persistent, launches=launches,
                fewer_tokens=dict(workload="the same looped block (L=8) on the first N tokens, ms per call",
                                  by_tokens=small))


def bench_looped_core(steps, warmup, device):
    """The looped core (titan::looped_core): per iteration the diagonal injection, n_core = 2 distinct
    blocks and the per-sequence depth freeze, at the looped-block geometry with L = 4 (eight FFN
    applications per token at full depth, as the L = 8 shared-weight line)."""
    import torch
    from looped_blockell import kernels
    w = dict(WORKLOADS["looped"])
    n_core, L, S = 2, 4, 512
    nseq = w["N"] // S
    gen = torch.Generator(device=device).manual_seed(w["seed"] + 7)
    blocks = [make_ffn(w, device, gen) for _ in range(n_core)]
    h = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    e = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)
    la = torch.zeros(w["d_model"], device=device)
    ld = torch.full((w["d_model"],), 0.3, device=device)
    scales = [torch.ones(w["d_model"], device=device) for _ in range(n_core)]
    full = torch.full((nseq,), L, dtype=torch.int32, device=device)
    mixed = (torch.arange(nseq, device=device) % L + 1).to(torch.int32)
    per_app = nonzero_flops(dict(w, L=1))   # one FFN application over all tokens

    def call(depths, persistent):
        return kernels.looped_core(h, e, la, ld, scales, [b[0][0] for b in blocks], [b[0][1] for b in blocks],
                                   [b[1][0] for b in blocks], [b[1][1] for b in blocks], [b[2][0] for b in blocks],
                                   [b[2][1] for b in blocks], L, depths=depths, seq_len=S, persistent=persistent)

    res = {}
    for name, depths in (("full_depth", full), ("mixed_depths", mixed)):
        # FLOPs of the applications the rows actually run (a frozen row does no work)
        apps = float(torch.clamp(depths, max=L).sum().item()) * S / w["N"] * n_core
        flops = per_app * apps
        sub = {}
        for form, persistent in (("launches", False), ("persistent", True)):
            ms, per = time_steps(lambda i: call(depths, persistent), steps, warmup)
            sub[form] = dict(ms_per_step=ms, value=flops / (ms * 1e-3) / 1e12, unit="TFLOP/s",
                             frac_of_bf16_peak=flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                             kernel_ms_avg=sum(per) / len(per))
        sub["ffn_applications_per_token"] = apps
        sub["flops"] = flops
        res[name] = sub
    best = min(("launches", "persistent"), key=lambda f: res["full_depth"][f]["ms_per_step"])
    b = res["full_depth"][best]
    return dict(workload="looped core: per iteration injection (decay*h + dt*e) -> 2 distinct pre-norm SwiGLU "
                         "blocks -> per-sequence depth freeze; d_model=1024 d_ff=4096 B=32 density=0.25 "
                         "N=32x512 tokens, L=4 (full_depth: every sequence runs 4 iterations = 8 FFN applications "
                         "per token; mixed_depths: sequence depths 1..4, frozen rows skipped); value: the faster "
                         "form at full depth, named in mode",
                mode=best, ms_per_step=b["ms_per_step"], value=b["value"], unit="TFLOP/s",
                frac_of_bf16_peak=b["frac_of_bf16_peak"], **res)


def bench_decode(steps, warmup, device):
    import torch
    from looped_blockell import kernels
    w = WORKLOADS["decode"]
    gen = torch.Generator(device=device).manual_seed(w["seed"])
    copies = [make_ffn(w, device, gen) for _ in range(w["copies"])]   # > 256 MB: defeats the MALL
    x = torch.randn(w["N"], w["d_model"], generator=gen, device=device).to(torch.bfloat16)

    def step(i):
        g, u, d = copies[i % len(copies)]
        kernels.swiglu_fwd(x, *g, *u, *d, add_residual=False)

    eager_ms, per = time_steps(step, steps, warmup)

    # The forward is a ~10 us weight stream, so host submission (python, the op's checks, two
    # launches) is as long as the GPU work: a decode loop runs it from a HIP graph.  One graph
    # holds one forward per weight copy (the rotation), and is replayed.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(len(copies)):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(len(copies)):
            step(i)
    reps = max(2, -(-steps // len(copies)))
    for _ in range(max(2, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        graph.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / (reps * len(copies))
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record(stream)
        graph.replay()
        b.record(stream)
    torch.cuda.synchronize()
    graph_kernel_ms = sum(a.elapsed_time(b) for a, b in ev) / (reps * len(copies))
    byts = algorithmic_bytes(w)
    # the line reports the faster of the two ways a decode loop runs the forward (both measured
    # on the host clock over whole steps; when the host keeps up, eager submission skips the
    # graph's per-node overhead)
    best, mode = (eager_ms, "eager launches") if eager_ms < ms else (ms, "HIP graph replay")
    gbs = byts / (best * 1e-3) / 1e9
    return dict(workload="decode SwiGLU FFN, 16 tokens, d_model=4096 d_ff=14336 B=64 density=0.10, "
                         f"{w['copies']} rotating weight copies",
                mode=mode, ms_per_step=best, value=gbs, unit="GB/s", frac_of_hbm_peak=gbs / PEAK_HBM_GBS,
                tflops=nonzero_flops(w) / (best * 1e-3) / 1e12, algorithmic_bytes=byts,
                graph_ms_per_step=ms, graph_gbs=byts / (ms * 1e-3) / 1e9, graph_steps=reps * len(copies),
                graph_ms_per_step_events=graph_kernel_ms,
                eager_ms_per_step=eager_ms, eager_gbs=byts / (eager_ms * 1e-3) / 1e9,
                eager_kernel_ms_avg=sum(per) / len(per))


def _cpu_info():
    """Threads this process may use for the CPU baseline, and the host CPU model."""
    cores = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        cores = min(cores, int(env))
    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    return cores, model


def _cpu_median(fn, reps):
    """One untimed warm-up, then the median wall time of `reps` runs."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return median(ts), ts


def _cpu_bell(rng, R, C, K, B, std=0.02):
    import torch
    from oracle import oracle as O
    v = torch.from_numpy((rng.standard_normal((R, K, B, B)) * std).astype("float32"))
    return v, torch.from_numpy(O.random_topology(R, C, K, rng))


def cpu_baselines(reps=3):
    """The PyTorch CPU float32 restatement of the reference layer (gather + einsum, chunked over
    1024 tokens) on the host cores: the headline workload in full and bounded token samples of the
    ternary, looped and decode workloads.  Median of `reps` runs after one warm-up each."""
    import numpy as np
    import torch
    from oracle import torch_cpu as TC
    cores, model = _cpu_info()
    torch.set_num_threads(cores)
    common = dict(cores=cores, kind="port", cpu_model=model, reps=reps,
                  implementation="PyTorch CPU float32 restatement of looped_blockell/layers/block_ell.py:149-182 "
                                 "composed as looped_blockell/layers/mlp.py:119-145, 1024-token chunks")
    res = {}
    with torch.inference_mode():
        # headline: all 16384 tokens
        w = WORKLOADS["bf16"]
        Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
        B = w["B"]
        rng = np.random.default_rng(w["seed"])
        g, u, d = _cpu_bell(rng, Rf, Cm, Kg, B), _cpu_bell(rng, Rf, Cm, Kg, B), _cpu_bell(rng, Rm, Cf, Kd, B)
        x = torch.from_numpy(rng.standard_normal((w["N"], w["d_model"])).astype("float32"))
        dt, ts = _cpu_median(lambda: TC.swiglu_fwd(x, g, u, d), reps)
        res["bf16"] = dict(common, value=nonzero_flops(w) / dt / 1e12, unit="TFLOP/s", tokens_per_s=w["N"] / dt,
                           seconds_median=dt, seconds=ts,
                           sample=f"headline workload, all {w['N']} tokens, float32")
        # ternary: a 1024-token sample of the 8192
        w = dict(WORKLOADS["ternary"], N=1024)
        Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
        B = w["B"]
        rng = np.random.default_rng(w["seed"])

        def tern(R, C, K):
            from oracle import oracle as O
            t = torch.from_numpy(rng.integers(-1, 2, size=(R, K, B, B)).astype("float32"))
            s = torch.from_numpy((0.015 + 0.002 * rng.random((R, K))).astype("float32"))
            return t, s, torch.from_numpy(O.random_topology(R, C, K, rng))

        tg, tu, td = tern(Rf, Cm, Kg), tern(Rf, Cm, Kg), tern(Rm, Cf, Kd)
        x = torch.from_numpy(rng.standard_normal((w["N"], w["d_model"])).astype("float32"))
        dt, ts = _cpu_median(lambda: TC.ternary_swiglu_fwd(x, tg, tu, td), reps)
        res["ternary"] = dict(common, value=nonzero_flops(w) / dt / 1e12, unit="TOP/s", tokens_per_s=w["N"] / dt,
                              seconds_median=dt, seconds=ts,
                              sample="ternary workload on 1024 of its 8192 tokens (int8 activations, exact "
                                     "integer partials in float32, per-block fp32 scales)")
        # looped: a 2048-token sample of the 32x512, all L = 8 iterations
        w = dict(WORKLOADS["looped"], N=2048)
        Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
        B = w["B"]
        rng = np.random.default_rng(w["seed"])
        g, u, d = _cpu_bell(rng, Rf, Cm, Kg, B), _cpu_bell(rng, Rf, Cm, Kg, B), _cpu_bell(rng, Rm, Cf, Kd, B)
        h = torch.from_numpy(rng.standard_normal((w["N"], w["d_model"])).astype("float32"))
        scale = torch.ones(w["d_model"])
        dt, ts = _cpu_median(lambda: TC.looped_swiglu(h, scale, g, u, d, L=w["L"]), reps)
        res["looped"] = dict(common, value=nonzero_flops(w) / dt / 1e12, unit="TFLOP/s", tokens_per_s=w["N"] / dt,
                             seconds_median=dt, seconds=ts,
                             sample="looped block (L = 8) on 2048 of its 16384 tokens, float32 state")
        # decode: the full 16-token step
        w = WORKLOADS["decode"]
        Rf, Rm, Cm, Cf, Kg, Kd = geometry(w)
        B = w["B"]
        rng = np.random.default_rng(w["seed"])
        g, u, d = _cpu_bell(rng, Rf, Cm, Kg, B), _cpu_bell(rng, Rf, Cm, Kg, B), _cpu_bell(rng, Rm, Cf, Kd, B)
        x = torch.from_numpy(rng.standard_normal((w["N"], w["d_model"])).astype("float32"))
        dt, ts = _cpu_median(lambda: TC.swiglu_fwd(x, g, u, d), max(reps, 5))
        res["decode"] = dict(common, value=algorithmic_bytes(w) / dt / 1e9, unit="GB/s (bf16-equivalent bytes)",
                             ms_per_step=dt * 1e3, seconds_median=dt, seconds=ts, reps=max(reps, 5),
                             sample="decode workload, the full 16-token step on one weight copy (float32 weights "
                                    "in host memory; GB/s counts the bf16 weight bytes the GPU streams)")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-main", action="store_true", help="headline workload only (for profiling)")
    ap.add_argument("--skip-main", action="store_true",
                    help="skip the headline workload (profiling one extra workload on its own; the line's "
                         "headline fields are then null)")
    ap.add_argument("--only", default="",
                    help="comma list of extra workloads to run: shared,backward,matmul,matmul_backward,ternary,"
                         "looped,looped_core,default_layer,decode,topology,formats")
    ap.add_argument("--no-fewer-tokens", action="store_true",
                    help="skip the fewer-token runs of the headline and looped workloads (profiling: the kernel "
                         "statistics then hold the named workload's launches only)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one 256 MiB device-to-device copy (a reference point for HBM byte counters)")
    args = ap.parse_args()
    FEWER_TOKENS[:] = [] if args.no_fewer_tokens else FEWER_TOKENS
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the Block-ELL FFN path is single-GPU; "
              "no multi-GPU figure is produced). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    from looped_blockell import kernels
    kernels.ops()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)

    if args.copy_calibration:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    empty = dict(value=None, ms_per_step=None, tokens_per_s=None, kernel_ms_avg=None, roofline=None, with_pack=None,
                 fewer_tokens=None)
    main_res = empty if args.skip_main else bench_bf16(args.steps, args.warmup, device)
    extra = {}
    if not args.only_main:
        todo = [s for s in args.only.split(",") if s] or ["shared", "backward", "matmul", "matmul_backward", "ternary",
                                                           "looped", "looped_core", "default_layer", "decode",
                                                           "topology", "formats"]
        fns = dict(shared=bench_bf16_shared, backward=bench_bf16_backward, matmul=bench_matmul,
                   matmul_backward=bench_matmul_backward,
                   ternary=bench_ternary, looped=bench_looped, looped_core=bench_looped_core,
                   default_layer=bench_default_layer, decode=bench_decode,
                   topology=bench_topology,
                   formats=bench_formats)
        for name in todo:
            st = max(5, args.steps // (4 if name in ("looped", "looped_core") else 1))
            try:
                extra[name] = fns[name](st, max(2, args.warmup), device)
            except Exception as e:  # report, keep the headline line
                extra[name] = dict(error=f"{type(e).__name__}: {e}")
    cpu = None
    if not args.no_cpu and not args.only_main:
        cpus = cpu_baselines()
        cpu = cpus.pop("bf16")
        for name, c in cpus.items():
            if name in extra and "error" not in extra[name]:
                extra[name]["cpu_baseline"] = c

    w = WORKLOADS["bf16"]
    line = {
        "metric": METRIC,
        "value": main_res["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random N(0,0.02) weights, random per-row topology, x ~ N(0,1))",
        "config": {"workload": "bf16 Block-ELL SwiGLU FFN forward, d_model=1024 d_ff=4096 B=32 density=0.25 "
                               "N=16384 tokens (weights packed once; with_pack: packed per call)",
                   "d_model": w["d_model"], "d_ff": w["d_ff"], "B": w["B"], "density": w["density"],
                   "tokens": w["N"], "parallelism": "single GPU"},
        "tokens_per_s": main_res["tokens_per_s"],
        "kernel_ms_avg": main_res["kernel_ms_avg"],
        "roofline": main_res["roofline"],
        "with_pack": main_res["with_pack"],
        "fewer_tokens": main_res.get("fewer_tokens"),
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
