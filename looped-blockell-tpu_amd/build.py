"""Build the native parts of looped_blockell in-tree.

  liblbk.so       hand-written HIP kernels for gfx950 + the C ABI (include/lbk.h)
  _titan_ext.so   thin PyTorch-ROCm extension registering the titan:: operators
                  over the C ABI (loaded with torch.ops.load_library)

Both land in looped_blockell/ next to the Python sources.  Usage:
    python looped-blockell-tpu_amd/build.py [--lib-only]
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
PKG = os.path.join(HERE, "looped_blockell")
LIB = os.path.join(PKG, "liblbk.so")
EXT = os.path.join(PKG, "_titan_ext.so")

HIP_SOURCES = ["lbk_bf16.hip", "lbk_split.hip", "lbk_decode.hip", "lbk_ternary.hip", "lbk_tsplit.hip", "lbk_bwd.hip", "lbk_topo.hip", "lbk_format.hip",
               "lbk_abi.hip", "lbk_noalloc.hip"]
ARCH = os.environ.get("LBK_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU forms are kept out of the generated code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-file extras.  VGPR-form MFMA keeps small loop-carried accumulators out of
# AGPR shuffles (the row-block kernels); the split SwiGLU kernels are left to the
# default allocator.
FILE_FLAGS = {
    "lbk_bf16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "lbk_ternary.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build_lib() -> str:
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, src.replace(".hip", ".o")) for src in HIP_SOURCES]
    cmds = [[hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c",
             os.path.join(CSRC, src), "-o", obj] for src, obj in zip(HIP_SOURCES, objs)]
    jobs = max(1, min(len(cmds), int(os.environ.get("LBK_BUILD_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        for fut in [pool.submit(_run, c) for c in cmds]:
            fut.result()
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def build_ext() -> str:
    import torch
    from torch.utils import cpp_extension as ce

    incs = ce.include_paths(device_type="cuda")
    libdirs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    py_inc = sysconfig.get_paths()["include"]
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-I{INCLUDE}", f"-I{py_inc}"]
    cmd += [f"-I{p}" for p in incs]
    cmd += [os.path.join(CSRC, "torch_ops.cpp")]
    cmd += [f"-L{p}" for p in libdirs]
    cmd += ["-L/opt/rocm/lib", f"-L{PKG}", "-llbk", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
            "-ltorch_hip", "-lamdhip64", "-Wl,-rpath,$ORIGIN"]
    cmd += [f"-Wl,-rpath,{p}" for p in libdirs]
    tmp = EXT + ".tmp"
    cmd += ["-o", tmp]
    _run(cmd)
    os.replace(tmp, EXT)
    return EXT


def build(lib_only: bool = False) -> None:
    build_lib()
    if not lib_only:
        build_ext()


if __name__ == "__main__":
    build(lib_only="--lib-only" in sys.argv)
