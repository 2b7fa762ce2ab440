"""Compile the gfx950 HIP kernels and the C ABI into ``aeisu_amd/libaeisu_amd.so``.

Every HIP translation unit is built with ``-Xclang -target-feature -Xclang
-packed-fp32-ops`` so the compiler never emits packed FP32 VALU instructions.
The library is built in-tree (it travels with the repository to the GPU box).
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libaeisu_amd.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form=1", f"-I{ROOT / 'include'}", f"-I{CSRC}", "-Wall", "-Wno-unused-function"]


# Per-source compiler options.  The fused head is latency-bound (four waves per SIMD); LLVM's
# iterative ILP scheduler orders its instructions for latency within the same 128-VGPR budget
# (no spills) and took 0.5 us off it at 1080p (A/B on one box).  The frame-input body (Mixed,
# FP8-MFMA, INT8) gains from it too (1080p Mixed 61.9 -> 60.1 us, INT8 540p x 8 111.2 -> 109.4 us,
# no spills), the FP16 policy's skip-input body (k_body_fused_fp16.hip) does not (71.4 -> 73.6 us)
# and keeps the default scheduler, as the other kernels do (max-ilp / max-memory-clause measured no
# better there).
FILE_FLAGS = {"k_fused.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
              "k_body_fused.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]}


def sources():
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return obj


ABI_SMOKE_SRC = ROOT / "tests" / "abi_smoke.cpp"
ABI_SMOKE = ROOT / "tests" / "abi_smoke"


def build_abi_smoke() -> Path:
    """The C++ program that exercises the public header against the built library (a GPU test runs it)."""
    cmd = [HIPCC, "-O2", "-std=c++17", f"--offload-arch={ARCH}", f"-I{ROOT / 'include'}", str(ABI_SMOKE_SRC),
           "-o", str(ABI_SMOKE), f"-L{PKG}", "-laeisu_amd", f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN/../aeisu_amd"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"abi_smoke build failed:\n{res.stderr}")
    return ABI_SMOKE


PROBES = {name: (ROOT / "tests" / f"{name}.hip", ROOT / "tests" / name)
          for name in ("mfma_fp8_probe", "mfma_f16_probe")}


def build_probes() -> list:
    """The GPU test programs that measure the MFMA instructions' accumulation against exact sums."""
    out = []
    for src, exe in PROBES.values():
        cmd = [HIPCC, "-O2", "-std=c++17", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
               "-packed-fp32-ops", str(src), "-o", str(exe)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"{exe.name} build failed:\n{res.stderr}")
        out.append(exe)
    return out


def build(jobs: int = 8) -> Path:
    """Compile every source (always), link the shared library and the C++ test programs."""
    BUILD.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_abi_smoke()
    build_probes()
    return LIB


if __name__ == "__main__":
    print(build())
