"""Mutation fuzzing of the artifact parser under AddressSanitizer (CPU only, no GPU).

The C ABI validates a SPYR8F8 artifact entirely on the host before any HIP call
(SrcPyrModel.cpp:243-470 semantics).  tests/fuzz_artifact.cpp feeds it mutants of every shipped
artifact (and of the converted .pt blobs) for every policy; the library's host code (engine.cpp)
is compiled here with AddressSanitizer and UndefinedBehaviorSanitizer on the host side only, and
the harness links the built library for the kernel launchers, which no mutant reaches without a
GPU.  Every mutant must end in AEISU_ERR_ARTIFACT (or, if it passes every check, at the first
HIP call) with no sanitizer report.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from aeisu_amd import _lib as L
from aeisu_amd import artifacts as A
from tests._util import ROOT, WEIGHTS

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ITERATIONS = 1500


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    if not (shutil.which(HIPCC) or os.path.exists(HIPCC)) or not L.LIB_PATH.exists():
        pytest.skip("needs hipcc and the built library")
    out = tmp_path_factory.mktemp("fuzz")
    inc = [f"-I{ROOT / 'include'}", f"-I{ROOT / 'aeisu_amd' / 'csrc'}"]
    engine = out / "engine.o"
    # host code only under the sanitizers: each -fsanitize= follows -Xarch_host
    host_san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-Xarch_host", "-fno-omit-frame-pointer"]
    subprocess.run([HIPCC, "-O1", "-g", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", *inc, *host_san, "-c", str(ROOT / "aeisu_amd" / "csrc" / "engine.cpp"),
                    "-o", str(engine)], check=True, capture_output=True, text=True)
    exe = out / "fuzz_artifact"
    link_san = ["-fsanitize=address", "-fsanitize=undefined", "-fno-gpu-sanitize"]
    subprocess.run([HIPCC, "-O1", "-g", "-std=c++17", *inc, *link_san, "--offload-arch=gfx950", "-x", "c++",
                    str(ROOT / "tests" / "fuzz_artifact.cpp"), "-x", "none", str(engine),
                    f"-L{L.LIB_PATH.parent}", "-laeisu_amd", f"-Wl,-rpath,{L.LIB_PATH.parent}", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    blobs = {}
    for name in ("aeisu_area.pt", "aeisu_int8_fp16.pt"):
        blob, _ = A.load_blob(WEIGHTS / name)
        path = out / (name + ".spyr")
        path.write_bytes(blob)
        blobs[name] = path
    return exe, blobs


@pytest.mark.parametrize("artifact,precision", [
    ("aeisu_area_mixed_fp8.bin", "mixed"), ("aeisu_area_mixed_fp8.bin", "fp16"),
    ("aeisu_area_mixed_fp8.bin", "mixed-fp8mma"), ("aeisu_div2k_l1_mixed_fp8.bin", "mixed"),
    ("aeisu_area.pt", "fp16"), ("aeisu_area.pt", "fp32"), ("aeisu_int8_fp16.pt", "int8"),
])
def test_artifact_mutants_are_rejected_cleanly(fuzzer, artifact, precision):
    exe, blobs = fuzzer
    path = blobs.get(artifact, WEIGHTS / artifact)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    seed = sum(map(ord, artifact + precision))
    res = subprocess.run([str(exe), str(path), str(L.PRECISION[precision]), str(ITERATIONS), str(seed)],
                         capture_output=True, text=True, errors="replace", env=env, timeout=600)
    report = res.stdout + res.stderr
    assert res.returncode == 0, report[-3000:]
    assert "AddressSanitizer" not in report and "runtime error" not in report, report[-3000:]
    codes = {int(line.split()[1].rstrip(":")): int(line.split()[2])
             for line in res.stdout.splitlines() if line.startswith("rc ")}
    assert sum(codes.values()) == ITERATIONS
    assert set(codes) <= {L.AEISU_ERR_ARTIFACT, L.AEISU_ERR_HIP}, codes
    assert codes.get(L.AEISU_ERR_ARTIFACT, 0) > ITERATIONS // 2
