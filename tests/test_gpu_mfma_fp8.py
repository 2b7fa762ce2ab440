"""Why the Mixed policy runs its E4M3 layers on the FP16 MFMA: the E4M3 MFMA does not sum exactly.

The emulation of the reference's Mixed deployment (oracle/deploy.py, ``mma_chain``) models each K=32
E4M3 MMA step as the exact sum of its 32 products rounded once to FP32; the policy's E4M3 layers match
it bit for bit on the GPU (tests/test_gpu_layers.py) because E4M3 values are exact in FP16 and the FP16
MFMA keeps FP32 precision.  tests/mfma_fp8_probe (built by aeisu_amd/build.py from
tests/mfma_fp8_probe.hip) runs crafted and random operands through v_mfma_f32_16x16x32_fp8_fp8 and
v_mfma_f32_16x16x32_f16 on the same values.  Measured on gfx950: the E4M3 MFMA sums each group of 8
products (the 8 K slots one lane supplies) aligned to that group's largest product and loses what lies
more than about 13 bits below it, even when that product cancels against another group; groups are
then combined at FP32 precision.  On random operands its error is about 2^-14.5 of the largest product
(median), against about 2^-24.5 for the FP16 MFMA.  No ordering of K makes such sums exact, which is why
AEISU_PRECISION_MIXED_FP8MMA misses the 2/255 bound and is not a deliverable policy.
"""
from __future__ import annotations

import json
import subprocess
import sys

import pytest

from tests._util import ROOT

pytestmark = pytest.mark.gpu


def test_e4m3_mfma_accumulation_is_not_exact(gpu):
    exe = ROOT / "tests" / "mfma_fp8_probe"
    if not exe.exists():
        pytest.fail("tests/mfma_fp8_probe is not built; run `python -m aeisu_amd.build`")
    print("case: tests/mfma_fp8_probe (E4M3 vs FP16 MFMA accumulation)", flush=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    r = json.loads(res.stdout)
    print(json.dumps(r), flush=True)
    sys.stdout.flush()
    kept8 = {b: k for b, k in r["window_fp8"]}
    kept16 = {b: k for b, k in r["window_f16"]}
    # one product 2^6 plus one 2^-(bits-6) in the same group of 8 K slots
    assert all(kept16[b] for b in kept16), "the FP16 MFMA keeps every bit FP32 can hold"
    assert all(kept8[b] for b in kept8 if b <= 12) and not any(kept8[b] for b in kept8 if b >= 15)
    # +2^16 and -2^16 cancel; 1.0 in the +2^16 product's group is lost by the E4M3 MFMA only
    assert r["cancel_same_fp8"] == 0.0 and r["cancel_same_f16"] == 1.0
    # +2^16 - 2^16 in group 0, 2^-e in group 1: the E4M3 MFMA aligns the groups to the cancelled 2^16
    # (about 24 bits: kept to 2^-8, lost below 2^-9); the FP16 MFMA keeps it
    cross8 = {e: k for e, k in r["cancel_cross_fp8"]}
    assert all(cross8[e] for e in cross8 if e <= 7) and not any(cross8[e] for e in cross8 if e >= 10)
    assert all(k for _, k in r["cancel_cross_f16"])
    # random operands: errors relative to the largest product
    assert r["random_fp8"]["median_log2_rel"] > -17.0
    assert r["random_f16"]["median_log2_rel"] < -22.0
    assert r["random_fp8"]["equal_fl32_exact"] < 0.1 < r["random_f16"]["equal_fl32_exact"]
