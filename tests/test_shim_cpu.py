"""CPU checks of the Python shim's argument handling (no GPU needed).

The shim mirrors aeisu/runtime.py: ``load_model(path, device)`` and ``upscale(model, source, tile)``
raise ValueError for a source that is not a CHW RGB image and for a tile that is not zero or a
positive multiple of 32 (aeisu/runtime.py:77-80), before any device work.  Beyond the reference:
a device that is not a HIP device, a precision the weight file does not carry, and an unknown
precision name are ValueErrors too, and the shim has no CPU fallback (aeisu_amd/_lib.py).
"""
from __future__ import annotations

import pytest
import torch

from aeisu_amd import runtime
from tests._util import WEIGHTS


@pytest.mark.parametrize("shape", [(8, 8), (1, 3, 8, 8), (4, 8, 8), (1, 8, 8)])
def test_upscale_rejects_non_chw_rgb(shape):
    with pytest.raises(ValueError, match="CHW"):
        runtime.upscale(None, torch.zeros(shape), tile=0)


@pytest.mark.parametrize("tile", [-32, 1, 16, 33, 100])
def test_upscale_rejects_bad_tiles(tile):
    with pytest.raises(ValueError, match="multiple of 32"):
        runtime.upscale(None, torch.zeros(3, 8, 8), tile=tile)


@pytest.mark.parametrize("path,precision", [
    ("aeisu_int8_fp16.pt", "mixed"), ("aeisu_int8_fp16.pt", "fp16"), ("aeisu_area_mixed_fp8.bin", "int8"),
    ("aeisu_area_mixed_fp8.bin", "fp32"), ("aeisu_area.pt", "mixed"), ("aeisu_area.pt", "int8"),
])
def test_load_model_rejects_precisions_the_file_lacks(path, precision):
    with pytest.raises(ValueError, match="provides"):
        runtime.load_model(WEIGHTS / path, precision=precision)


def test_upscaler_needs_a_hip_device_and_a_known_precision():
    blob = (WEIGHTS / "aeisu_area_mixed_fp8.bin").read_bytes()
    with pytest.raises(ValueError, match="precision"):
        runtime.Upscaler(blob, "bf16")
    with pytest.raises(ValueError, match="HIP device"):
        runtime.Upscaler(blob, "mixed", device="cpu")
