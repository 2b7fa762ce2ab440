"""Shared helpers for the parity tests (test-side only)."""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch
from torch.nn import functional as F

ROOT = Path(__file__).resolve().parents[1]
WEIGHTS = ROOT / "weights"
GOLDEN = ROOT / "tests" / "golden"


def pad_frame(src: torch.Tensor) -> torch.Tensor:
    """[B,3,H,W] -> replicate-padded frame on the align32/halo16 grid (aeisu/runtime.py:82-84)."""
    h, w = src.shape[-2:]
    ey, ex = -h % 32, -w % 32
    py, px = 16 + ey // 2, 16 + ex // 2
    return F.pad(src.float(), (px, 32 + ex - px, py, 32 + ey - py), mode="replicate")


def crop_output(out: torch.Tensor, h: int, w: int) -> torch.Tensor:
    """Crop the 2x output of a padded frame back to the source's 2H x 2W window."""
    ey, ex = -h % 32, -w % 32
    py, px = 16 + ey // 2, 16 + ex // 2
    return out[..., 2 * py:2 * (py + h), 2 * px:2 * (px + w)]


def nhwc_to_nchw(t: torch.Tensor) -> torch.Tensor:
    return t.permute(0, 3, 1, 2).contiguous()


def psnr(a: torch.Tensor, b: torch.Tensor) -> float:
    mse = float(((a.double() - b.double()) ** 2).mean())
    return math.inf if mse == 0 else 10 * math.log10(1.0 / mse)


def y_psnr(pred: torch.Tensor, target: torch.Tensor, crop: int = 2) -> float:
    """Encoded-Y PSNR with a border crop (BT.601 luma as aeisu/metrics.py:11-39)."""
    def luma(x):
        x = x.double().clamp(0, 1)
        return 16 / 255 + (65.481 * x[..., 0, :, :] + 128.553 * x[..., 1, :, :] + 24.966 * x[..., 2, :, :]) / 255
    a, b = luma(pred), luma(target)
    if crop:
        a, b = a[..., crop:-crop, crop:-crop], b[..., crop:-crop, crop:-crop]
    mse = float(((a - b) ** 2).mean())
    return math.inf if mse == 0 else 10 * math.log10(1.0 / mse)


def golden(tag: str):
    return np.load(GOLDEN / f"reference_{tag}.npz")
