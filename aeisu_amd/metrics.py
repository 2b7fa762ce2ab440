"""Encoded-Y PSNR and SSIM of an upscaled frame against its target.

Definitions of the reference evaluation (aeisu/metrics.py:11-39): the prediction is
clamped to [0, 1], both images lose a ``crop``-pixel border, luma is BT.601 encoded Y
(16 + 65.481 R + 128.553 G + 24.966 B) / 255, PSNR = -10 log10(MSE) on that luma, and
SSIM uses an 11x11 Gaussian window (sigma 1.5, valid positions only) with constants
C1 = 0.01^2, C2 = 0.03^2, averaged over the window positions.  All arithmetic in float64.
LPIPS (an optional network metric in the reference) is not provided: its pretrained
weights cannot be fetched here.
"""
from __future__ import annotations

import math
from typing import Dict

import torch
from torch.nn import functional as F

_LUMA = (65.481, 128.553, 24.966)


def luma(rgb: torch.Tensor) -> torch.Tensor:
    """CHW RGB in [0, 1] -> 1HW encoded Y in [16/255, 235/255]."""
    w = torch.tensor(_LUMA, dtype=rgb.dtype, device=rgb.device)
    return (torch.einsum("c,chw->hw", w, rgb)[None] + 16.0) / 255.0


def _gaussian_window(size: int = 11, sigma: float = 1.5, device=None) -> torch.Tensor:
    x = torch.arange(size, dtype=torch.float64, device=device) - (size - 1) / 2
    g = torch.exp(-(x * x) / (2 * sigma * sigma))
    g = g / g.sum()
    return torch.outer(g, g)[None, None]


def distortion(prediction: torch.Tensor, target: torch.Tensor, crop: int = 2) -> Dict[str, float]:
    """{'y_mse', 'y_psnr', 'y_ssim'} of a CHW prediction against a same-size CHW target."""
    if prediction.shape != target.shape or prediction.ndim != 3:
        raise ValueError(f"distortion() compares two CHW images of one shape, got {tuple(prediction.shape)} "
                         f"and {tuple(target.shape)}")
    if not (torch.isfinite(prediction).all() and torch.isfinite(target).all()):
        raise ValueError("distortion() got a non-finite value")
    if crop < 0 or min(prediction.shape[-2:]) < 11 + 2 * crop:
        raise ValueError(f"a {prediction.shape[-2]}x{prediction.shape[-1]} image leaves no 11x11 SSIM window after "
                         f"a {crop}-pixel border crop")
    a = prediction.clamp(0, 1).double()
    b = target.double()
    if crop:
        a, b = a[:, crop:-crop, crop:-crop], b[:, crop:-crop, crop:-crop]
    ya, yb = luma(a)[None], luma(b)[None]
    mse = float(((ya - yb) ** 2).mean())
    win = _gaussian_window(device=ya.device)
    mu_a, mu_b = F.conv2d(ya, win), F.conv2d(yb, win)
    var_a = F.conv2d(ya * ya, win) - mu_a * mu_a
    var_b = F.conv2d(yb * yb, win) - mu_b * mu_b
    cov = F.conv2d(ya * yb, win) - mu_a * mu_b
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    ssim = ((2 * mu_a * mu_b + c1) * (2 * cov + c2)) / ((mu_a * mu_a + mu_b * mu_b + c1) * (var_a + var_b + c2))
    return {"y_mse": mse, "y_psnr": math.inf if mse == 0 else -10.0 * math.log10(mse), "y_ssim": float(ssim.mean())}
