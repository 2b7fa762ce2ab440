"""Seeded synthetic RGB frames for the benchmark configurations.

The reference publishes no test images; its benchmark configurations are
specified in words.  This module renders them deterministically:

* ``scene``: a sum of two linear colour gradients, ``shapes`` random solid
  polygons / ellipses with edges antialiased by 4x4 area supersampling, an
  optional 2-octave value-noise texture inside the shapes, and uniform noise
  of +-0.02, clipped to [0, 1]   (configs 0-3).
* ``pink_noise``: per-channel 1/f-spectrum colour noise (mean 0.45, std 0.2,
  clipped) rendered at twice the size and 2x bicubic-downsampled (config 4).
* ``scene_pair`` / ``pink_pair``: the same with the 2x render returned as an
  HR target for PSNR (scenes are 2x area-downsampled).

All random parameters come from ``numpy.random.default_rng(seed)``; pixel
arithmetic is float32 torch on the CPU so that frames are identical wherever
they are generated.
"""
from __future__ import annotations

import math

import numpy as np
import torch
from torch.nn import functional as F


def _coverage_polygon(xs: torch.Tensor, ys: torch.Tensor, verts: np.ndarray) -> torch.Tensor:
    """Even-odd point-in-polygon test on sample coordinates (broadcast tensors)."""
    inside = torch.zeros(torch.broadcast_shapes(xs.shape, ys.shape), dtype=torch.bool)
    n = len(verts)
    for i in range(n):
        x0, y0 = (float(v) for v in verts[i])
        x1, y1 = (float(v) for v in verts[(i + 1) % n])
        if y0 == y1:
            continue
        crosses = (ys >= min(y0, y1)) & (ys < max(y0, y1))
        xint = x0 + (ys - y0) * ((x1 - x0) / (y1 - y0))
        inside ^= crosses & (xs < xint)
    return inside


def _value_noise(h: int, w: int, cell: int, rng: np.random.Generator) -> torch.Tensor:
    """Bilinear value noise in [-1, 1] with lattice spacing ``cell`` pixels."""
    gh, gw = h // cell + 2, w // cell + 2
    grid = torch.from_numpy(rng.uniform(-1.0, 1.0, (1, 1, gh, gw)).astype(np.float32))
    up = F.interpolate(grid, scale_factor=cell, mode="bilinear", align_corners=True)
    return up[0, 0, :h, :w]


def scene(height: int, width: int, seed: int, shapes: int = 12, texture: bool = False) -> torch.Tensor:
    """3 x height x width float32 frame in [0, 1]."""
    rng = np.random.default_rng(seed)
    yy = torch.arange(height, dtype=torch.float32).view(-1, 1) / max(height - 1, 1)
    xx = torch.arange(width, dtype=torch.float32).view(1, -1) / max(width - 1, 1)
    img = torch.zeros(3, height, width)
    for _ in range(2):
        c0 = torch.from_numpy(rng.uniform(0.0, 0.5, 3).astype(np.float32)).view(3, 1, 1)
        gx = torch.from_numpy(rng.uniform(-0.25, 0.25, 3).astype(np.float32)).view(3, 1, 1)
        gy = torch.from_numpy(rng.uniform(-0.25, 0.25, 3).astype(np.float32)).view(3, 1, 1)
        img += c0 + gx * xx + gy * yy
    tex = None
    if texture:
        tex = 0.1 * 0.5 * (_value_noise(height, width, 32, rng) + 0.5 * _value_noise(height, width, 8, rng))
    sub = (torch.arange(4, dtype=torch.float32) + 0.5) / 4.0
    scale = float(min(height, width))
    for _ in range(shapes):
        colour = torch.from_numpy(rng.uniform(0.0, 1.0, 3).astype(np.float32)).view(3, 1, 1)
        cx, cy = rng.uniform(0, width), rng.uniform(0, height)
        radius = rng.uniform(0.05, 0.25) * scale
        if rng.uniform() < 0.5:
            kind, rx, ry, rot = "ellipse", radius, radius * rng.uniform(0.3, 1.0), rng.uniform(0, math.pi)
            reach = radius
        else:
            kind = "polygon"
            count = int(rng.integers(3, 7))
            ang = np.sort(rng.uniform(0, 2 * math.pi, count))
            rad = radius * rng.uniform(0.4, 1.0, count)
            verts = np.stack((cx + rad * np.cos(ang), cy + rad * np.sin(ang)), 1)
            reach = float(rad.max())
        x0, x1 = max(int(cx - reach) - 1, 0), min(int(cx + reach) + 2, width)
        y0, y1 = max(int(cy - reach) - 1, 0), min(int(cy + reach) + 2, height)
        if x0 >= x1 or y0 >= y1:
            continue
        px = (torch.arange(x0, x1, dtype=torch.float32).view(1, -1, 1, 1) + sub.view(1, 1, 1, 4))
        py = (torch.arange(y0, y1, dtype=torch.float32).view(-1, 1, 1, 1) + sub.view(1, 1, 4, 1))
        if kind == "ellipse":
            dx, dy = px - cx, py - cy
            c, s = math.cos(rot), math.sin(rot)
            u, v = dx * c + dy * s, -dx * s + dy * c
            inside = (u / rx) ** 2 + (v / ry) ** 2 <= 1.0
        else:
            inside = _coverage_polygon(px, py, verts)
        cov = inside.float().mean(dim=(2, 3))                  # [h, w] area coverage
        fill = colour.expand(3, y1 - y0, x1 - x0)
        if tex is not None:
            fill = fill + tex[y0:y1, x0:x1]
        region = img[:, y0:y1, x0:x1]
        img[:, y0:y1, x0:x1] = region * (1 - cov) + fill * cov
    img += torch.from_numpy(rng.uniform(-0.02, 0.02, (3, height, width)).astype(np.float32))
    return img.clamp(0, 1)


def scene_pair(height: int, width: int, seed: int, shapes: int = 12, texture: bool = True):
    """(LR, HR): the scene rendered at 2x (the HR target) and 2x area-downsampled to height x width."""
    hr = scene(2 * height, 2 * width, seed, shapes=shapes, texture=texture)
    return F.avg_pool2d(hr[None], 2)[0], hr


def pink_noise(height: int, width: int, seed: int) -> torch.Tensor:
    """3 x height x width 1/f colour noise, rendered at 2x then bicubic-downsampled."""
    return pink_pair(height, width, seed)[0]


def pink_pair(height: int, width: int, seed: int):
    """(LR, HR) of ``pink_noise``: the 2x render is the HR target."""
    rng = np.random.default_rng(seed)
    hh, ww = 2 * height, 2 * width
    fy = np.fft.fftfreq(hh).reshape(-1, 1)
    fx = np.fft.rfftfreq(ww).reshape(1, -1)
    f = np.sqrt(fx * fx + fy * fy)
    f[0, 0] = 1.0
    chans = []
    for _ in range(3):
        spec = (rng.standard_normal(f.shape) + 1j * rng.standard_normal(f.shape)) / f
        spec[0, 0] = 0.0
        field = np.fft.irfft2(spec, s=(hh, ww)).astype(np.float64)
        field = (field - field.mean()) / max(field.std(), 1e-12)
        chans.append(np.clip(0.45 + 0.2 * field, 0.0, 1.0).astype(np.float32))
    hr = torch.from_numpy(np.stack(chans))[None]
    lr = F.interpolate(hr, size=(height, width), mode="bicubic", align_corners=False, antialias=True)
    return lr[0].clamp(0, 1), hr[0]


CONFIGS = {
    0: dict(batch=1, height=256, width=256, dtype="fp32", kind="scene", texture=False),
    1: dict(batch=1, height=1080, width=1920, dtype="fp16", kind="scene", texture=True),
    2: dict(batch=1, height=1080, width=1920, dtype="fp16", kind="scene", texture=True),
    3: dict(batch=8, height=540, width=960, dtype="fp16", kind="scene", texture=True),
    4: dict(batch=4, height=1440, width=2560, dtype="fp16", kind="pink", texture=False),
}


def config_frames(config: int, seed: int = 0, batch: int | None = None,
                  size: tuple[int, int] | None = None) -> torch.Tensor:
    """B x 3 x H x W frames of a benchmark configuration (frame i uses seed + i); ``batch`` and
    ``size`` = (H, W) override the configuration's for resolution sweeps."""
    spec = CONFIGS[config]
    n = spec["batch"] if batch is None else batch
    h, w = (spec["height"], spec["width"]) if size is None else size
    frames = []
    for i in range(n):
        if spec["kind"] == "scene":
            frames.append(scene(h, w, seed + i, texture=spec["texture"]))
        else:
            frames.append(pink_noise(h, w, seed + i))
    out = torch.stack(frames)
    if spec["dtype"] == "fp16":
        out = out.half()
    return out
