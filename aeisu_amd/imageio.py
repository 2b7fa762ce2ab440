"""RGB image files <-> CHW float tensors, and image-tree helpers.

Semantics of the reference (aeisu/runtime.py:17-27, aeisu/data.py:14-29): files are
decoded to 8-bit RGB and scaled by 1/255; outputs are clamped to [0, 1] and written
as 8-bit RGB PNG with round-half-up quantisation floor(255 x + 0.5).
"""
from __future__ import annotations

from pathlib import Path
from typing import Dict, List, Tuple

import numpy as np
import torch

IMAGE_EXTENSIONS = {".png", ".jpg", ".jpeg", ".bmp", ".tif", ".tiff", ".webp"}


def read_rgb(path) -> torch.Tensor:
    from PIL import Image
    with Image.open(path) as image:
        array = np.array(image.convert("RGB"), dtype=np.uint8, copy=True)
    return torch.from_numpy(array).permute(2, 0, 1).float() / 255.0


def quantize_u8(image: torch.Tensor) -> np.ndarray:
    """CHW float -> HWC uint8 with clamp and round-half-up."""
    array = image.detach().cpu().float().clamp(0, 1).permute(1, 2, 0).numpy()
    return np.floor(array * 255.0 + 0.5).astype(np.uint8)


def save_rgb(path, image: torch.Tensor) -> None:
    from PIL import Image
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    Image.fromarray(quantize_u8(image)).save(path)


def list_images(root) -> List[Path]:
    root = Path(root)
    return sorted(p for p in root.rglob("*") if p.is_file() and p.suffix.lower() in IMAGE_EXTENSIONS)


def paired_images(source, target) -> List[Tuple[Path, Path]]:
    """Pairs of files with identical relative stems under two roots."""
    def index(root) -> Dict[str, Path]:
        out: Dict[str, Path] = {}
        for p in list_images(root):
            key = p.relative_to(root).with_suffix("").as_posix()
            if key in out:
                raise ValueError(f"{root} holds two images with the relative stem {key!r}")
            out[key] = p
        return out
    a, b = index(Path(source)), index(Path(target))
    if not a or a.keys() != b.keys():
        raise ValueError(f"input and target folders differ in their relative stems "
                         f"({len(a)} inputs, {len(b)} targets, {len(a.keys() ^ b.keys())} unmatched)")
    return [(a[k], b[k]) for k in sorted(a)]
