"""Score the MI355X runtime on paired low/high-resolution images.

    python -m aeisu_amd.evaluate --checkpoint weights/aeisu_area.pt --input lr/ --target hr/ --output eval/

Every input image is upscaled by the HIP runtime (``upscale(model, image, tile)``, clipped float32),
scored against its target with encoded-Y PSNR/SSIM after a ``--crop`` border (aeisu_amd.metrics), and
kept.  The output folder layout is the reference's evaluation format (evaluate.py:15-58), so tools
that read the reference's results read these:

* ``images/<stem>.png`` (8-bit, round-half-up) and ``images/<stem>.npz`` (key ``rgb``: float32 HWC);
* ``per_image.csv``: columns ``image, y_mse, y_psnr, y_ssim``, one row per pair in stem order;
* ``summary.json``: ``pairs``, ``mean_per_image`` (equal weight per image; a non-finite mean, such as
  the PSNR of an exact reproduction, is written as the string ``"Infinity"``), ``aggregation``,
  ``checkpoint_sha256``, ``precision``, ``border_crop_hr``, ``outputs``, ``device``, ``tile_lr``, and
  ``runtime``.

The folder must be empty or absent.  Scores are streamed to the CSV as each image finishes, so a run
stopped part-way still leaves the scores of the images it completed.
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import math
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np
import torch

from .imageio import paired_images, read_rgb, save_rgb
from .metrics import distortion
from .runtime import load_model, upscale

SCORES = ("y_mse", "y_psnr", "y_ssim")
PRECISIONS = ("fp16", "mixed", "mixed-fp8mma", "int8", "fp32")


def file_digest(path: Path) -> str:
    """SHA-256 of a file, read in 1 MiB blocks."""
    digest = hashlib.sha256()
    with Path(path).open("rb") as fh:
        while block := fh.read(1 << 20):
            digest.update(block)
    return digest.hexdigest()


def _finite_or_label(v: float):
    """JSON has no infinity: a non-finite mean is stored as the string "Infinity"."""
    return v if math.isfinite(v) else "Infinity"


@dataclass
class ScoreLog:
    """Per-image scores: appended to per_image.csv as they arrive, averaged at the end."""
    csv_path: Path
    rows: List[Dict[str, object]] = field(default_factory=list)

    def __post_init__(self) -> None:
        self._fh = self.csv_path.open("w", newline="", encoding="utf-8")
        self._writer = csv.writer(self._fh)
        self._writer.writerow(("image",) + SCORES)

    def add(self, key: str, scores: Dict[str, float]) -> None:
        self._writer.writerow([key] + [scores[s] for s in SCORES])
        self._fh.flush()
        self.rows.append({"image": key, **{s: scores[s] for s in SCORES}})

    def means(self) -> Dict[str, object]:
        return {s: _finite_or_label(float(np.mean([r[s] for r in self.rows]))) for s in SCORES}

    def close(self) -> None:
        self._fh.close()


def _store(images: Path, key: str, prediction: torch.Tensor) -> None:
    """images/<key>.png and images/<key>.npz of one prediction (CHW float, already clipped)."""
    base = images / key
    base.parent.mkdir(parents=True, exist_ok=True)
    save_rgb(base.with_name(base.name + ".png"), prediction)
    np.savez_compressed(base.with_name(base.name + ".npz"), rgb=prediction.permute(1, 2, 0).contiguous().numpy())


def evaluate(checkpoint: Path, inputs: Path, targets: Path, output: Path, tile: int = 128, crop: int = 2,
             precision: Optional[str] = None, device: str = "cuda",
             log: Callable[[str], None] = print) -> Tuple[List[Dict[str, object]], Dict[str, object]]:
    """Evaluate ``checkpoint`` on the pairs under ``inputs``/``targets``; returns (rows, summary)."""
    inputs, targets, output = Path(inputs), Path(targets), Path(output)
    if output.is_dir() and next(output.iterdir(), None) is not None:
        raise FileExistsError(f"evaluation output {output} is not empty")
    pairs = [(src.relative_to(inputs).with_suffix("").as_posix(), src, tgt)
             for src, tgt in paired_images(inputs, targets)]
    model = load_model(checkpoint, device, precision)
    output.mkdir(parents=True, exist_ok=True)
    scores_log = ScoreLog(output / "per_image.csv")
    try:
        for n, (key, src, tgt) in enumerate(pairs, 1):
            prediction = upscale(model, read_rgb(src), tile)
            scores = distortion(prediction, read_rgb(tgt), crop)
            _store(output / "images", key, prediction)
            scores_log.add(key, scores)
            log(f"[{n}/{len(pairs)}] {key}  Y-PSNR {scores['y_psnr']:.4f} dB  Y-SSIM {scores['y_ssim']:.5f}")
    finally:
        scores_log.close()
    summary = {
        "pairs": len(scores_log.rows), "mean_per_image": scores_log.means(), "aggregation": "equal per-image weighting",
        "checkpoint_sha256": file_digest(Path(checkpoint)), "precision": model.precision, "border_crop_hr": crop,
        "outputs": "clipped float32 before half-up PNG rounding", "device": str(model.device), "tile_lr": tile,
        "runtime": "libaeisu_amd (MI355X HIP kernels)",
    }
    (output / "summary.json").write_text(json.dumps(summary, indent=2) + "\n", encoding="utf-8")
    return scores_log.rows, summary


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--checkpoint", type=Path, required=True, help="folded .pt, SPYR8F8 .bin or INT8 .pt")
    ap.add_argument("--input", type=Path, required=True, help="folder of low-resolution images")
    ap.add_argument("--target", type=Path, required=True, help="folder of targets with the same relative stems")
    ap.add_argument("--output", type=Path, required=True, help="empty or absent folder for the results")
    ap.add_argument("--device", default="cuda", help="HIP device, e.g. cuda or cuda:1")
    ap.add_argument("--tile", type=int, default=128, help="LR core size, multiple of 32; zero for full frame")
    ap.add_argument("--crop", type=int, default=2, help="HR border excluded from the scores")
    ap.add_argument("--precision", choices=PRECISIONS, default=None, help="arithmetic policy")
    ap.add_argument("--lpips", action="store_true", help="not available: needs pretrained AlexNet weights")
    args = ap.parse_args(argv)
    if args.lpips:
        raise FileNotFoundError("LPIPS is not available: its pretrained AlexNet weights are not installed here")
    evaluate(args.checkpoint, args.input, args.target, args.output, args.tile, args.crop, args.precision, args.device)


if __name__ == "__main__":
    main()
