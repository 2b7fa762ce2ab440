"""Evaluate the MI355X runtime on paired images (the reference's evaluate.py).

    python -m aeisu_amd.evaluate --checkpoint weights/aeisu_area.pt --input lr/ --target hr/ --output eval/

Follows evaluate.py:15-58 of the reference: pairs are matched by relative stem, each
prediction is ``upscale(model, read_rgb(lr), tile)`` (clipped float32), scored with
encoded-Y PSNR/SSIM after a ``--crop`` border (aeisu_amd.metrics), and saved as
images/<stem>.png (round-half-up) and images/<stem>.npz (float32 HWC); per_image.csv
and summary.json hold the scores and their equal-weight means.  The output folder must
be empty or absent.
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import math
from pathlib import Path

import numpy as np

from .imageio import paired_images, read_rgb, save_rgb
from .metrics import distortion
from .runtime import load_model, upscale


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as fh:
        for block in iter(lambda: fh.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def evaluate(checkpoint: Path, inputs: Path, targets: Path, output: Path, tile: int = 128, crop: int = 2,
             precision=None, device: str = "cuda", log=print):
    if output.exists() and any(output.iterdir()):
        raise FileExistsError("Choose an empty evaluation output folder")
    model = load_model(checkpoint, device, precision)
    pairs = paired_images(inputs, targets)
    output.mkdir(parents=True, exist_ok=True)
    rows = []
    for i, (src, tgt) in enumerate(pairs):
        pred = upscale(model, read_rgb(src), tile)
        scores = distortion(pred, read_rgb(tgt), crop)
        ident = src.relative_to(inputs).with_suffix("")
        dst = output / "images" / ident
        dst.parent.mkdir(parents=True, exist_ok=True)
        save_rgb(dst.parent / (dst.name + ".png"), pred)
        np.savez_compressed(dst.parent / (dst.name + ".npz"), rgb=pred.permute(1, 2, 0).numpy())
        rows.append({"image": ident.as_posix(), **scores})
        log(f"{i + 1}/{len(pairs)} {ident}: Y PSNR={scores['y_psnr']:.4f}")
    with (output / "per_image.csv").open("w", newline="", encoding="utf-8") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    means = {k: float(np.mean([r[k] for r in rows])) for k in rows[0] if k != "image"}
    means = {k: v if math.isfinite(v) else "Infinity" for k, v in means.items()}
    summary = {"pairs": len(rows), "mean_per_image": means, "aggregation": "equal per-image weighting",
               "checkpoint_sha256": _sha256(Path(checkpoint)), "precision": model.precision,
               "border_crop_hr": crop, "outputs": "clipped float32 before half-up PNG rounding",
               "device": str(model.device), "tile_lr": tile, "runtime": "libaeisu_amd (MI355X HIP kernels)"}
    (output / "summary.json").write_text(json.dumps(summary, indent=2) + "\n", encoding="utf-8")
    return rows, summary


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--checkpoint", type=Path, required=True)
    ap.add_argument("--input", type=Path, required=True)
    ap.add_argument("--target", type=Path, required=True)
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--tile", type=int, default=128)
    ap.add_argument("--crop", type=int, default=2)
    ap.add_argument("--precision", choices=("fp16", "mixed", "mixed-fp8mma", "int8"), default=None)
    ap.add_argument("--lpips", action="store_true", help="not available: needs pretrained AlexNet weights")
    args = ap.parse_args(argv)
    if args.lpips:
        raise FileNotFoundError("LPIPS needs pretrained AlexNet weights, which this installation does not provide")
    evaluate(args.checkpoint, args.input, args.target, args.output, args.tile, args.crop, args.precision, args.device)


if __name__ == "__main__":
    main()
