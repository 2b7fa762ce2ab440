"""Upscale an image file or image tree on the MI355X runtime (the reference's infer.py).

    python -m aeisu_amd.infer --checkpoint weights/aeisu_area_mixed_fp8.bin --input lr/ --output hr/

Flags and behaviour follow infer.py:9-26 of the reference: ``--tile`` is the LR core size
(multiple of 32, 0 = whole frame), outputs are 8-bit PNGs written with round-half-up, and
existing files are never overwritten.  ``--precision`` selects the arithmetic policy of
the loaded artifact (default: the file's natural one).  There is no CPU path.
"""
from __future__ import annotations

import argparse
from pathlib import Path

from .imageio import list_images, read_rgb, save_rgb
from .runtime import load_model, upscale


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--checkpoint", type=Path, required=True)
    ap.add_argument("--input", type=Path, required=True)
    ap.add_argument("--output", type=Path, required=True)
    ap.add_argument("--device", default="cuda", help="HIP device, e.g. cuda or cuda:0")
    ap.add_argument("--tile", type=int, default=128, help="LR core size, multiple of 32; zero for full frame")
    ap.add_argument("--precision", choices=("fp16", "mixed", "mixed-fp8mma", "int8"), default=None)
    args = ap.parse_args(argv)
    model = load_model(args.checkpoint, args.device, args.precision)
    images = [args.input] if args.input.is_file() else list_images(args.input)
    if not images:
        raise ValueError("No input images found")
    for path in images:
        dst = args.output if args.input.is_file() else args.output / path.relative_to(args.input).with_suffix(".png")
        if path.resolve() == dst.resolve() or dst.exists():
            raise FileExistsError(f"Refusing to overwrite: {dst}")
        save_rgb(dst, upscale(model, read_rgb(path), args.tile))
        print(f"{path.name} -> {dst}", flush=True)


if __name__ == "__main__":
    main()
