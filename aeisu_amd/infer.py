"""Command-line upscaling of an image file or a folder tree on the MI355X runtime.

    python -m aeisu_amd.infer --checkpoint weights/aeisu_area_mixed_fp8.bin --input lr/ --output hr/

Contract of the reference's CLI (infer.py:9-26): the same flags (``--tile`` is the LR core
size, a multiple of 32, 0 for the whole frame), 8-bit PNG outputs written with round-half-up,
and no existing file is ever replaced.  Here the whole job is planned first: every source is
paired with its destination and every destination is checked before the first image is
decoded, so a conflict leaves the output tree untouched; two sources that map to one PNG
(x.jpg and x.png in one folder) are a conflict too, and each PNG is checked again just before
it is written.  ``--precision`` picks the
arithmetic policy of the loaded artifact (default: the file's natural one).  All arithmetic
runs in the HIP runtime; there is no CPU path.
"""
from __future__ import annotations

import argparse
from dataclasses import dataclass
from pathlib import Path
from typing import List, Sequence

from .imageio import list_images, read_rgb, save_rgb
from .runtime import load_model, upscale

PRECISIONS = ("fp16", "mixed", "mixed-fp8mma", "int8", "fp32")


@dataclass(frozen=True)
class Job:
    source: Path
    destination: Path


def plan(source: Path, output: Path) -> List[Job]:
    """Pairs of (image, PNG to write): one file maps to ``output`` itself, a folder tree is mirrored
    under ``output`` with every suffix replaced by .png."""
    if source.is_file():
        jobs = [Job(source, output)]
    else:
        jobs = [Job(p, output / p.relative_to(source).with_suffix(".png")) for p in list_images(source)]
    if not jobs:
        raise ValueError("No input images found")
    seen = set()
    clashes = []
    for j in jobs:
        dest = j.destination.resolve()
        if j.destination.exists() or dest == j.source.resolve() or dest in seen:
            clashes.append(j.destination)
        seen.add(dest)
    if clashes:
        raise FileExistsError(f"Refusing to overwrite: {clashes[0]}" +
                              (f" (and {len(clashes) - 1} more)" if len(clashes) > 1 else ""))
    return jobs


def parse_args(argv: Sequence[str] | None) -> argparse.Namespace:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--checkpoint", type=Path, required=True, help="folded .pt, SPYR8F8 .bin or INT8 .pt")
    parser.add_argument("--input", type=Path, required=True, help="an image file or a folder of images")
    parser.add_argument("--output", type=Path, required=True, help="PNG path (file input) or folder")
    parser.add_argument("--device", default="cuda", help="HIP device, e.g. cuda or cuda:1")
    parser.add_argument("--tile", type=int, default=128, help="LR core size, multiple of 32; zero for full frame")
    parser.add_argument("--precision", choices=PRECISIONS, default=None, help="arithmetic policy")
    return parser.parse_args(argv)


def main(argv: Sequence[str] | None = None) -> None:
    args = parse_args(argv)
    jobs = plan(args.input, args.output)
    model = load_model(args.checkpoint, args.device, args.precision)
    for n, job in enumerate(jobs, 1):
        result = upscale(model, read_rgb(job.source), args.tile)
        if job.destination.exists():
            raise FileExistsError(f"Refusing to overwrite: {job.destination}")
        save_rgb(job.destination, result)
        print(f"[{n}/{len(jobs)}] {job.source.name} -> {job.destination}", flush=True)


if __name__ == "__main__":
    main()
