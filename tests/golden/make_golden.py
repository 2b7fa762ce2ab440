"""Write golden input/output vectors from the reference's own Python model.

Run in the build container only (it needs the reference checkout, which never
travels to the GPU box):

    python tests/golden/make_golden.py --reference /root/reference

It imports ``aeisu.runtime.load_model`` / ``upscale`` and ``FoldedAEISU``
from the reference (aeisu/runtime.py:45-103, aeisu/model.py:546-596) and
records, for the released folded checkpoints:

* ``cfg0_*``  -- config 0: the 3x256x256 seed-0 synthetic frame through
  ``upscale(tile=0)``; stored as crops plus per-channel statistics (the full
  3x512x512 output is not committed).
* ``small_*`` -- a 3x40x56 random frame: ``upscale`` at tile 0 and tile 32,
  and the raw packed coefficients of ``predict_coefficients`` on the padded
  frame, stored whole.
* ``tiling_*`` -- the 69x83 tile-32 case of tests/test_reference.py:109-117
  run with the released weights.

Only tensors are written (``.npz``, no pickles); inputs are regenerated from
seeds by the tests and checked against the stored SHA-256 of their bytes.
"""
from __future__ import annotations

import argparse
import hashlib
import sys
from pathlib import Path

import numpy as np
import torch
from torch.nn import functional as F

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().float().contiguous().numpy().tobytes()).hexdigest()


def small_frame(h: int, w: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.rand(3, h, w, generator=g)


CROPS = {"top_left": (0, 0), "centre": (224, 224), "bottom_right": (448, 448), "right_edge": (100, 448)}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, str(REPO))
    sys.path.insert(0, args.reference)
    from aeisu.runtime import load_model, upscale          # reference code, read-only import
    from aeisu_amd import frames

    torch.set_num_threads(8)
    for tag, ckpt in (("area", "aeisu_area.pt"), ("div2k", "aeisu_div2k_l1.pt")):
        model = load_model(Path(args.reference) / "weights" / ckpt, "cpu")
        out = {}
        src0 = frames.scene(256, 256, 0)
        y0 = upscale(model, src0, 0)
        out["cfg0_input_sha256"] = np.array(digest(src0))
        for name, (r, c) in CROPS.items():
            out[f"cfg0_crop_{name}"] = y0[:, r:r + 64, c:c + 64].numpy()
            out[f"cfg0_crop_{name}_origin"] = np.array([r, c])
        out["cfg0_mean"] = y0.mean(dim=(1, 2)).double().numpy()
        out["cfg0_std"] = y0.std(dim=(1, 2)).double().numpy()
        out["cfg0_sha256"] = np.array(digest(y0))

        src1 = small_frame(40, 56, 1)
        out["small_input"] = src1.numpy()
        out["small_tile0"] = upscale(model, src1, 0).numpy()
        out["small_tile32"] = upscale(model, src1, 32).numpy()
        ey, ex = -40 % 32, -56 % 32
        py, px = 16 + ey // 2, 16 + ex // 2
        padded = F.pad(src1[None], (px, 32 + ex - px, py, 32 + ey - py), mode="replicate")
        with torch.inference_mode():
            out["small_meta"] = model.predict_coefficients(padded).numpy()

        src2 = small_frame(69, 83, 2)
        out["tiling_input"] = src2.numpy()
        out["tiling_tile0"] = upscale(model, src2, 0).numpy()
        out["tiling_tile32"] = upscale(model, src2, 32).numpy()
        np.savez_compressed(HERE / f"reference_{tag}.npz", **out)
        print(tag, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
