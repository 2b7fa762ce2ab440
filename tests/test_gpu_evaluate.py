"""Evaluation path through the C ABI runtime: aeisu_amd.evaluate / aeisu_amd.infer on PNG folders.

Bars (north star): the FP16 policy's Y-PSNR equals the FP32 oracle's within 0.01 dB; the
Mixed policy's Y-PSNR is within 0.05 dB of the Mixed deployment emulated by the oracle;
file outputs follow the reference's evaluate.py (per_image.csv, summary.json, PNG + NPZ).
"""
from __future__ import annotations

import csv
import json
import sys

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from aeisu_amd import frames as FR
from aeisu_amd import imageio as IO
from aeisu_amd import metrics as MT
from oracle import deploy as D
from oracle import model as M
from oracle import spyr8f8
from tests._util import WEIGHTS, crop_output, pad_frame

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def pairs(tmp_path_factory, gpu):
    root = tmp_path_factory.mktemp("eval")
    for i, (h, w) in enumerate([(96, 128), (72, 104)]):
        hr = FR.pink_noise(2 * h, 2 * w, 70 + i) if i == 0 else FR.scene(2 * h, 2 * w, 71, shapes=6, texture=True)
        IO.save_rgb(root / "hr" / f"img{i}.png", hr)
        lr = F.interpolate(IO.read_rgb(root / "hr" / f"img{i}.png")[None], scale_factor=0.5, mode="area")[0]
        IO.save_rgb(root / "lr" / f"img{i}.png", lr)
    return root


def test_evaluate_fp16_matches_fp32_oracle(pairs, tmp_path):
    from aeisu_amd.evaluate import evaluate
    say("case: evaluate aeisu_area.pt (fp16 policy) on 2 PNG pairs, tile 0 and 32")
    state = M.load_folded(WEIGHTS / "aeisu_area.pt")
    for tile in (0, 32):
        out = tmp_path / f"t{tile}"
        rows, summary = evaluate(WEIGHTS / "aeisu_area.pt", pairs / "lr", pairs / "hr", out, tile=tile, log=say)
        for row, (lr, hr) in zip(rows, IO.paired_images(pairs / "lr", pairs / "hr")):
            ref = MT.distortion(M.upscale(state, IO.read_rgb(lr), 0), IO.read_rgb(hr))
            say(f"  tile {tile} {row['image']}: gpu {row['y_psnr']:.4f} dB, oracle {ref['y_psnr']:.4f} dB")
            assert abs(row["y_psnr"] - ref["y_psnr"]) < 0.01
            assert abs(row["y_ssim"] - ref["y_ssim"]) < 1e-4
        with (out / "per_image.csv").open() as fh:
            assert list(csv.DictReader(fh).fieldnames) == ["image", "y_mse", "y_psnr", "y_ssim"]
        s = json.loads((out / "summary.json").read_text())
        assert s["pairs"] == 2 and s["tile_lr"] == tile and s["precision"] == "fp16"
        png = IO.read_rgb(out / "images" / "img0.png")
        npz = torch.from_numpy(np.load(out / "images" / "img0.npz")["rgb"]).permute(2, 0, 1)
        assert torch.equal(png, torch.from_numpy(IO.quantize_u8(npz)).permute(2, 0, 1).float() / 255)


def test_evaluate_mixed_within_005db_of_emulation(pairs, tmp_path):
    from aeisu_amd.evaluate import evaluate
    say("case: evaluate aeisu_area_mixed_fp8.bin (mixed) vs oracle mixed emulation")
    rows, _ = evaluate(WEIGHTS / "aeisu_area_mixed_fp8.bin", pairs / "lr", pairs / "hr", tmp_path / "m", tile=0,
                       log=say)
    weights = D.weights_from_spyr(spyr8f8.read_file(WEIGHTS / "aeisu_area_mixed_fp8.bin"))
    for row, (lr, hr) in zip(rows, IO.paired_images(pairs / "lr", pairs / "hr")):
        src = IO.read_rgb(lr)
        h, w = src.shape[-2:]
        emu = crop_output(D.forward(pad_frame(src[None].half().float()), weights, "mixed"), h, w)[0].clamp(0, 1)
        ref = MT.distortion(emu, IO.read_rgb(hr))
        say(f"  {row['image']}: gpu {row['y_psnr']:.4f} dB, emulation {ref['y_psnr']:.4f} dB")
        assert abs(row["y_psnr"] - ref["y_psnr"]) < 0.05


def test_infer_cli_writes_the_evaluated_png(pairs, tmp_path):
    from aeisu_amd.evaluate import evaluate
    from aeisu_amd.infer import main as infer_main
    say("case: infer CLI on a folder")
    infer_main(["--checkpoint", str(WEIGHTS / "aeisu_area.pt"), "--input", str(pairs / "lr"),
                "--output", str(tmp_path / "inf"), "--tile", "32"])
    evaluate(WEIGHTS / "aeisu_area.pt", pairs / "lr", pairs / "hr", tmp_path / "ev", tile=32, log=say)
    for name in ("img0.png", "img1.png"):
        assert torch.equal(IO.read_rgb(tmp_path / "inf" / name), IO.read_rgb(tmp_path / "ev" / "images" / name))
    with pytest.raises(FileExistsError):
        infer_main(["--checkpoint", str(WEIGHTS / "aeisu_area.pt"), "--input", str(pairs / "lr"),
                    "--output", str(tmp_path / "inf")])
