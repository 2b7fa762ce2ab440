"""Evaluation-path pieces that need no GPU: encoded-Y PSNR/SSIM and image I/O.

Definitions pinned against the reference (aeisu/metrics.py:11-39, aeisu/runtime.py:17-27,
aeisu/data.py:14-29) by closed forms and a brute-force windowed SSIM written with loops.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from aeisu_amd import imageio as IO
from aeisu_amd import metrics as MT


def _ssim_bruteforce(a: np.ndarray, b: np.ndarray) -> float:
    """Mean SSIM of two HW float64 arrays, valid 11x11 Gaussian (sigma 1.5) windows, explicit loops."""
    g = np.exp(-((np.arange(11) - 5.0) ** 2) / (2 * 1.5 ** 2))
    g /= g.sum()
    w = np.outer(g, g)
    vals = []
    for y in range(a.shape[0] - 10):
        for x in range(a.shape[1] - 10):
            pa, pb = a[y:y + 11, x:x + 11], b[y:y + 11, x:x + 11]
            ma, mb = (w * pa).sum(), (w * pb).sum()
            va, vb = (w * pa * pa).sum() - ma * ma, (w * pb * pb).sum() - mb * mb
            cv = (w * pa * pb).sum() - ma * mb
            vals.append(((2 * ma * mb + 1e-4) * (2 * cv + 9e-4)) / ((ma * ma + mb * mb + 1e-4) * (va + vb + 9e-4)))
    return float(np.mean(vals))


def test_luma_closed_form():
    white, black = torch.ones(3, 1, 1, dtype=torch.float64), torch.zeros(3, 1, 1, dtype=torch.float64)
    assert MT.luma(white).item() == pytest.approx(235 / 255, abs=1e-12)
    assert MT.luma(black).item() == pytest.approx(16 / 255, abs=1e-15)


def test_distortion_against_bruteforce():
    g = torch.Generator().manual_seed(2)
    a = torch.rand(3, 21, 24, generator=g)
    b = (a + 0.05 * torch.randn(3, 21, 24, generator=g)).clamp(0, 1)
    got = MT.distortion(a, b, crop=2)
    ya = MT.luma(a.double()[:, 2:-2, 2:-2])[0].numpy()
    yb = MT.luma(b.double()[:, 2:-2, 2:-2])[0].numpy()
    mse = float(((ya - yb) ** 2).mean())
    assert got["y_mse"] == pytest.approx(mse, rel=1e-12)
    assert got["y_psnr"] == pytest.approx(-10 * math.log10(mse), rel=1e-12)
    assert got["y_ssim"] == pytest.approx(_ssim_bruteforce(ya, yb), abs=1e-12)
    # the prediction is clamped, the target is not
    assert MT.distortion(a * 3, b)["y_mse"] == pytest.approx(MT.distortion((a * 3).clamp(0, 1), b)["y_mse"])


def test_distortion_identity_and_errors():
    a = torch.rand(3, 16, 16)
    same = MT.distortion(a, a, crop=2)
    assert same["y_psnr"] == math.inf and same["y_ssim"] == pytest.approx(1.0, abs=1e-12)
    with pytest.raises(ValueError):
        MT.distortion(a, a[:, :15])
    with pytest.raises(ValueError):
        MT.distortion(a, torch.full_like(a, float("nan")))
    with pytest.raises(ValueError):
        MT.distortion(a[:, :14, :14], a[:, :14, :14], crop=2)          # 14 < 11 + 2 * 2
    with pytest.raises(ValueError):
        MT.distortion(a, a, crop=-1)


def test_png_round_half_up_and_round_trip(tmp_path):
    k = torch.arange(256, dtype=torch.float32)
    img = (k / 255).view(1, 16, 16).expand(3, 16, 16).contiguous()
    IO.save_rgb(tmp_path / "a.png", img)
    back = IO.read_rgb(tmp_path / "a.png")
    assert torch.equal(back, img)
    half = torch.tensor([0.5 / 255, 0.4999 / 255, 254.5 / 255, 1.7, -0.2]).view(1, 1, 5).expand(3, 1, 5)
    assert IO.quantize_u8(half)[0, :, 0].tolist() == [1, 0, 255, 255, 0]


def test_paired_images(tmp_path):
    for root in ("lr", "hr"):
        (tmp_path / root / "sub").mkdir(parents=True)
        IO.save_rgb(tmp_path / root / "sub" / "x.png", torch.zeros(3, 4, 4))
    pairs = IO.paired_images(tmp_path / "lr", tmp_path / "hr")
    assert [p[0].name for p in pairs] == ["x.png"]
    IO.save_rgb(tmp_path / "lr" / "y.png", torch.zeros(3, 4, 4))
    with pytest.raises(ValueError):
        IO.paired_images(tmp_path / "lr", tmp_path / "hr")
    IO.save_rgb(tmp_path / "hr" / "y.png", torch.zeros(3, 4, 4))
    IO.save_rgb(tmp_path / "hr" / "y.jpg", torch.zeros(3, 4, 4))
    with pytest.raises(ValueError):
        IO.paired_images(tmp_path / "lr", tmp_path / "hr")


def test_infer_plan_checks_every_destination_first(tmp_path):
    """The CLI pairs each image with its PNG and refuses the whole job if any destination exists
    (the reference never overwrites, infer.py:21-23), before decoding or writing anything."""
    import numpy as np
    from PIL import Image
    from aeisu_amd.infer import plan
    src = tmp_path / "in"
    (src / "sub").mkdir(parents=True)
    for name in ("x.jpg", "sub/y.png"):
        Image.fromarray(np.zeros((8, 8, 3), np.uint8)).save(src / name)
    jobs = plan(src, tmp_path / "out")
    assert [j.destination.relative_to(tmp_path / "out").as_posix() for j in jobs] == ["sub/y.png", "x.png"]
    assert plan(src / "x.jpg", tmp_path / "one.png")[0].destination == tmp_path / "one.png"
    (tmp_path / "out" / "sub").mkdir(parents=True)
    (tmp_path / "out" / "sub" / "y.png").write_bytes(b"")
    with pytest.raises(FileExistsError, match="Refusing to overwrite"):
        plan(src, tmp_path / "out")
    assert not (tmp_path / "out" / "x.png").exists()
    (tmp_path / "empty").mkdir()
    with pytest.raises(ValueError, match="No input images found"):
        plan(tmp_path / "empty", tmp_path / "o2")


def test_infer_plan_rejects_two_sources_with_one_destination(tmp_path):
    """x.jpg and x.png in one folder both map to out/x.png: the plan refuses the job (the reference
    raises on the second write, infer.py:21-23) instead of letting one output replace the other."""
    import numpy as np
    from PIL import Image
    from aeisu_amd.infer import plan
    src = tmp_path / "in"
    src.mkdir()
    for name in ("x.jpg", "x.png", "z.tif"):
        Image.fromarray(np.zeros((8, 8, 3), np.uint8)).save(src / name)
    with pytest.raises(FileExistsError, match="Refusing to overwrite"):
        plan(src, tmp_path / "out")
    assert not (tmp_path / "out").exists()


def test_infer_cli_accepts_fp32_policy():
    from aeisu_amd.infer import PRECISIONS, parse_args
    assert "fp32" in PRECISIONS
    args = parse_args(["--checkpoint", "m.pt", "--input", "a", "--output", "b", "--precision", "fp32"])
    assert args.precision == "fp32"


def test_score_log_writes_reference_csv_and_infinity(tmp_path):
    """per_image.csv columns and the "Infinity" encoding of a non-finite mean (the reference's
    evaluation format, evaluate.py:46-53)."""
    import csv
    import math
    from aeisu_amd.evaluate import ScoreLog
    log = ScoreLog(tmp_path / "per_image.csv")
    log.add("a", {"y_mse": 0.0, "y_psnr": math.inf, "y_ssim": 1.0})
    log.add("b/c", {"y_mse": 1e-4, "y_psnr": 40.0, "y_ssim": 0.98})
    log.close()
    with (tmp_path / "per_image.csv").open() as fh:
        rows = list(csv.DictReader(fh))
    assert list(rows[0]) == ["image", "y_mse", "y_psnr", "y_ssim"]
    assert [r["image"] for r in rows] == ["a", "b/c"] and rows[0]["y_psnr"] == "inf"
    means = log.means()
    assert means["y_psnr"] == "Infinity" and means["y_mse"] == pytest.approx(5e-5) and means["y_ssim"] == pytest.approx(0.99)
