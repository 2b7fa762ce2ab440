"""Frames at the largest geometry the boundary accepts, on the GPU, against the CPU oracle.

aeisu_configure accepts frames up to 8192 x 8192 and rejects larger ones, as the reference's
runtime test expects (SrcPyrRuntimeTest.cpp:302-303).  At 8192 x 8192 an FP32 output frame is
3.2 GB and a batch of two FP16 output frames 3.2 GB, so every byte offset the kernels form
(32-bit raw-buffer offsets inside a frame, 64-bit frame bases) is exercised near its limit.
The largest batch (1024 frames) is checked against single-frame runs.

The oracle cannot run a whole 8192 x 8192 frame in seconds, so it runs the frame's bottom-right
corner: the last 384 x 384 input pixels, a sub-frame whose origin is a multiple of 32, so that
its padded grid (align 32, halo 16: aeisu/runtime.py:82-84) lines up with the whole frame's on
the half- and quarter-resolution grids.  An output pixel depends on input pixels less than 32
pixels away (the head's 5 x 5 taps, refine's 3 x 3 on the half grid, the four 3 x 3 layers on the
quarter grid, the 4 x 4 analysis window; the reference's tiled path takes 32 pixels of context for
the same reason, aeisu/runtime.py:72, 95-96), so the sub-frame's own top and left padding reaches
no output pixel more than 256 input pixels from its edges: the last 128 x 128 input pixels' output
(256 x 256 x 3 values, the frame's largest offsets) is the whole frame's output there.

Bounds: the FP16 policy against the FP32 reference path <= 1e-3; Mixed and INT8 against their
emulation <= 2/255, with the residual deviation of gfx950's FP16 MFMA accumulation that the
full-size tests allow (at most 1e-6 of the values between 2/255 and 4/255; at this crop's
196,608 values that is none).
"""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import deploy as D
from oracle import model as M
from oracle import spyr8f8
from tests._util import WEIGHTS, crop_output, pad_frame

pytestmark = pytest.mark.gpu

MAX = 8192          # largest frame side aeisu_configure accepts
SUB = 384           # oracle sub-frame side (bottom-right corner)
KEEP = 128          # compared input pixels at the sub-frame's far edges


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def R(gpu):
    torch.set_num_threads(16)
    from aeisu_amd import runtime
    return runtime


def _frames(batch: int, dtype, seed: int) -> torch.Tensor:
    """[batch, 3, MAX, MAX] on the device: smooth colour fields, a finer pattern and +-0.02 noise,
    in [0, 1] (the oracle reads the corner back, so the device's own arithmetic defines the input)."""
    dev = torch.device("cuda")
    y = torch.arange(MAX, device=dev, dtype=torch.float32)[:, None]
    x = torch.arange(MAX, device=dev, dtype=torch.float32)[None, :]
    gen = torch.Generator(device=dev).manual_seed(seed)
    out = torch.empty(batch, 3, MAX, MAX, device=dev, dtype=dtype)
    for b in range(batch):
        for c in range(3):
            f = (0.5 + 0.22 * torch.sin(x * (0.011 + 0.003 * c) + y * (0.006 * (c + 1)) + 0.7 * b + seed)
                 + 0.12 * torch.sin((0.09 * x - 0.07 * y) * (1.0 + 0.25 * c)))
            f += 0.04 * (torch.rand(MAX, MAX, device=dev, generator=gen) - 0.5)
            out[b, c] = f.clamp_(0.0, 1.0).to(dtype)
            del f
    return out


def _corner(frames: torch.Tensor, b: int) -> torch.Tensor:
    return frames[b, :, MAX - SUB:, MAX - SUB:].float().cpu()


def _got_corner(out: torch.Tensor, b: int) -> torch.Tensor:
    k = 2 * KEEP
    return out[b, :, 2 * MAX - k:, 2 * MAX - k:].float().cpu()


def _check_quantized(tag: str, got: torch.Tensor, ref: torch.Tensor) -> None:
    err = (got - ref).abs()
    over = int((err > 2 / 255).sum())
    say(f"  {tag}: max|gpu - emulation| {err.max().item() * 255:.3f}/255, {over} of {err.numel()} above 2/255")
    assert over <= 1e-6 * err.numel() and err.max().item() <= 4 / 255


def test_configure_rejects_beyond_maximum(R):
    model = R.load_model(WEIGHTS / "aeisu_area_mixed_fp8.bin", precision="mixed")
    try:
        for batch, h, w in [(1, MAX + 1, 64), (1, 64, MAX + 1), (1025, 32, 32), (0, 32, 32), (1, 0, 32), (1, 32, -4)]:
            with pytest.raises(ValueError):
                model.handle(batch, h, w)
        hd = model.handle(1, MAX, MAX)                        # the maximum itself configures
        assert model.geometry(hd)[:2] == (MAX + 32, MAX + 32)
    finally:
        model.close()


@pytest.mark.parametrize("precision,artifact", [("mixed", "aeisu_area_mixed_fp8.bin"), ("int8", "aeisu_int8_fp16.pt"),
                                                ("fp16", "aeisu_area.pt")])
def test_maximum_batch_equals_single_frames(R, precision, artifact):
    """The largest batch aeisu_configure accepts (1024 frames, here of 12 x 20 pixels) gives each
    frame exactly what the frame gives alone."""
    say(f"case: {precision}, batch 1024 x 3 x 12 x 20")
    gen = torch.Generator().manual_seed(5)
    frames = torch.rand(1024, 3, 12, 20, generator=gen).half().cuda()
    model = R.load_model(WEIGHTS / artifact, precision=precision)
    try:
        out = model.run(frames)
        for i in (0, 1, 511, 1022, 1023):
            assert torch.equal(out[i:i + 1], model.run(frames[i:i + 1].contiguous())), f"frame {i}"
    finally:
        model.close()


@pytest.mark.parametrize("precision,artifact,in_dtype,out_dtype,batch", [
    ("fp16", "aeisu_area.pt", torch.float32, torch.float32, 1),
    ("mixed", "aeisu_area_mixed_fp8.bin", torch.float16, torch.float16, 2),
    ("mixed", "aeisu_area_mixed_fp8.bin", torch.float32, torch.float32, 1),
    ("int8", "aeisu_int8_fp16.pt", torch.float16, torch.float32, 1),
])
def test_maximum_frame_corner_vs_oracle(R, precision, artifact, in_dtype, out_dtype, batch):
    say(f"case: {precision}, {batch} x 3 x {MAX} x {MAX}, {in_dtype} in, {out_dtype} out")
    frames = _frames(batch, in_dtype, seed=11)
    model = R.load_model(WEIGHTS / artifact, precision=precision)
    try:
        out = model.run(frames, out_dtype=out_dtype)
        torch.cuda.synchronize()
        assert out.shape == (batch, 3, 2 * MAX, 2 * MAX) and out.dtype == out_dtype
        b = batch - 1                                         # the batch's last frame: largest offsets
        got = _got_corner(out, b)
        sub = _corner(frames, b)
        if precision == "mixed" and batch == 1:
            # the per-layer path (coefficients through device memory: 2.2 GB at this size) agrees
            from aeisu_amd import _lib as L
            unfused = model.run(frames, out_dtype=out_dtype, flags=L.FLAG_UNFUSED)
            torch.cuda.synchronize()
            assert torch.equal(out, unfused)
            del unfused
        del out, frames
        torch.cuda.empty_cache()
    finally:
        model.close()
    k = 2 * KEEP
    if precision == "fp16":
        ref = M.upscale(M.load_folded(WEIGHTS / artifact), sub, 0)[:, -k:, -k:]
        err = (got - ref).abs().max().item()
        say(f"  max|gpu - fp32 reference| = {err:.3g}")
        assert err <= 1e-3
        return
    if precision == "mixed":
        w = D.weights_from_spyr(spyr8f8.read_file(WEIGHTS / artifact))
    else:
        w = D.weights_from_int8(torch.load(WEIGHTS / artifact, map_location="cpu", weights_only=True))
    ref = crop_output(D.forward(pad_frame(sub[None]), w, precision, out_dtype), SUB, SUB)[0][:, -k:, -k:]
    _check_quantized(f"{precision} frame {b}", got, ref)
