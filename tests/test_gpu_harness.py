"""The reference native runtime's own test case, run on the MI355X runtime.

The reference's runtime harness (optimized/native/src/neural/srcpyr/SrcPyrRuntimeTest.cpp) builds a
synthetic FP16 frame, r = x / (W - 1), g = y / (H - 1), b = ((17 x + 29 y) mod 97) / 96 (lines
314-326), runs it through the native engine's Fp8, Fp16 and Mixed precisions on the shipped
adaptive_fp8.bin, and fails on any non-finite output value or when PSNR(Fp8 vs Fp16) or
PSNR(Mixed vs Fp16) over the RGB values is below 35 dB (lines 415-457).  Its default frame is
64 x 48 (line 264); --width/--height run other sizes up to 8192 (lines 272-303).

Here the same frames go through the FP16, Mixed and FP8-MFMA policies (the E4M3-operand route, this
runtime's counterpart of the Fp8 precision) on the same artifact, under the same gate.  The blue
channel's sawtooth makes this a hard input: on the CPU oracle the Mixed emulation is 35.8 dB from the
FP16 emulation at 64 x 48 and the FP16 emulation 0.025 from the FP32 reference path, so the
runtime's policies are also held to their own oracles on the small frames: Mixed to its emulation
(2/255), the FP32 policy to the FP32 reference path (1e-3) and the FP16 policy to its emulation (2/255;
its distance from the FP32 path, which its FP16 weights set, is reported).
"""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import deploy as D
from oracle import model as M
from oracle import spyr8f8
from tests._util import WEIGHTS, crop_output, pad_frame, psnr

pytestmark = pytest.mark.gpu

ARTIFACT = WEIGHTS / "aeisu_area_mixed_fp8.bin"
GATE_DB = 35.0                                  # SrcPyrRuntimeTest.cpp:268, 454-457


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def harness_frame(w: int, h: int) -> torch.Tensor:
    """[3, h, w] FP16: the harness's synthetic input (SrcPyrRuntimeTest.cpp:314-326)."""
    y = torch.arange(h, dtype=torch.float64)[:, None].expand(h, w)
    x = torch.arange(w, dtype=torch.float64)[None, :].expand(h, w)
    r = x / max(1, w - 1)
    g = y / max(1, h - 1)
    b = torch.remainder(17 * x + 29 * y, 97) / 96.0
    return torch.stack([r, g, b]).float().half()


@pytest.fixture(scope="module")
def models(gpu):
    torch.set_num_threads(16)
    from aeisu_amd import runtime
    out = {p: runtime.load_model(ARTIFACT, precision=p) for p in ("fp16", "mixed", "mixed-fp8mma")}
    yield out
    for m in out.values():
        m.close()


@pytest.mark.parametrize("w,h", [(64, 48), (33, 17), (1920, 1080)])
def test_reference_harness_gate(models, w, h):
    say(f"case: reference harness frame {w}x{h}, FP16 / Mixed / FP8-MFMA policies")
    src = harness_frame(w, h)[None].cuda().contiguous()
    # run() checks the non-finite flag of every frame (the harness's "Non-finite output")
    outs = {p: m.run(src).float().cpu() for p, m in models.items()}
    for p, o in outs.items():
        assert o.shape == (1, 3, 2 * h, 2 * w) and torch.isfinite(o).all(), p
    p_mixed = psnr(outs["mixed"], outs["fp16"])
    p_fp8 = psnr(outs["mixed-fp8mma"], outs["fp16"])
    say(f"  PSNR vs the FP16 policy: Mixed {p_mixed:.2f} dB, FP8-MFMA {p_fp8:.2f} dB (gate {GATE_DB} dB)")
    assert p_mixed >= GATE_DB and p_fp8 >= GATE_DB


@pytest.mark.parametrize("w,h", [(64, 48), (33, 17)])
def test_reference_harness_frame_vs_oracles(models, w, h):
    from aeisu_amd import runtime
    say(f"case: reference harness frame {w}x{h} against the Mixed emulation and the FP32 reference path")
    frame = harness_frame(w, h)
    src = frame[None].cuda().contiguous()
    got = models["mixed"].run(src).float().cpu()[0]
    wts = D.weights_from_spyr(spyr8f8.read_file(ARTIFACT))
    emu = crop_output(D.forward(pad_frame(frame[None].float()), wts, "mixed"), h, w)[0]
    err = (got - emu).abs().max().item()
    say(f"  Mixed: max|gpu - emulation| = {err * 255:.3f}/255")
    assert err <= 2 / 255
    fp32 = runtime.load_model(WEIGHTS / "aeisu_area.pt", precision="fp32")
    try:
        got32 = fp32.run(src.float()).cpu()[0]
    finally:
        fp32.close()
    ref = M.upscale(M.load_folded(WEIGHTS / "aeisu_area.pt"), frame.float(), 0)
    err32 = (got32 - ref).abs().max().item()
    say(f"  FP32 policy: max|gpu - fp32 reference| = {err32:.3g}")
    assert err32 <= 1e-3
    # The FP16 policy runs FP16 weights and stores every activation in FP16, as the reference's FP16
    # engine does.  On this sawtooth its distance from the FP32 path is that of its emulation: 0.025
    # at 64 x 48 on adaptive_fp8.bin, whose project weights are FP16 only, and 0.007 on the folded
    # checkpoint, whose FP32 project weights the policy uses (FP16 weights and activations elsewhere),
    # against 4-6e-4 on natural frames.  Reported, and held to the emulation of the same weights
    # within 2/255 (measured 1.2e-3: the FP32-sum rounding of the GPU's layers, spread by this input).
    fp16pt = runtime.load_model(WEIGHTS / "aeisu_area.pt", precision="fp16")
    try:
        cases = [("adaptive_fp8.bin", models["fp16"], wts),
                 ("aeisu_area.pt", fp16pt, D.weights_from_folded(M.load_folded(WEIGHTS / "aeisu_area.pt")))]
        for name, model, wq in cases:
            got16 = model.run(src, out_dtype=torch.float32).cpu()[0]
            emu16 = crop_output(D.forward(pad_frame(frame[None].float()), wq, "fp16", torch.float32), h, w)[0]
            say(f"  FP16 policy, {name}: max|gpu - fp32 reference| = {(got16 - ref).abs().max().item():.3g}, "
                f"max|gpu - fp16 emulation| = {(got16 - emu16).abs().max().item():.3g}, "
                f"max|fp16 emulation - fp32 reference| = {(emu16 - ref).abs().max().item():.3g}")
            assert (got16 - emu16).abs().max().item() <= 2 / 255
    finally:
        fp16pt.close()
