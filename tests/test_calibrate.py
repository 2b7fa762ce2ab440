"""SPYR8F8 writer and FP8 calibration (CPU parts).

Pinned against the reference's own data: its two Mixed artifacts (byte-exact
re-serialisation) and the calibration record of the DIV2K-L1 artifact
(tests/golden/div2k_calibration_record.json, made by make_calibration_golden.py).
The activation-scale search needs the GPU runtime and is tested in
test_gpu_calibrate.py.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from aeisu_amd import artifacts as A
from aeisu_amd import calibrate as C
from aeisu_amd import fp8
from oracle import model as M
from oracle import quant as Q
from oracle import spyr8f8
from tests._util import GOLDEN, WEIGHTS, pad_frame


def test_fp8_codec_matches_oracle():
    halves = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    with np.errstate(all="ignore"):
        assert np.array_equal(fp8.encode(halves), Q.e4m3_encode(halves))
    rng = np.random.default_rng(3)
    for scale in (1e-4, 1e-2, 1.0, 40.0, 1e5):
        x = (rng.standard_normal(200_000) * scale).astype(np.float32)
        assert np.array_equal(fp8.encode(x), Q.e4m3_encode(x))
    finite = ~np.isnan(fp8.DECODE)
    assert np.array_equal(fp8.DECODE[finite], Q.e4m3_decode_table()[finite])
    assert fp8.encode(np.float32([np.inf, -np.inf, 1e9])).tolist() == [0x7E, 0xFE, 0x7E]   # SATFINITE


@pytest.mark.parametrize("name", ["aeisu_area_mixed_fp8.bin", "aeisu_div2k_l1_mixed_fp8.bin"])
def test_writer_reproduces_reference_artifacts(name):
    """read_records + write re-serialise the reference's files byte for byte (layout, padding, SHA-256)."""
    blob = (WEIGHTS / name).read_bytes()
    records, header = A.read_records(blob)
    assert A.write(records, **header) == blob


def test_writer_output_reads_back():
    recs = [("activation_scales", A.DT_F32, A.LAYOUT_VECTOR, np.arange(10, dtype=np.float32) + 1),
            ("x.weight_fp8", A.DT_E4M3, A.LAYOUT_OIHW, np.arange(24, dtype=np.uint8).reshape(2, 3, 2, 2))]
    blob = A.write(recs)
    assert len(blob) % 64 == 0
    got = spyr8f8.read(blob)["tensors"]                 # independent reader (checks SHA-256, layout)
    assert np.array_equal(got["activation_scales"], recs[0][3])
    assert np.array_equal(got["x.weight_fp8"], recs[1][3])


@pytest.fixture(scope="module")
def div2k():
    rec = json.loads((GOLDEN / "div2k_calibration_record.json").read_text())
    state = M.load_folded(WEIGHTS / "aeisu_div2k_l1.pt")
    art = spyr8f8.read_file(WEIGHTS / "aeisu_div2k_l1_mixed_fp8.bin")["tensors"]
    return rec, C.layer_weights(state), art


def test_weight_quantization_reproduces_reference(div2k):
    """Percentile selection, LS-refined scale and E4M3 codes against the DIV2K artifact and its record."""
    rec, lw, art = div2k
    channels = same_pct = close_scale = 0
    codes_equal = codes_total = 0
    worst = 0.0
    for layer in A.LAYERS:
        codes, scales, recs = C.quantize_weight(lw[layer][0].numpy())
        ref_scales = art[layer + ".weight_scale"].astype(np.float64)
        for r, (pct, rec_scale) in zip(recs, rec["weights"][layer]):
            channels += 1
            same_pct += r["selected_percentile"] == pct
            # the record's scale is the initial percentile / 448 (before least squares)
            w = np.abs(lw[layer][0][r["output_channel"]].numpy().astype(np.float64).ravel())
            assert abs(np.percentile(w, pct) / 448 / rec_scale - 1) < 5e-5
            rel = abs(r["scale"] / ref_scales[r["output_channel"]] - 1)
            worst = max(worst, rel)
            close_scale += rel < 1e-5
        codes_equal += int((codes == art[layer + ".weight_fp8"]).sum())
        codes_total += codes.size
    assert same_pct == channels == 608
    assert close_scale >= 0.97 * channels, (close_scale, channels)
    assert worst < 2e-3
    assert codes_equal >= codes_total - 16, (codes_equal, codes_total)


@pytest.mark.parametrize("pt,binf", [("aeisu_area.pt", "aeisu_area_mixed_fp8.bin"),
                                     ("aeisu_div2k_l1.pt", "aeisu_div2k_l1_mixed_fp8.bin")])
def test_weight_codes_match_both_artifacts(pt, binf):
    """Calibrating each released checkpoint's weights gives (nearly) the shipped artifact's FP8 weights."""
    lw = C.layer_weights(M.load_folded(WEIGHTS / pt))
    art = spyr8f8.read_file(WEIGHTS / binf)["tensors"]
    equal = total = close = chans = 0
    for layer in A.LAYERS:
        codes, scales, _ = C.quantize_weight(lw[layer][0].numpy())
        equal += int((codes == art[layer + ".weight_fp8"]).sum())
        total += codes.size
        close += int((np.abs(scales / art[layer + ".weight_scale"] - 1) < 1e-5).sum())
        chans += scales.size
    assert equal >= total - 16 and close >= 0.97 * chans, (equal, total, close, chans)


def test_bias_correction_relation_and_formula(div2k):
    rec, lw, art = div2k
    for layer, corr in rec["fp8_bias_correction"].items():       # artifact: bias_fp8 = bias + correction
        d = art[layer + ".bias_fp8"].astype(np.float64) - art[layer + ".bias"].astype(np.float64)
        assert np.abs(d - np.asarray(corr)).max() < 5e-7
    # formula vs brute force on a grouped 3x3 conv: mean over an input field of (W - Q(W)) * x, away from borders
    g = torch.Generator().manual_seed(5)
    w = torch.randn(8, 4, 3, 3, generator=g)
    codes, scales, _ = C.quantize_weight(w.numpy())
    dq = torch.from_numpy(fp8.decode(codes) * scales.reshape(-1, 1, 1, 1))
    x = torch.rand(2, 8, 40, 40, generator=g) + torch.linspace(0, 2, 8).view(1, 8, 1, 1)
    err = F.conv2d(x, (w - dq).float(), groups=2).mean(dim=(0, 2, 3)).double().numpy()
    got = C.bias_correction(w.numpy(), codes, scales, x.mean(dim=(0, 2, 3)).numpy(), groups=2)
    assert np.abs(got - err).max() < 2e-3 * np.abs(err).max() + 1e-6


def test_boundary_activations_match_oracle_controller():
    """The calibrator's FP32 statistics forward reproduces the oracle controller (tail of boundary 9)."""
    state = M.load_folded(WEIGHTS / "aeisu_area.pt")
    lw = C.layer_weights(state)
    blob = A.folded_to_fp16(torch.load(WEIGHTS / "aeisu_area.pt", map_location="cpu", weights_only=True))
    stencil = A.read_tensors(blob)["analysis_stencil"]
    from aeisu_amd import frames as FR
    src = FR.scene(48, 80, 9, shapes=5, texture=True)[None]
    acts = C.boundary_activations(lw, C._analysis_kernel(stencil), src)
    meta = F.conv2d(acts[9], *lw["tail"])
    ref = M.controller(pad_frame(src), state)
    assert (meta - ref).abs().max().item() < 2e-4 * ref.abs().max().item()
    assert [a.shape[1] for a in acts] == [32, 32, 64, 64, 64, 64, 64, 128, 32, 64]
