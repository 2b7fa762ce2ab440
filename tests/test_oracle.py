"""CPU checks that pin the oracle (the checker of the HIP runtime).

Each check is chosen so that a plausible mistake in the oracle -- a wrong
parity index, sign, tap order, transposed operand or rounding mode -- fails:
known-answer tables from the reference's own tests, closed forms, invariants,
brute force on tiny inputs, and golden vectors written by the reference model
(tests/golden/make_golden.py).
"""
from __future__ import annotations

import hashlib
import math

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import deploy as D
from oracle import model as M
from oracle import quant as Q
from oracle import spyr8f8
from tests._util import WEIGHTS, crop_output, golden, pad_frame, psnr


@pytest.fixture(scope="module", autouse=True)
def _threads():
    torch.set_num_threads(4)


@pytest.fixture(scope="module")
def area():
    return M.load_folded(WEIGHTS / "aeisu_area.pt")


# --- reconstruction pieces (aeisu/reconstruction.py) -----------------------------------------------
def test_coefficient_clamp_known_answers():
    # tests/test_reference.py:31-34
    v = torch.tensor([-20., -12., -4., -2., 0., 2., 4., 12., 20.])
    expected = torch.tensor([-2.5, -2.5, -2.1, -2., 0., 2., 2.1, 2.5, 2.5])
    torch.testing.assert_close(M.coefficient_clamp(v), expected)


def test_parity_packing_closed_form():
    # tests/test_reference.py:36-45: coefficient k of LR pixel (y, x) = channel 16*(2*(y%2)+x%2)+k
    meta = torch.empty(1, 64, 2, 3)
    for parity in range(4):
        for k in range(16):
            meta[:, parity * 16 + k] = parity * .1 + k * .001
    coeff = M.unpack_coefficients(meta)
    for y in range(4):
        for x in range(6):
            expected = torch.arange(16) * .001 + (2 * (y % 2) + x % 2) * .1
            torch.testing.assert_close(coeff[0, :, y, x], expected)


def test_basis_projection_invariants():
    raw = torch.randn(16, 4, 25, generator=torch.Generator().manual_seed(17))
    basis = M.project_basis(raw)
    assert basis.shape == (25, 16, 4)
    torch.testing.assert_close(basis.sum(0), torch.zeros(16, 4), atol=5e-8, rtol=0)
    assert float(basis.abs().sum(0).max()) <= 0.5000002
    torch.testing.assert_close(M.project_basis(torch.zeros_like(raw)), torch.zeros(25, 16, 4))
    # the layout is [tap, component, phase]: component 3 phase 2 is raw[3, 2] centred and scaled
    c = raw[3, 2] - raw[3, 2].mean()
    torch.testing.assert_close(basis[:, 3, 2], c * 0.5 / c.abs().sum())


def test_zero_coefficients_with_bilinear_base_is_bilinear_upsampling():
    # tests/test_reference.py:56-61
    src = torch.rand(1, 3, 12, 16, generator=torch.Generator().manual_seed(3))
    meta = torch.zeros(1, 64, 6, 8)
    out = M.reconstruct(src, meta, M.exact_bilinear_base(), torch.randn(25, 16, 4))
    expected = F.interpolate(src, scale_factor=2, mode="bilinear", align_corners=False)
    torch.testing.assert_close(out, expected, atol=3e-7, rtol=0)


def test_flat_field_invariant(area):
    # the bank has zero DC, so a constant image gives c * sum(base) whatever the coefficients
    src = torch.full((1, 3, 8, 12), 0.37)
    meta = torch.randn(1, 64, 4, 6, generator=torch.Generator().manual_seed(5)) * 3
    out = M.reconstruct(src, meta, area["base"], area["basis"])
    for ph in range(4):
        expected = 0.37 * float(area["base"][:, ph].sum())
        torch.testing.assert_close(out[:, :, ph >> 1::2, ph & 1::2], torch.full_like(out[:, :, ::2, ::2], expected),
                                   atol=2e-6, rtol=0)


def test_reconstruct_brute_force():
    g = torch.Generator().manual_seed(9)
    h, w = 6, 8
    src = torch.rand(1, 3, h, w, generator=g, dtype=torch.float64)
    meta = torch.randn(1, 64, h // 2, w // 2, generator=g, dtype=torch.float64) * 2
    base = torch.randn(25, 4, generator=g, dtype=torch.float64) * .1
    basis = torch.randn(25, 16, 4, generator=g, dtype=torch.float64) * .1
    out = M.reconstruct(src, meta, base, basis)
    s, mt = src.numpy()[0], meta.numpy()[0]
    for y in range(h):
        for x in range(w):
            rho = 2 * (y % 2) + (x % 2)
            a = [mt[16 * rho + k, y // 2, x // 2] for k in range(16)]
            a = [t if abs(t) <= 2 else math.copysign(min(2.5, 2 + .05 * (abs(t) - 2)), t) for t in a]
            for ph in range(4):
                for c in range(3):
                    acc = 0.0
                    for t in range(25):
                        wgt = float(base[t, ph]) + sum(a[k] * float(basis[t, k, ph]) for k in range(16))
                        yy = min(max(y + t // 5 - 2, 0), h - 1)
                        xx = min(max(x + t % 5 - 2, 0), w - 1)
                        acc += wgt * s[c, yy, xx]
                    assert abs(acc - float(out[0, c, 2 * y + ph // 2, 2 * x + ph % 2])) < 1e-9


def test_exact_bilinear_base_values():
    b = M.exact_bilinear_base()
    assert torch.allclose(b.sum(0), torch.ones(4))
    # TL phase: taps (1,1)=1/16, (1,2)=3/16, (2,1)=3/16, (2,2)=9/16  (aeisu/model.py:180-184)
    assert b[6, 0] == 1 / 16 and b[7, 0] == 3 / 16 and b[11, 0] == 3 / 16 and b[12, 0] == 9 / 16
    assert b[18, 3] == 1 / 16 and b[12, 3] == 9 / 16


def test_pad_geometry_matches_reference_formula():
    for h in (1, 31, 32, 33, 69, 1080, 1440):
        ey = -h % 32
        top, bottom, _, _ = M.pad_geometry(h, h)
        assert top == 16 + ey // 2 and top + bottom == 32 + ey and (h + top + bottom) % 32 == 0


# --- golden vectors from the reference's own model --------------------------------------------------
@pytest.mark.parametrize("tag,ckpt", [("area", "aeisu_area.pt"), ("div2k", "aeisu_div2k_l1.pt")])
def test_golden_vectors(tag, ckpt):
    from aeisu_amd import frames
    g = golden(tag)
    state = M.load_folded(WEIGHTS / ckpt)
    src = torch.from_numpy(g["small_input"])
    torch.testing.assert_close(M.upscale(state, src, 0), torch.from_numpy(g["small_tile0"]), atol=1e-6, rtol=0)
    torch.testing.assert_close(M.upscale(state, src, 32), torch.from_numpy(g["small_tile32"]), atol=1e-6, rtol=0)
    meta = M.controller(pad_frame(src[None]), state)
    torch.testing.assert_close(meta, torch.from_numpy(g["small_meta"]), atol=1e-6, rtol=0)
    src2 = torch.from_numpy(g["tiling_input"])
    torch.testing.assert_close(M.upscale(state, src2, 32), torch.from_numpy(g["tiling_tile32"]), atol=1e-6, rtol=0)
    src0 = frames.scene(256, 256, 0)
    assert hashlib.sha256(src0.numpy().tobytes()).hexdigest() == str(g["cfg0_input_sha256"])
    y0 = M.upscale(state, src0, 0)
    for name in ("top_left", "centre", "bottom_right", "right_edge"):
        r, c = g[f"cfg0_crop_{name}_origin"]
        torch.testing.assert_close(y0[:, r:r + 64, c:c + 64], torch.from_numpy(g[f"cfg0_crop_{name}"]), atol=1e-6, rtol=0)


def test_tiling_equals_whole(area):
    src = torch.from_numpy(golden("area")["tiling_input"])
    torch.testing.assert_close(M.upscale(area, src, 32), M.upscale(area, src, 0), atol=2e-6, rtol=2e-6)


def test_upscale_errors(area):
    with pytest.raises(ValueError):
        M.upscale(area, torch.rand(1, 8, 8), 0)
    with pytest.raises(ValueError):
        M.upscale(area, torch.rand(3, 8, 8), 48)
    bad = torch.rand(3, 8, 8)
    bad[1, 2, 3] = float("nan")
    with pytest.raises(FloatingPointError):
        M.upscale(area, bad, 0)


# --- planted mistakes must be caught ----------------------------------------------------------------
def test_planted_parity_mistake_is_caught(area):
    g = golden("area")
    src = torch.from_numpy(g["small_input"])
    padded = pad_frame(src[None])
    meta = torch.from_numpy(g["small_meta"])
    good = crop_output(M.reconstruct(padded, meta, area["base"], area["basis"]).clamp(0, 1), 40, 56)[0]
    torch.testing.assert_close(good, torch.from_numpy(g["small_tile0"]), atol=1e-6, rtol=0)
    swapped = meta.reshape(1, 4, 16, *meta.shape[-2:])[:, [0, 2, 1, 3]].reshape(meta.shape)   # rho index transposed
    bad = crop_output(M.reconstruct(padded, swapped, area["base"], area["basis"]).clamp(0, 1), 40, 56)[0]
    assert (bad - torch.from_numpy(g["small_tile0"])).abs().max() > 1e-3


def test_planted_stencil_sign_mistake_is_caught(area):
    g = golden("area")
    state = dict(area)
    state["analysis_diag135"] = -area["analysis_diag135"]
    meta = M.controller(pad_frame(torch.from_numpy(g["small_input"])[None]), state)
    assert (meta - torch.from_numpy(g["small_meta"])).abs().max() > 1e-3


# --- number formats ---------------------------------------------------------------------------------
def test_e4m3_table_and_round_trip():
    t = Q.e4m3_decode_table()
    assert t[0x7E] == 448 and np.isnan(t[0x7F]) and np.isnan(t[0xFF]) and t[0x01] == 2.0 ** -9
    assert t[0x08] == 2.0 ** -6 and t[0x38] == 1.0
    finite = [c for c in range(256) if (c & 0x7F) != 0x7F]
    codes = Q.e4m3_encode(t[finite])
    # +0/-0 both decode to zero; every other code round-trips exactly
    assert all(int(a) == b or (t[b] == 0 and t[int(a)] == 0) for a, b in zip(codes, finite))


def test_e4m3_ties_to_even_and_saturation():
    t = Q.e4m3_decode_table()
    pos = t[:0x7F]
    mids = (pos[:-1] + pos[1:]) / 2
    got = Q.e4m3_encode(mids.astype(np.float32))
    lo = np.arange(0, 0x7E)
    expected = np.where(lo % 2 == 0, lo, lo + 1)               # ties land on the even code
    assert np.array_equal(got.astype(int), expected)
    assert Q.e4m3_round(np.float32([449, 500, 1e6, -1e6])).tolist() == [448, 448, 448, -448]
    # agrees with torch's cast wherever torch does not overflow
    x = np.random.default_rng(0).uniform(-440, 440, 5000).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(Q.e4m3_round(x), ref)


def test_quantize_s8_rounding():
    v = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, 200.0, -200.0, 126.6])
    assert Q.quantize_s8(v, 1.0).tolist() == [0, 2, 2, -0, -2, 127, -127, 127]


# --- artifacts (reference SPYR8F8 and .pt): Appendix-B identities ------------------------------------
@pytest.mark.parametrize("pt,binf", [("aeisu_area.pt", "aeisu_area_mixed_fp8.bin"),
                                     ("aeisu_div2k_l1.pt", "aeisu_div2k_l1_mixed_fp8.bin")])
def test_fp8_artifact_matches_checkpoint(pt, binf):
    state = M.load_folded(WEIGHTS / pt)
    art = spyr8f8.read_file(WEIGHTS / binf)
    t = art["tensors"]
    assert art["architecture"] == "aif16x5_learnedrgb4dir8_s32_parallel32x4_learnedbase_oc25_v1"
    assert np.array_equal(t["project.weight_fp16"], state["project_540.weight"].half().numpy())
    bott0 = torch.cat((state["bottleneck_270_a1.weight"], state["bottleneck_270_b1.weight"]))
    assert np.array_equal(t["bottleneck0.weight_fp16"], bott0.half().numpy())
    assert np.array_equal(t["tail.weight_fp16"], state["metadata_head.weight"].half().numpy())
    assert np.array_equal(t["refine.bias"], state["refine_540.bias"].numpy())
    assert np.array_equal(t["adaptive_base"], state["base_kernel"].numpy())
    assert np.abs(t["adaptive_basis"] - state["basis"].numpy()).max() < 5e-8
    stencil = np.concatenate([state[k].reshape(-1).numpy() for k in M.ANALYSIS_KEYS])
    assert np.array_equal(t["analysis_stencil"], stencil)
    for layer, src in (("compress", "compress_270.weight"), ("expand", "expand_270.weight")):
        deq = Q.e4m3_decode(t[layer + ".weight_fp8"]) * t[layer + ".weight_scale"].reshape(-1, 1, 1, 1)
        w = state[src].numpy()
        step = t[layer + ".weight_scale"].reshape(-1, 1, 1, 1) * 32          # 1/16 relative at 448 codes max
        assert np.all(np.abs(deq - w) <= np.maximum(step, np.abs(w) / 15))


def test_int8_scales_are_fp8_scales_mapped():
    rec = torch.load(WEIGHTS / "aeisu_int8_fp16.pt", map_location="cpu", weights_only=True)
    fp8 = spyr8f8.read_file(WEIGHTS / "aeisu_area_mixed_fp8.bin")["tensors"]["activation_scales"]
    np.testing.assert_allclose(np.asarray(rec["activation_scales"], np.float64), fp8 * 448 / 127, rtol=1e-6)


# --- precision policies (CPU emulation) -------------------------------------------------------------
def test_fp16_policy_within_1e3_on_scene_frames(area):
    from aeisu_amd import frames
    w = D.weights_from_folded(area)
    for seed in (31, 7):
        src = frames.scene(96, 160, seed, shapes=6, texture=True).half()
        pad = pad_frame(src[None].float())
        ref = M.forward(pad, area).clamp(0, 1)
        out = D.forward(pad, w, "fp16", out_dtype=torch.float16)
        assert (out - ref).abs().max().item() <= 1e-3


def test_mixed_and_int8_policies_pass_the_native_gate(area):
    from aeisu_amd import frames
    src = frames.scene(96, 160, 31, shapes=6, texture=True).half()
    pad = pad_frame(src[None].float())
    ref = M.forward(pad, area).clamp(0, 1)
    mixed = D.forward(pad, D.weights_from_spyr(spyr8f8.read_file(WEIGHTS / "aeisu_area_mixed_fp8.bin")), "mixed")
    int8 = D.forward(pad, D.weights_from_int8(torch.load(WEIGHTS / "aeisu_int8_fp16.pt", weights_only=True)), "int8")
    assert psnr(mixed, ref) >= 50 and psnr(int8, ref) >= 45     # native gate is 35 dB (SrcPyrRuntimeTest.cpp:454-457)
