"""CPU checks that pin the reduced-precision emulation (oracle/deploy.py).

The reference ships no Python for its FP8 / INT8 deployments, so the emulation
is pinned three ways, each chosen so that a plausible mistake fails:

1. Rounding points, against a brute-force restatement in exact rational
   arithmetic (``fractions.Fraction`` rounded to nearest even at the stated
   precision) on inputs built to expose them: the FP32 MMA chain over K=32
   chunks in the reference's order, the K=16 chains of the FP16 layers
   (project, refine, tail) with their FP32 bias add, slope and FP16 store, the ``fmaf`` epilogues, the FP16 tail bias,
   the FMA-contracted expand residual, saturating E4M3 and INT8 requantization.
2. Every FP8 and INT8 layer against the FP32 checkpoint's layer applied to the
   same dequantized input: each output lies within the weight-quantization
   error + bias correction + half an output quantum (+ saturation), and the
   layer's least-squares slope against the float64 layer on the dequantized
   weights is 1 within 0.3 %.  Inputs and outputs are
   decoded with this file's own activation-scale table, taken from the
   reference's launch sites, not with the emulation's.
3. The bias correction: ``bias_fp8 - bias`` is the exporter's recorded
   correction (DIV2K, tests/test_calibrate.py), and running with ``bias_fp8``
   brings the output closer to the FP32 model than ``bias`` does on the input
   class each model was calibrated for.

``test_planted_*`` plant the mistakes a restatement is likely to make in the
oracle (``bias`` for ``bias_fp8``, an off-by-one activation-scale index, an
unrounded tail bias, a split multiply-add in the expand residual, float64 sums
instead of chunked FP32 accumulation, phase-major compress chunks, one rounding
of an FP16 layer's whole sum, interleaved FP16 chunks, column-major refine
taps) and assert
that the corresponding check fails.
"""
from __future__ import annotations

from fractions import Fraction as Fr

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import deploy as D
from oracle import model as M
from oracle import quant as Q
from oracle import spyr8f8
from tests._util import WEIGHTS, pad_frame, psnr

# Activation-scale indices (input, output) of each quantized layer, from the reference's launch
# sites: compress 1/s1 in, 1/s2 out (SrcPyrCudaRuntime.cu:4397-4408); bottleneck b: s(b+2) in,
# 1/s(b+3) out (4427-4436); expand s6 in, 1/s7 out and s7 for the residual (4587-4601); the INT8
# runtime uses the same boundaries (optimized/shader/runtime.py:60-76: compress scales[1], [2];
# pairs scales[index+1], [index+2]; expand scales[6], [7]).
REF_SCALES = {"compress": (1, 2), "bottleneck0": (2, 3), "bottleneck1": (3, 4), "bottleneck2": (4, 5),
              "bottleneck3": (5, 6), "expand": (6, 7)}


@pytest.fixture(scope="module", autouse=True)
def _threads():
    torch.set_num_threads(4)


@pytest.fixture(scope="module")
def area_mixed():
    return D.weights_from_spyr(spyr8f8.read_file(WEIGHTS / "aeisu_area_mixed_fp8.bin"))


@pytest.fixture(scope="module")
def div2k_mixed():
    return D.weights_from_spyr(spyr8f8.read_file(WEIGHTS / "aeisu_div2k_l1_mixed_fp8.bin"))


@pytest.fixture(scope="module")
def area_int8():
    return D.weights_from_int8(torch.load(WEIGHTS / "aeisu_int8_fp16.pt", map_location="cpu", weights_only=True))


# ------------------------------------------------------------------------------------------------
# exact rational arithmetic
# ------------------------------------------------------------------------------------------------
def rne(x: Fr, p: int, emin: int) -> Fr:
    """x rounded to nearest even with p significant bits, gradual underflow below 2^emin."""
    if x == 0:
        return Fr(0)
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fr(2) ** e > a:
        e -= 1
    q = Fr(2) ** (max(e, emin) - (p - 1))
    r = round(a / q) * q                     # Fraction.__round__ rounds half to even
    return r if x > 0 else -r


def r32(x: Fr) -> Fr:
    return rne(x, 24, -126)


def r16(x: Fr) -> Fr:
    return rne(x, 11, -14)


def e4m3(x: Fr) -> Fr:
    v = rne(x, 4, -6)
    return max(min(v, Fr(448)), Fr(-448))


def f(v) -> Fr:
    return Fr(float(v))


def rand_e4m3(rng, shape, lo_exp=-9, hi_exp=8) -> np.ndarray:
    """E4M3 values spread over a chosen exponent range (mixed magnitudes expose rounding)."""
    codes = rng.integers(0, 256, size=shape).astype(np.uint8)
    vals = Q.e4m3_decode(codes)
    vals = np.where(np.isnan(vals), 0.0, vals).astype(np.float32)
    keep = (np.abs(vals) >= 2.0 ** lo_exp) & (np.abs(vals) <= 2.0 ** hi_exp)
    return np.where(keep, vals, 0.0).astype(np.float32)


# ------------------------------------------------------------------------------------------------
# 1. rounding points
# ------------------------------------------------------------------------------------------------
def check_fmaf():
    rng = np.random.default_rng(1)
    n = 4000
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    b = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(np.float32)
    c = (rng.standard_normal(n) * np.exp2(rng.integers(-60, 30, n))).astype(np.float32)
    c[::7] = -(a[::7].astype(np.float64) * b[::7]).astype(np.float32)     # near-cancellation
    # a float64 sum that lands exactly on a float32 midpoint: (1+2^-12)^2 = 1 + 2^-11 + 2^-24,
    # plus 2^-80 lies just above it and must round up
    a = np.append(a, np.float32([1 + 2 ** -12, 1 + 2 ** -12, -(1 + 2 ** -12)]))
    b = np.append(b, np.float32([1 + 2 ** -12, 1 + 2 ** -12, 1 + 2 ** -12]))
    c = np.append(c, np.float32([2.0 ** -80, -2.0 ** -80, -2.0 ** -80]))
    got = Q.fmaf(torch.from_numpy(a), torch.from_numpy(b), torch.from_numpy(c)).numpy()
    for i in range(len(a)):
        want = r32(f(a[i]) * f(b[i]) + f(c[i]))
        assert Fr(float(got[i])) == want, (i, a[i], b[i], c[i])


def test_fmaf_single_rounding():
    check_fmaf()


def test_planted_double_rounding_fmaf_is_caught(monkeypatch):
    def double_rounded(a, b, c):
        a64, b64 = torch.as_tensor(a).double(), torch.as_tensor(b).double()
        return (a64 * b64 + torch.as_tensor(c).double()).float()
    monkeypatch.setattr(Q, "fmaf", double_rounded)
    with pytest.raises(AssertionError):
        check_fmaf()


def _brute_compress(x: np.ndarray, w: np.ndarray, pix) -> list:
    """Per output channel: chunks j of K indices 32j..32j+31 (K = c*4 + phase), acc <- r32(acc + sum)."""
    b, y, xx = pix
    out = []
    for o in range(w.shape[0]):
        acc = Fr(0)
        for j in range(w.shape[1] // 32):
            acc = r32(acc + sum(f(x[b, k, y, xx]) * f(w[o, k, 0, 0]) for k in range(32 * j, 32 * j + 32)))
        out.append(acc)
    return out


def _brute_grouped(x: np.ndarray, w: np.ndarray, pix) -> list:
    """Per output channel: 9 tap chunks in row-major (dy, dx) order over the group's 32 channels, zero pad."""
    b, y, xx = pix
    h, wd = x.shape[-2:]
    out = []
    for o in range(w.shape[0]):
        g = o // (w.shape[0] // 2)
        acc = Fr(0)
        for dy in range(3):
            for dx in range(3):
                yy, xs = y + dy - 1, xx + dx - 1
                if 0 <= yy < h and 0 <= xs < wd:
                    s = sum(f(x[b, 32 * g + c, yy, xs]) * f(w[o, c, dy, dx]) for c in range(32))
                else:
                    s = Fr(0)
                acc = r32(acc + s)
        out.append(acc)
    return out


def check_mma_chain():
    """D.mma_chain(D.chunk_sums(...)) equals the rational restatement of the reference's MMA chains,
    on inputs whose chunks mix magnitudes so that chunk order and composition change the result."""
    rng = np.random.default_rng(7)
    cases = []
    # compress 128 -> 8 outputs, expand 64 -> 8 outputs (1x1), one chunk per magnitude band
    for cin, layer in ((128, "compress"), (64, "expand")):
        x = rand_e4m3(rng, (1, cin, 3, 4))
        w = rand_e4m3(rng, (8, cin, 1, 1))
        for j in range(cin // 32):                 # alternate large and tiny chunks
            scale = 2.0 ** (6 if j % 2 == 0 else -7)
            x[:, 32 * j:32 * j + 32] = Q.e4m3_round(x[:, 32 * j:32 * j + 32] * scale)
        cases.append((layer, x, w))
    x = rand_e4m3(rng, (1, 64, 4, 5))
    w = rand_e4m3(rng, (8, 32, 3, 3))
    w[:, :, 1, :] = Q.e4m3_round(w[:, :, 1, :] * 2.0 ** 7)     # middle row taps large
    cases.append(("bottleneck0", x, w))
    mismatched_single_rounding = 0
    for layer, x, w in cases:
        xt, wt = torch.from_numpy(x), torch.from_numpy(w)
        got = D.mma_chain(D.chunk_sums(xt, wt, layer)).numpy()
        once = F.conv2d(xt.double(), wt.double(), padding=w.shape[-1] // 2,
                        groups=2 if layer.startswith("bottleneck") else 1).float().numpy()
        brute = _brute_grouped if layer.startswith("bottleneck") else _brute_compress
        for pix in [(0, yy, xx) for yy in range(x.shape[2]) for xx in range(x.shape[3])]:
            want = brute(x, w, pix)
            for o, v in enumerate(want):
                assert Fr(float(got[pix[0], o, pix[1], pix[2]])) == v, (layer, pix, o)
                mismatched_single_rounding += Fr(float(once[pix[0], o, pix[1], pix[2]])) != v
    # the inputs do exercise the chunking: one rounding of the exact total differs somewhere
    assert mismatched_single_rounding > 0


def test_mma_chain_matches_rational_restatement():
    check_mma_chain()


def test_planted_float64_accumulation_is_caught(monkeypatch):
    monkeypatch.setattr(D, "mma_chain", lambda parts: torch.stack(list(parts)).sum(0).float())
    with pytest.raises(AssertionError):
        check_mma_chain()


def test_planted_phase_major_compress_chunks_are_caught(monkeypatch):
    real = D.chunk_sums

    def phase_major(x, w, layer):
        if layer != "compress":
            return real(x, w, layer)
        x64, w64 = x.double(), w.double()
        return [F.conv2d(x64[:, ph::4], w64[:, ph::4]) for ph in range(4)]
    monkeypatch.setattr(D, "chunk_sums", phase_major)
    with pytest.raises(AssertionError):
        check_mma_chain()


def check_fp8_epilogue(w):
    """fmaf(acc, r32(s_in*ws), bias_fp8) -> leaky(prelu) -> e4m3(r32(v * r32(1/s_out))), every layer,
    with this file's scale table."""
    rng = np.random.default_rng(3)
    for layer in D.BODY:
        cout = w[layer + ".b8"].numel()
        acc = (rng.standard_normal((1, cout, 2, 3)) * np.exp2(rng.integers(-2, 12, (1, cout, 2, 3)))).astype(np.float32)
        got = D.fp8_epilogue(torch.from_numpy(acc), w, layer).numpy()
        si, so = REF_SCALES[layer]
        s_in, s_out = f(w["act"][si]), f(w["act"][so])
        inv = r32(1 / s_out)
        for c in range(cout):
            scale = r32(s_in * f(w[layer + ".ws"][c]))
            for yy in range(2):
                for xx in range(3):
                    v = r32(f(acc[0, c, yy, xx]) * scale + f(w[layer + ".b8"][c]))
                    if v < 0:
                        v = r32(v * f(w[layer + ".prelu"][c]))
                    assert Fr(float(got[0, c, yy, xx])) == e4m3(r32(v * inv)), (layer, c)


def test_fp8_epilogue_matches_rational_restatement(area_mixed, div2k_mixed):
    check_fp8_epilogue(area_mixed)
    check_fp8_epilogue(div2k_mixed)


def test_planted_scale_index_is_caught(monkeypatch, area_mixed):
    monkeypatch.setitem(D.SCALE_INDEX, "bottleneck1", (2, 4))      # act[i+2] in place of act[i+3] (input side)
    with pytest.raises(AssertionError):
        check_fp8_epilogue(area_mixed)


def check_expand_residual(w):
    """work = r16(r32(q * s7 + skip)) for E4M3 q, the artifact's s7 and FP16 skips.  Skips sized like
    the product make the product's FP32 rounding matter now and then; those cases (found by a
    vectorized float32 comparison of the split and contracted forms) and a random sample of the
    rest are checked in rational arithmetic."""
    rng = np.random.default_rng(11)
    s7 = np.float32(w["act"][REF_SCALES["expand"][1]])
    n = 1 << 20
    q = rand_e4m3(rng, n, -9, 8)
    skip = (q * s7 * rng.uniform(-2, 2, n)).astype(np.float16).astype(np.float32)
    # pixel_shuffle on [1, 4, 1, n/4]: output (i, 2*col + j) takes input channel 2i + j, column col
    qs = torch.from_numpy(q).view(1, 4, 1, n // 4)
    sk = torch.from_numpy(skip.reshape(4, n // 4)).view(2, 2, n // 4).permute(0, 2, 1).reshape(1, 1, 2, n // 2)
    got = D.expand_residual(qs, float(s7), sk).numpy()[0, 0].reshape(2, n // 4, 2).transpose(0, 2, 1).reshape(-1)
    split = ((q * s7).astype(np.float32) + skip).astype(np.float16).astype(np.float32)
    candidates = np.flatnonzero(split != got)
    sample = np.concatenate([candidates[:64], rng.choice(n, 256, replace=False)])
    differ = 0
    s7f = f(s7)
    for i in sample:
        want = r16(r32(f(q[i]) * s7f + f(skip[i])))
        differ += want != r16(r32(r32(f(q[i]) * s7f) + f(skip[i])))
        assert Fr(float(got[i])) == want, (i, q[i], skip[i])
    assert differ >= 8          # the sample contains cases where the contraction matters


def test_expand_residual_is_one_fma_then_fp16(area_mixed):
    check_expand_residual(area_mixed)


def test_planted_split_expand_residual_is_caught(monkeypatch, area_mixed):
    monkeypatch.setattr(D, "fmaf", lambda a, b, c: torch.as_tensor(a).float() * torch.as_tensor(b, dtype=torch.float32)
                        + torch.as_tensor(c).float())
    with pytest.raises(AssertionError):
        check_expand_residual(area_mixed)


def _fp16_inputs(rng, cin, h, wd, big_chunks):
    """FP16 activations whose K=16 chunks alternate between large and tiny magnitudes (chunk c large
    when c in big_chunks), random signs, a few FP16 subnormals and exact zeros."""
    x = rng.standard_normal((1, cin, h, wd))
    for c in range(cin // 16):
        x[:, 16 * c:16 * c + 16] *= 2.0 ** (6 if c in big_chunks else -7)
    x[rng.random(x.shape) < 0.03] = 0.0
    sub = rng.random(x.shape) < 0.02
    x[sub] = rng.integers(-1023, 1024, int(sub.sum())) * 2.0 ** -24
    return x.astype(np.float16).astype(np.float32)


def _brute_fp16_layer(x, w, pix, bias, slope, tail=False):
    """FP32 accumulators and FP16 outputs of one pixel of an FP16 layer in exact rational arithmetic:
    acc <- r32(acc + sum of a K=16 step) over the reference's steps (1x1: channels 16s..16s+15; 3x3:
    taps row-major, each channels 0-15 then 16-31), then r32(acc + bias) (tail: + r16(bias)), the
    slope for negative values, r16."""
    _, y, xx = pix
    cin, k = w.shape[1], w.shape[-1]
    taps = [(r, s) for r in range(k) for s in range(k)]
    accs, out = [], []
    for o in range(w.shape[0]):
        acc = Fr(0)
        for r, s in taps:
            yy, xs = y + r - k // 2, xx + s - k // 2
            for c0 in range(0, cin, 16):
                part = Fr(0)
                if 0 <= yy < x.shape[2] and 0 <= xs < x.shape[3]:
                    for c in range(c0, c0 + 16):
                        part += f(x[0, c, yy, xs]) * f(w[o, c, r, s])
                acc = r32(acc + part)
        accs.append(acc)
        if tail:
            out.append(r16(r32(acc + r16(f(bias[o])))))
            continue
        v = r32(acc + f(bias[o]))
        if v < 0:
            v = r32(v * f(np.float32(slope)))
        out.append(r16(v))
    return accs, out


def check_fp16_chain(w):
    """D.fp16_chain (the FP32 accumulator) and D.project / D.refine / D.tail (the FP16 layer) equal the
    rational restatement of the reference's K=16 MMA chains and epilogues (SrcPyrCudaRuntime.cu:2539-2547,
    2568-2583; SrcPyrNativeFp16Refine.cuh:425-475, 494-538), on inputs whose chunks mix magnitudes so
    that one rounding of the whole sum gives different accumulators somewhere."""
    rng = np.random.default_rng(11)
    single_differs = 0
    for layer, cin, h, wd, big in (("project", 32, 3, 5, {0}), ("project", 32, 2, 4, {1}),
                                   ("refine", 32, 3, 4, {0}), ("tail", 64, 2, 5, {0, 2})):
        x = _fp16_inputs(rng, cin, h, wd, big)
        xt = torch.from_numpy(x)
        wt = np.asarray(w[layer + ".w"], np.float32)
        fn = {"project": D.project, "refine": D.refine, "tail": D.tail}[layer]
        got = fn(xt, w).numpy()
        chain = D.fp16_chain(xt, w[layer + ".w"]).numpy()
        once = F.conv2d(xt.double(), w[layer + ".w"].double(), padding=wt.shape[-1] // 2).float().numpy()
        bias = np.asarray(w[layer + ".b"], np.float32)
        for pix in [(0, yy, xx) for yy in range(h) for xx in range(wd)]:
            accs, want = _brute_fp16_layer(x, wt, pix, bias, 0.1, tail=layer == "tail")
            for o, (a, v) in enumerate(zip(accs, want)):
                assert Fr(float(chain[0, o, pix[1], pix[2]])) == a, (layer, "acc", pix, o)
                assert Fr(float(got[0, o, pix[1], pix[2]])) == v, (layer, pix, o)
                single_differs += Fr(float(once[0, o, pix[1], pix[2]])) != a
    # the inputs do exercise the chunking: one rounding of the exact total differs somewhere
    assert single_differs > 0


def test_fp16_chain_matches_rational_restatement(area_mixed):
    check_fp16_chain(area_mixed)


def test_fp16_chain_is_exact_on_wide_products():
    """Steps whose products span more than float64's 53 bits (2^13 next to 2^-48) are still summed
    exactly: 2^13 + 2^-11 and 2^13 - 2^-12 are float32 midpoints and the 2^-48 products decide them."""
    x = np.zeros((1, 16, 1, 3), np.float32)
    wt = np.zeros((2, 16, 1, 1), np.float32)
    x[0, 0, 0, :] = 64.0
    wt[:, 0] = 128.0                                      # 2^13
    x[0, 1, 0, :] = [2.0 ** -24, -2.0 ** -24, 3 * 2.0 ** -24]
    wt[:, 1] = 2.0 ** -24                                  # +-2^-48, 3 * 2^-48
    x[0, 2, 0, :] = 2.0 ** -5
    wt[:, 2, 0, 0] = [2.0 ** -6, -2.0 ** -7]               # 2^13 + 2^-11, 2^13 - 2^-12: midpoints
    got = D.fp16_chain(torch.from_numpy(x), torch.from_numpy(wt)).numpy()
    broken = 0
    for p in range(3):
        for o in range(2):
            exact = sum((f(x[0, c, 0, p]) * f(wt[o, c, 0, 0]) for c in range(16)), Fr(0))
            assert Fr(float(got[0, o, 0, p])) == r32(exact), (p, o)
            broken += r32(exact) != r32(Fr(2) ** 13 + f(wt[o, 2, 0, 0]) * f(x[0, 2, 0, p]))
    assert broken > 0                                       # the tiny products do break ties


def test_planted_single_rounding_of_fp16_layers_is_caught(monkeypatch, area_mixed):
    monkeypatch.setattr(D, "fp16_chain", lambda x, w: D._conv64(x, w))
    with pytest.raises(AssertionError):
        check_fp16_chain(area_mixed)


def test_planted_interleaved_fp16_chunks_are_caught(monkeypatch, area_mixed):
    real = D.fp16_steps

    def interleaved(x, w):
        if w.shape[-1] != 1:
            return real(x, w)
        n = x.shape[1] // 16
        return [(x[:, c::n], w[:, c::n]) for c in range(n)]
    monkeypatch.setattr(D, "fp16_steps", interleaved)
    with pytest.raises(AssertionError):
        check_fp16_chain(area_mixed)


def test_planted_column_major_refine_taps_are_caught(monkeypatch, area_mixed):
    real = D.fp16_steps

    def column_major(x, w):
        if w.shape[-1] != 3:
            return real(x, w)
        h, wd = x.shape[-2:]
        xp = F.pad(x, (1, 1, 1, 1))
        return [(xp[:, c:c + 16, r:r + h, s:s + wd], w[:, c:c + 16, r:r + 1, s:s + 1])
                for s in range(3) for r in range(3) for c in (0, 16)]
    monkeypatch.setattr(D, "fp16_steps", column_major)
    with pytest.raises(AssertionError):
        check_fp16_chain(area_mixed)


def check_tail(w):
    """meta = r16(r32(r32(sum) + r16(bias))): FP16 tail bias added to the FP32 accumulator
    (SrcPyrNativeFp16Refine.cuh:494-538, bias rounded on the host SrcPyrCudaRuntime.cu:2999-3006).
    One non-zero input channel per pixel makes the sum one exact product."""
    rng = np.random.default_rng(5)
    n = 512
    dec = np.zeros((1, 64, 1, n), np.float32)
    vals = (rng.standard_normal(n) * np.exp2(rng.integers(-6, 6, n))).astype(np.float16).astype(np.float32)
    chans = rng.integers(0, 64, n)
    dec[0, chans, 0, np.arange(n)] = vals
    wt = dict(w)
    got = D.tail(torch.from_numpy(dec), wt).numpy()
    bias = np.asarray(wt["tail.b"], np.float32)
    weight = np.asarray(wt["tail.w"], np.float32)[:, :, 0, 0]
    differ = 0
    for p in range(n):
        for o in range(64):
            s = r32(f(vals[p]) * f(weight[o, chans[p]]))
            want = r16(r32(s + r16(f(bias[o]))))
            differ += want != r16(r32(s + f(bias[o])))
            assert Fr(float(got[0, o, 0, p])) == want, (p, o)
    assert differ > 0


def test_tail_adds_fp16_rounded_bias(area_mixed):
    check_tail(area_mixed)


def test_planted_unrounded_tail_bias_is_caught(monkeypatch, area_mixed):
    monkeypatch.setattr(D, "tail", lambda dec, w: Q.f16(D._conv64(dec, w["tail.w"]) + D._chan(w["tail.b"])))
    with pytest.raises(AssertionError):
        check_tail(area_mixed)


def check_int8_stages(w):
    """quantize_s8 input, fmaf(acc, factor, bias) -> v*fl32(0.1) -> clamp(rint(r32(v * r32(1/s_out))))."""
    rng = np.random.default_rng(9)
    skip = torch.from_numpy((rng.standard_normal((1, 32, 4, 4)) * 0.5).astype(np.float16).astype(np.float32))
    got_in = D.int8_input(skip, w).numpy()
    inv1 = r32(1 / f(w["act"][REF_SCALES["compress"][0]]))
    x = F.pixel_unshuffle(skip, 2).numpy()
    for idx in np.ndindex(x.shape):
        t = r32(f(x[idx]) * inv1)
        assert got_in[idx] == max(-127, min(127, round(t)))
    for layer in D.BODY:
        cout = w[layer + ".b"].numel()
        acc = rng.integers(-40000, 40000, (1, cout, 1, 4)).astype(np.float32)
        got = D.int8_epilogue(torch.from_numpy(acc), w, layer).numpy()
        inv = r32(1 / f(w["act"][REF_SCALES[layer][1]]))
        for c in range(cout):
            for k in range(4):
                v = r32(f(acc[0, c, 0, k]) * f(w[layer + ".factor"][c]) + f(w[layer + ".b"][c]))
                if v < 0:
                    v = r32(v * f(np.float32(0.1)))
                assert got[0, c, 0, k] == max(-127, min(127, round(r32(v * inv)))), (layer, c)


def test_int8_stages_match_rational_restatement(area_int8):
    check_int8_stages(area_int8)


def test_planted_int8_scale_index_is_caught(monkeypatch, area_int8):
    monkeypatch.setitem(D.SCALE_INDEX, "bottleneck2", (4, 4))       # output side off by one
    with pytest.raises(AssertionError):
        check_int8_stages(area_int8)


# ------------------------------------------------------------------------------------------------
# 2. layers against the FP32 checkpoint
# ------------------------------------------------------------------------------------------------
def check_layer_bounds(w, state, src, precision):
    """Each quantized layer of the emulation, decoded with REF_SCALES, against leaky(W32 x + b32) on the
    same dequantized input x:  |y - y32| <= |(W_q - W32) x + (b_q - b32)| + half an output quantum
    + saturation excess, elementwise; and the least-squares slope of y on the float64 layer with
    the dequantized weights (all channels pooled) is 1 within 0.3 %."""
    rec = {}
    D.controller(src, w, precision, rec)
    act = w["act"].double()
    layers32 = D.fp32_layers(state)
    ins = [rec["compress_in"], rec["low0"], rec["low1"], rec["low2"], rec["low3"], rec["low4"]]
    outs = [rec["low0"], rec["low1"], rec["low2"], rec["low3"], rec["low4"], rec["expand_out"]]
    for li, layer in enumerate(D.BODY):
        si, so = REF_SCALES[layer]
        s_in, s_out = float(act[si]), float(act[so])
        x, y = ins[li].double() * s_in, outs[li].double() * s_out
        w32, b32 = layers32[layer]["w"].double(), layers32[layer]["b"].double()
        groups = 2 if layer.startswith("bottleneck") else 1
        pad = w32.shape[-1] // 2
        pre32 = F.conv2d(x, w32, padding=pad, groups=groups) + b32.view(1, -1, 1, 1)
        y32 = torch.where(pre32 >= 0, pre32, 0.1 * pre32)
        if precision == "mixed":
            wq = w[layer + ".w8"].double() * w[layer + ".ws"].double().view(-1, 1, 1, 1)
            bq, qmax = w[layer + ".b8"].double(), 448.0
            mag = torch.maximum(y.abs(), y32.abs())
            half_q = torch.maximum(mag * 2.0 ** -4, torch.full_like(mag, 2.0 ** -10 * s_out))
        else:
            wq = w[layer + ".wq"].double() * (w[layer + ".factor"].double() / s_in).view(-1, 1, 1, 1)
            bq, qmax = w[layer + ".b"].double(), 127.0
            half_q = torch.full_like(y, 0.5 * s_out)
        dev = F.conv2d(x, wq - w32, padding=pad, groups=groups) + (bq - b32).view(1, -1, 1, 1)
        sat = torch.clamp(y32.abs() - qmax * s_out, min=0)
        bound = dev.abs() + half_q + sat + 1e-6 * y32.abs() + 1e-12
        err = (y - y32).abs()
        bad = int((err > bound).sum())
        assert bad == 0, f"{layer}: {bad} outputs outside the quantization bound (max ratio {(err / bound).max():.3f})"
        # scale consistency: against the same layer in float64 on the artifact's dequantized weights,
        # only the (unbiased, round-to-nearest) output quantization remains, so each channel's
        # least-squares slope is 1 to well under the 0.9 % that separates the closest pair of scales
        preq = F.conv2d(x, wq, padding=pad, groups=groups) + bq.view(1, -1, 1, 1)
        yq = torch.where(preq >= 0, preq, 0.1 * preq).clamp(-qmax * s_out, qmax * s_out)
        slope = float((y * yq).sum() / (yq * yq).sum())
        assert abs(slope - 1) < 0.003, f"{layer}: layer slope {slope:.5f}"


def _frames(kind, seeds, h=192, w=288):
    from aeisu_amd import frames
    for s in seeds:
        img = frames.pink_noise(h, w, s) if kind == "pink" else frames.scene(h, w, s, texture=True)
        yield pad_frame(img.half()[None].float())


@pytest.mark.parametrize("tag", ["area-mixed", "div2k-mixed", "area-int8"])
def test_layers_within_quantization_bound_of_fp32_checkpoint(tag, area_mixed, div2k_mixed, area_int8):
    w = {"area-mixed": area_mixed, "div2k-mixed": div2k_mixed, "area-int8": area_int8}[tag]
    state = M.load_folded(WEIGHTS / ("aeisu_div2k_l1.pt" if tag.startswith("div2k") else "aeisu_area.pt"))
    for src in _frames("pink" if tag.startswith("div2k") else "scene", (31,)):
        check_layer_bounds(w, state, src, "int8" if tag.endswith("int8") else "mixed")


def test_planted_output_scale_index_is_caught(monkeypatch, area_mixed):
    monkeypatch.setitem(D.SCALE_INDEX, "bottleneck3", (5, 5))      # act[i+2] in place of act[i+3]
    state = M.load_folded(WEIGHTS / "aeisu_area.pt")
    with pytest.raises(AssertionError):
        check_layer_bounds(area_mixed, state, next(_frames("scene", (31,))), "mixed")


def test_int8_weights_are_fp32_checkpoint_quantized():
    """factor = s_in * per-channel weight scale: q * factor / s_in is the FP32 weight within half a
    step, and the INT8 biases are the FP32 biases (optimized/shader/runtime.py:55-78)."""
    rec = torch.load(WEIGHTS / "aeisu_int8_fp16.pt", map_location="cpu", weights_only=True)
    w = D.weights_from_int8(rec)
    layers32 = D.fp32_layers(M.load_folded(WEIGHTS / "aeisu_area.pt"))
    for layer in D.BODY:
        s_in = float(w["act"][REF_SCALES[layer][0]])
        step = (w[layer + ".factor"].double() / s_in).view(-1, 1, 1, 1)
        err = (w[layer + ".wq"].double() * step - layers32[layer]["w"].double()).abs()
        assert bool((err <= 0.5 * step * (1 + 1e-4) + 1e-9).all()), layer
        assert torch.equal(w[layer + ".b"], layers32[layer]["b"]), layer


# ------------------------------------------------------------------------------------------------
# 3. bias correction
# ------------------------------------------------------------------------------------------------
def check_bias_correction_helps(w, state, kind):
    """bias_fp8 = bias + the expected weight-quantization error (calibrate.py, the DIV2K record):
    on the input class a model was calibrated for, the emulation with it is closer to the FP32
    model than the same emulation with the uncorrected bias, by >= 0.3 dB on average."""
    plain = dict(w)
    for layer in D.BODY:                   # the same emulation with bias_fp8 replaced by bias
        plain[layer + ".b8"] = w[layer + ".b"]
    gains = []
    for src in _frames(kind, (0, 1, 2), 128, 192):
        ref = M.forward(src, state).clamp(0, 1)
        gains.append(psnr(D.forward(src, w, "mixed", out_dtype=torch.float32), ref)
                     - psnr(D.forward(src, plain, "mixed", out_dtype=torch.float32), ref))
    assert np.mean(gains) >= 0.3, gains


@pytest.mark.parametrize("tag", ["area", "div2k"])
def test_bias_correction_brings_output_closer_to_fp32(tag, area_mixed, div2k_mixed):
    if tag == "area":
        check_bias_correction_helps(area_mixed, M.load_folded(WEIGHTS / "aeisu_area.pt"), "scene")
    else:
        check_bias_correction_helps(div2k_mixed, M.load_folded(WEIGHTS / "aeisu_div2k_l1.pt"), "pink")


def test_planted_bias_for_bias_fp8_is_caught(monkeypatch, div2k_mixed):
    monkeypatch.setattr(D, "FP8_BIAS", ".b")
    with pytest.raises(AssertionError):
        check_bias_correction_helps(div2k_mixed, M.load_folded(WEIGHTS / "aeisu_div2k_l1.pt"), "pink")


def test_area_bias_correction_within_weight_error_bound():
    """No correction record ships for the area artifact; its correction must still be a weight-
    quantization error applied to a feasible mean input: |bias_fp8 - bias| <= sum |W32 - W_q| * 448 s_in
    (the largest E4M3 input magnitude), and zero for the FP16 layers."""
    t = spyr8f8.read_file(WEIGHTS / "aeisu_area_mixed_fp8.bin")["tensors"]
    layers32 = D.fp32_layers(M.load_folded(WEIGHTS / "aeisu_area.pt"))
    act = t["activation_scales"].astype(np.float64)
    for layer in D.BODY:
        wq = Q.e4m3_decode(t[layer + ".weight_fp8"]).astype(np.float64) * t[layer + ".weight_scale"].reshape(-1, 1, 1, 1)
        dw = np.abs(layers32[layer]["w"].double().numpy() - wq).sum(axis=(1, 2, 3))
        corr = np.abs(t[layer + ".bias_fp8"].astype(np.float64) - t[layer + ".bias"])
        assert np.all(corr <= dw * 448 * act[REF_SCALES[layer][0]] + 1e-7), layer
        assert corr.max() > 0, layer
    for layer in ("project", "refine", "tail"):
        assert np.array_equal(t[layer + ".bias_fp8"], t[layer + ".bias"]), layer


# ------------------------------------------------------------------------------------------------
# head of the quantized policies: the clamped coefficient rounded to FP16
# ------------------------------------------------------------------------------------------------
def _all_fp16_codes() -> torch.Tensor:
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.float16)


def check_clamp_fp16(clamp) -> None:
    """Properties that fix the FP16 clamp up to its rounding, over all 65536 FP16 codes:
    identity (bit for bit, -0 included) for |a| <= 2; an FP16 value; within half an FP16 ulp plus
    (0.05 - fp16(0.05)) (|a| - 2) of the reference's FP32 clamp; odd; non-decreasing in |a|;
    +-inf -> +-2.5 and NaN -> NaN."""
    a16 = _all_fp16_codes()
    a = a16.float()
    c = clamp(a)
    finite = torch.isfinite(a)
    small = finite & (a.abs() <= 2)
    assert torch.equal(c[small].half().view(torch.int16), a16[small].view(torch.int16))
    big = finite & (a.abs() > 2)
    assert torch.equal(c[finite], c[finite].half().float())
    ref = M.coefficient_clamp(a[big]).double()
    ulp = (torch.nextafter(c[big].abs().half(), torch.tensor(float("inf"), dtype=torch.float16)).double()
           - c[big].abs().double())
    bound = ulp / 2 + (0.05 - D.H005) * (a[big].abs().double() - 2) + 1e-9
    assert torch.all((c[big].double() - ref).abs() <= bound)
    nonnan = ~torch.isnan(a)
    assert torch.equal(clamp(-a[nonnan]), -c[nonnan])
    pos = a[finite & (a > 0)].sort().values
    cp = clamp(pos)
    assert torch.all(cp[1:] >= cp[:-1])
    assert clamp(torch.tensor([float("inf"), float("-inf")])).tolist() == [2.5, -2.5]
    assert torch.isnan(clamp(torch.tensor([float("nan")]))).all()


def test_coefficient_clamp_fp16_pins():
    check_clamp_fp16(D.coefficient_clamp_fp16)


@pytest.mark.parametrize("mistake", ["no_cap", "no_sign", "fp32_slope_unrounded", "no_select"])
def test_planted_clamp_fp16_mistakes_are_caught(mistake):
    def bad(t):
        a = t.half().double()
        m = a.abs()
        if mistake == "fp32_slope_unrounded":
            soft = torch.clamp((m - 2) * 0.05 + 2, max=2.5)          # not an FP16 value
        else:
            soft = ((m - 2) * D.H005 + 2).half().double()
            if mistake != "no_cap":
                soft = torch.clamp(soft, max=2.5)
        c = soft if mistake == "no_select" else torch.where(m <= 2, m, soft)
        c = torch.where(torch.isnan(a), a, c if mistake == "no_sign" else torch.copysign(c, a))
        return c.float()
    with pytest.raises(AssertionError):
        check_clamp_fp16(bad)


def test_head_fp16_clamp_stays_within_its_bound_of_the_reference_head(area_mixed):
    """The quantized policies' head (FP16 clamped coefficients) against the reference FP32 clamp on a
    scene frame whose coefficients are scaled so that most exceed the clamp: <= 0.1/255."""
    from aeisu_amd import frames
    src = frames.scene(48, 64, 4, shapes=6, texture=True)[None].half().float()
    padded = F.pad(src, (16, 16, 16, 16), mode="replicate")
    meta = (D.controller(padded, area_mixed, "mixed") * 3).half().float()
    exact = D.head(padded, meta, area_mixed, out_dtype=torch.float32)
    qc = D.head(padded, meta, area_mixed, out_dtype=torch.float32, clamp=D.coefficient_clamp_fp16)
    err = (exact - qc).abs().max().item()
    assert 0 < err <= 0.1 / 255
