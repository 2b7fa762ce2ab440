"""Emulation of the reduced-precision GPU deployments -- TEST INFRASTRUCTURE ONLY.

Three arithmetic policies, each a CPU restatement (torch float32/float64 plus
the exact number-format rounding of ``oracle.quant``):

* ``fp16``  -- every controller activation stored in FP16, FP16 weights, FP32
  accumulation, FP32 head math on FP16 coefficients; the analysis features
  and the project GEMM stay FP32-accurate (the project weights reach |w|~31
  and FP16 operands there alone cost ~4e-3 of output error).  (Reference FP16
  native route: SrcPyrCudaRuntime.cu:4131-4873 with the cuDNN/WMMA FP16 stages,
  which rounds features and project weights to FP16.)
* ``mixed`` -- the reference "Mixed" deployment: FP16 project/refine/tail,
  FP8-E4M3 compress, 4 grouped bottlenecks and expand with per-channel
  weight scales and per-tensor activation scales.  Quantization points follow
  optimized/native/src/neural/srcpyr/SrcPyrCudaRuntime.cu:2480-2583 (features
  and project), SrcPyrNativeFp8Compress.cuh:94-129,222-236 (compress),
  SrcPyrNativeFp8Conv.cuh:459-471,528-606 (bottlenecks),
  SrcPyrNativeFp8Expand.cuh:233-237,280-302 (expand + skip add),
  SrcPyrNativeFp16Refine.cuh:472-475,494-538 (refine + tail),
  adaptive/AdaptiveReconstruction.cuh:288-417 (head); scale indices and host
  reciprocals SrcPyrCudaRuntime.cu:4395-4445, bias selection (``bias_fp8``)
  SrcPyrCudaRuntime.cu:3814-3817, FP16 tail bias 2999-3006.
* ``int8`` -- the reference conventional INT8/FP16 policy: symmetric INT8
  activations with ``quantize_s8`` and INT32 accumulation, ``acc*factor+bias``
  epilogues (optimized/shader/src/int8_kernels.cuh:2-62,159-201), expand
  output ``fp16(q*s_out + skip)`` (int8_kernels.cuh:52-60), scale indices
  optimized/shader/runtime.py:60-76.  Project, refine and tail use the same
  FP16/FP32-accumulate arithmetic as ``mixed`` (the reference uses HFMA2
  partial sums and a Winograd refine, fusion_kernels.cu:125-190,249-351; this
  build keeps FP32 accumulation).

Accumulation of the E4M3 layers.  The reference runs each of them as a chain
of ``mma.sync.m16n8k32 ... e4m3.e4m3.f32`` instructions, each adding the sum of
32 products to the FP32 accumulator (SrcPyrNativeFp8Compress.cuh:166-226,
SrcPyrNativeFp8Conv.cuh:528-606, SrcPyrNativeFp8Expand.cuh:141-227).  The
emulation models one instruction as D = fl32(C + exact sum of its 32
products) (an E4M3 x E4M3 product has at most 8 significant bits and the sums
stay below 2^26 in multiples of 2^-18, so float64 holds them exactly), applied
chunk by chunk in the reference's K order:

* compress: 4 chunks; chunk j holds unshuffled channels 32j..32j+31, i.e.
  skip channels 8j..8j+7 of all four phases (K index c*4 + phase);
* bottleneck: 9 chunks, one per tap in row-major (dy, dx) order, each the 32
  input channels of the output channel's group;
* expand: 2 chunks, input channels 0..31 then 32..63.

INT8 sums are integers (exact in any order).  The FP16 layers run as chains of
``mma.sync.m16n8k16 ... f32.f16.f16.f32`` (refine, tail) or WMMA 16x16x16
(project) steps from a zero accumulator, each step modelled the same way as
D = fl32(C + exact sum of its 16 products), followed by a separate FP32 bias
add (``fp16_steps`` / ``fp16_chain``):

* project: 2 steps, features 0..15 then 16..31 (channel = feature*4 + phase);
* refine: 18 steps, the 9 taps in row-major order, each input channels 0..15
  then 16..31;
* tail: 4 steps, refine channels 0..15, 16..31, 32..47, 48..63.

Modelling assumption, not a pinned fact: NVIDIA does not specify how a tensor
core step rounds its sum, and the reference ships no output of its FP16/FP8
kernels, so "exact sum rounded once per step" is this emulation's model of the
reference's MMA steps (E4M3 and FP16 alike).  The pins below fix the model's
rounding points, K order and quantization points; agreement of the Mixed and
INT8 policies with the reference's CUDA output itself is parity unpinned.
gfx950's FP16 MFMAs do not compute this model either (they align each pass of
8 products to the largest term and drop bits 24 below it;
tests/test_gpu_mfma_f16.py), which is the one source of the GPU's residual
deviation from this emulation.

Pinning (tests/test_deploy.py): every stage function is checked against a
brute-force rational-arithmetic restatement of the reference expression on
inputs built to expose its rounding points (chunked FP32 accumulation of the
E4M3 layers and of the FP16 K=16 chains, ``fmaf`` epilogue, FP16 tail bias, contracted expand residual, saturating
E4M3 / INT8 requantization); every FP8 and INT8 layer is bounded against the
FP32 checkpoint's layer on the same dequantized input (weight-quantization
error + bias correction + half an output quantum) and a per-layer scale
slope of 1 within 0.3 %; ``bias_fp8`` is shown to bring the output closer to
the FP32 model than ``bias`` on the input class each model was calibrated
for, and the artifacts' ``bias_fp8 - bias`` equals the exporter's recorded
correction (DIV2K); planted mistakes (``bias`` for ``bias_fp8``, off-by-one
activation-scale indices, an unrounded tail bias, a split expand residual,
float64 or phase-major instead of the reference's chunked FP32 accumulation,
one rounding of an FP16 layer's whole sum, interleaved FP16 chunks, a
double-rounded fmaf) each fail one of those checks.
"""
from __future__ import annotations

from typing import Dict, Mapping, Sequence

import numpy as np
import torch
from torch.nn import functional as F

from . import model as M
from .quant import e4m3_decode, e4m3_round_t, f16, fmaf, quantize_s8, round_f32

LAYERS = ("project", "compress", "bottleneck0", "bottleneck1", "bottleneck2",
          "bottleneck3", "expand", "refine", "tail")
BODY = ("compress", "bottleneck0", "bottleneck1", "bottleneck2", "bottleneck3", "expand")

# Activation-scale indices (input, output) of each quantized layer: compress s1 -> s2
# (SrcPyrCudaRuntime.cu:4397-4408), bottleneck b s(b+2) -> s(b+3) (4427-4436), expand
# s6 -> s7 (4587-4601); the INT8 route uses the same table (optimized/shader/runtime.py:60-76).
# Bias of the E4M3 layers: Fp8Bias() returns the bias-corrected ``bias_fp8`` for the adaptive-filter
# artifacts (SrcPyrCudaRuntime.cu:3814-3817); project, refine and tail keep ``bias``.
FP8_BIAS = ".b8"
SCALE_INDEX = {"compress": (1, 2), "bottleneck0": (2, 3), "bottleneck1": (3, 4),
               "bottleneck2": (4, 5), "bottleneck3": (5, 6), "expand": (6, 7)}


def _analysis_from_vector(v) -> Dict[str, torch.Tensor]:
    """24 analysis constants (SrcPyrArchitecture.h:42-51 order) -> model.py names."""
    v = torch.as_tensor(np.asarray(v, dtype=np.float32))
    return {
        "analysis_rgb_basis": v[0:9].reshape(3, 3), "analysis_rgb_mix": v[9:12],
        "analysis_dx_rows": v[12:15], "analysis_dy_cols": v[15:18],
        "analysis_diag45": v[18:21], "analysis_diag135": v[21:24],
    }


def weights_from_folded(state: Mapping[str, torch.Tensor]) -> Dict[str, object]:
    """FP16 deployment weights from a folded FP32 state (oracle.model.load_folded)."""
    w: Dict[str, object] = {k: state[k] for k in M.ANALYSIS_KEYS}
    names = {"project": "project_540", "compress": "compress_270", "expand": "expand_270",
             "refine": "refine_540", "tail": "metadata_head"}
    for layer, src in names.items():
        w[layer + ".w"] = f16(state[src + ".weight"])
        w[layer + ".b"] = state[src + ".bias"].float()
    for i in range(4):
        a, b = f"bottleneck_270_a{i + 1}", f"bottleneck_270_b{i + 1}"
        w[f"bottleneck{i}.w"] = f16(torch.cat((state[a + ".weight"], state[b + ".weight"])))
        w[f"bottleneck{i}.b"] = torch.cat((state[a + ".bias"], state[b + ".bias"])).float()
    w["project.w32"] = state["project_540.weight"].float()
    w["base"], w["basis"] = state["base"].float(), state["basis"].float()
    return w


def fp32_layers(state: Mapping[str, torch.Tensor]) -> Dict[str, Dict[str, torch.Tensor]]:
    """FP32 checkpoint weights per deployed layer name (bottleneck i = cat(a_{i+1}, b_{i+1}))."""
    out = {"compress": ("compress_270",), "expand": ("expand_270",)}
    layers = {k: {"w": state[v[0] + ".weight"].float(), "b": state[v[0] + ".bias"].float()} for k, v in out.items()}
    for i in range(4):
        a, b = f"bottleneck_270_a{i + 1}", f"bottleneck_270_b{i + 1}"
        layers[f"bottleneck{i}"] = {"w": torch.cat((state[a + ".weight"], state[b + ".weight"])).float(),
                                    "b": torch.cat((state[a + ".bias"], state[b + ".bias"])).float()}
    return layers


def weights_from_spyr(art) -> Dict[str, object]:
    """Mixed/FP16 deployment weights from an oracle.spyr8f8.read() result."""
    t = art["tensors"]
    w: Dict[str, object] = dict(_analysis_from_vector(t["analysis_stencil"]))
    for layer in LAYERS:
        w[layer + ".w"] = torch.from_numpy(t[layer + ".weight_fp16"].astype(np.float32))
        w[layer + ".b"] = torch.from_numpy(t[layer + ".bias"])
        w[layer + ".b8"] = torch.from_numpy(t[layer + ".bias_fp8"])
        w[layer + ".w8"] = torch.from_numpy(e4m3_decode(t[layer + ".weight_fp8"]))
        w[layer + ".ws"] = torch.from_numpy(t[layer + ".weight_scale"])
        w[layer + ".prelu"] = torch.from_numpy(t[layer + ".prelu"])
    w["act"] = torch.from_numpy(t["activation_scales"])
    w["base"] = torch.from_numpy(t["adaptive_base"])
    w["basis"] = torch.from_numpy(t["adaptive_basis"])
    return w


def weights_from_int8(record) -> Dict[str, object]:
    """INT8/FP16 weights from the shader_precision_v1 payload (optimized/shader/runtime.py:34-53)."""
    w: Dict[str, object] = dict(_analysis_from_vector(record["analysis_parameters"].numpy()))
    for layer in ("project", "refine", "tail"):
        w[layer + ".w"] = record["half_weights"][layer].float()
        w[layer + ".b"] = record["half_biases"][layer].float()
    for layer in BODY:
        w[layer + ".wq"] = record["int8_weights"][layer].float()
        w[layer + ".factor"] = record["int8_factors"][layer].float()
        w[layer + ".b"] = record["int8_biases"][layer].float()
    w["act"] = torch.as_tensor(record["activation_scales"], dtype=torch.float32)
    w["base"], w["basis"] = record["base"].float(), record["bank"].float()
    return w


# ------------------------------------------------------------------------------------------------
# accumulation
# ------------------------------------------------------------------------------------------------
def _conv64(x: torch.Tensor, w: torch.Tensor, groups: int = 1) -> torch.Tensor:
    """Convolution summed exactly (float64) and rounded once to float32 (FP16 layers, INT8 sums)."""
    return F.conv2d(x.double(), w.double(), padding=w.shape[-1] // 2, groups=groups).float()


def chunk_sums(x: torch.Tensor, w: torch.Tensor, layer: str) -> Sequence[torch.Tensor]:
    """Exact float64 partial sums of the K=32 chunks of an E4M3 layer, in the reference's order.

    ``x`` holds E4M3 values [B, Cin, H, W] (for compress: the unshuffled skip, channel c*4+phase),
    ``w`` E4M3 weight values [Cout, Cin, k, k].
    """
    x64, w64 = x.double(), w.double()
    if layer == "compress" or layer == "expand":
        return [F.conv2d(x64[:, 32 * j:32 * j + 32], w64[:, 32 * j:32 * j + 32]) for j in range(x.shape[1] // 32)]
    h, wd = x.shape[-2:]
    xp = F.pad(x64, (1, 1, 1, 1))
    return [F.conv2d(xp[:, :, dy:dy + h, dx:dx + wd], w64[:, :, dy:dy + 1, dx:dx + 1], groups=2)
            for dy in range(3) for dx in range(3)]


def mma_chain(parts: Sequence[torch.Tensor]) -> torch.Tensor:
    """FP32 accumulator over exact chunk sums: acc <- fl32(acc + chunk), acc starting at 0.

    acc is a float32 multiple of 2^-18 and the chunk an exact multiple of 2^-18 below 2^26, so
    their float64 sum is exact and its rounding to float32 is the single rounding of one MMA.
    """
    acc = torch.zeros_like(parts[0], dtype=torch.float32)
    for part in parts:
        acc = (acc.double() + part).float()
    return acc


# FP16 layers (project, refine, tail): chains of K=16 MMA steps with an FP32 accumulator


def fp16_steps(x: torch.Tensor, w: torch.Tensor):
    """The reference's K=16 steps of an FP16 layer, in its order, as (input, weight) pairs of 1x1
    convolutions over the same output grid.

    1x1 layers take input channels 16s..16s+15 at step s: project 0-15 then 16-31
    (SrcPyrCudaRuntime.cu:2539-2547, ``k`` over ``s_act[... + k * 16]``), tail 0-15 .. 48-63
    (SrcPyrNativeFp16Refine.cuh:509-532).  The 3x3 refine takes its taps in row-major (r, s) order and
    each tap's channels 0-15 then 16-31 (SrcPyrNativeFp16Refine.cuh:425-466), zero outside the grid.
    """
    cin = x.shape[1]
    if w.shape[-1] == 1:
        return [(x[:, c:c + 16], w[:, c:c + 16]) for c in range(0, cin, 16)]
    h, wd = x.shape[-2:]
    xp = F.pad(x, (1, 1, 1, 1))
    return [(xp[:, c:c + 16, r:r + h, s:s + wd], w[:, c:c + 16, r:r + 1, s:s + 1])
            for r in range(3) for s in range(3) for c in range(0, cin, 16)]


def _split20(v: torch.Tensor):
    """FP16 values v -> integer-valued float64 (hi, lo) with v * 2^24 = hi * 2^20 + lo, 0 <= lo < 2^20.

    Every FP16 value is an integer multiple of 2^-24 below 2^16 in magnitude, so |hi| <= 2^20."""
    n = v.double() * 2.0 ** 24
    hi = torch.floor(n / 2.0 ** 20)
    return hi, n - hi * 2.0 ** 20


def fp16_chain(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """FP32 accumulator of an FP16 layer: acc <- fl32(acc + exact sum of one K=16 step), from 0.

    One step is the reference's ``mma.sync.m16n8k16 ... f32.f16.f16.f32`` (or WMMA 16x16x16), modelled
    as the exact sum of its 16 products added to the accumulator and rounded once to FP32.  ``x`` and
    ``w`` hold FP16 values.  The step sum is computed exactly as an integer multiple of 2^-48: each
    operand is split into 20-bit integer halves (``_split20``), the four half-products are summed by a
    float64 convolution whose partial sums stay below 2^45 (exact), and the halves are recombined in
    int64 (values up to 2^14 in magnitude; larger ones raise OverflowError).  The accumulator stays a multiple of 2^-48 (a float32 rounding of such a value), so the
    int64 sum with it is exact and is rounded once to float32 (``round_f32`` breaks the float64 ties).
    """
    acc = None
    for xs, ws in fp16_steps(x, w):
        xh, xl = _split20(xs)
        wh, wl = _split20(ws)
        b, co = xs.shape[0], ws.shape[0]
        c = F.conv2d(torch.cat((xh, xl)), torch.cat((wh, wl)))
        hh, hl, lh, ll = c[:b, :co], c[:b, co:], c[b:, :co], c[b:, co:]
        if not bool((hh.abs() * 2.0 ** 40 + (hl + lh).abs() * 2.0 ** 20 + ll.abs() < 2.0 ** 62).all()):
            raise OverflowError("FP16 step sum beyond the exact int64 range (|sum| >= 2^14)")
        s = (hh.long() << 40) + ((hl.long() + lh.long()) << 20) + ll.long()
        if acc is not None:
            s = s + (acc.double() * 2.0 ** 48).long()
        approx = s.double()
        err = (s - approx.long()).double()
        acc = round_f32(approx * 2.0 ** -48, err * 2.0 ** -48)
    return acc


# ------------------------------------------------------------------------------------------------
# stages
# ------------------------------------------------------------------------------------------------
def _chan(v: torch.Tensor) -> torch.Tensor:
    return v.view(1, -1, 1, 1)


def _inv(s) -> float:
    """float32(1) / float32(s): the host-side reciprocal of SrcPyrCudaRuntime.cu:4403 and
    optimized/shader/src/int8_kernels.cuh:84,149."""
    return float(np.float32(1.0) / np.float32(s))


def _scales(w, layer: str):
    i, o = SCALE_INDEX[layer]
    act = w["act"]
    return float(act[i]), float(act[o])


def features(src: torch.Tensor, w: Mapping[str, object]) -> torch.Tensor:
    """FP16-rounded packed analysis features [B,32,Hp/2,Wp/2] (channel = c*4 + phase)."""
    return f16(F.pixel_unshuffle(M.rgb_to_feature8(src, w), 2))


def project(feat: torch.Tensor, w) -> torch.Tensor:
    """FP16 skip = fp16(leaky(fl32(acc + b))), acc the K=16 chain over the 32 feature channels
    (SrcPyrCudaRuntime.cu:2539-2547 accumulate, 2568-2583 bias add, slope and FP16 store)."""
    acc = fp16_chain(feat, w["project.w"]) + _chan(w["project.b"])
    return f16(M.leaky(acc))


def fp8_compress_input(skip: torch.Tensor, w) -> torch.Tensor:
    """E4M3 values of unshuffle(skip) * fl32(1/s1) (SrcPyrNativeFp8Compress.cuh:94-129)."""
    s_in, _ = _scales(w, "compress")
    return e4m3_round_t(F.pixel_unshuffle(skip, 2) * torch.tensor(_inv(s_in), dtype=torch.float32))


def fp8_pre_round(acc, w, layer: str):
    """The float32 value an E4M3 layer's epilogue rounds, and the magnitude of the terms it came
    from (|acc * scale| + |bias|, times 1/s_out: the scale of its accumulated rounding differences)."""
    s_in, s_out = _scales(w, layer)
    scale = torch.tensor(s_in, dtype=torch.float32) * w[layer + ".ws"].float()
    bias = w[layer + FP8_BIAS].float()
    v = fmaf(acc, _chan(scale), _chan(bias))
    v = torch.where(v < 0, v * _chan(w[layer + ".prelu"]), v)
    inv = torch.tensor(_inv(s_out), dtype=torch.float32)
    return v * inv, ((acc * _chan(scale)).abs() + _chan(bias).abs()) * inv


def fp8_epilogue(acc, w, layer: str) -> torch.Tensor:
    """fmaf(acc, fl32(s_in * wscale), bias_fp8) -> LeakyReLU -> e4m3(v * fl32(1/s_out)).

    SrcPyrNativeFp8Compress.cuh:145-163,229-236 (and the same lines of the grouped and expand kernels).
    """
    return e4m3_round_t(fp8_pre_round(acc, w, layer)[0])


def fp8_acc(x: torch.Tensor, w, layer: str) -> torch.Tensor:
    """FP32 accumulator of an E4M3 layer on E4M3 values ``x``."""
    return mma_chain(chunk_sums(x, w[layer + ".w8"], layer))


def fp8_layer(x: torch.Tensor, w, layer: str) -> torch.Tensor:
    """One E4M3 layer: E4M3 values in, E4M3 values out."""
    return fp8_epilogue(fp8_acc(x, w, layer), w, layer)


def expand_residual(q: torch.Tensor, s7: float, skip: torch.Tensor) -> torch.Tensor:
    """fp16(fmaf(pixel_shuffle(q), s7, skip)): ``float(q) * s7 + skip`` contracted into one FMA by
    nvcc -O3 (SrcPyrNativeFp8Expand.cuh:290-302; int8_kernels.cuh:60 under --use_fast_math)."""
    return f16(fmaf(F.pixel_shuffle(q, 2), float(np.float32(s7)), skip))


def int8_input(skip: torch.Tensor, w) -> torch.Tensor:
    """quantize_s8(unshuffle(skip), 1/s1) (int8_kernels.cuh:24-29)."""
    s_in, _ = _scales(w, "compress")
    return quantize_s8(F.pixel_unshuffle(skip, 2), _inv(s_in))


def int8_pre_round(acc, w, layer: str):
    """The float32 value an INT8 layer's epilogue rounds to an integer, and its terms' magnitude."""
    _, s_out = _scales(w, layer)
    v = fmaf(acc, _chan(w[layer + ".factor"]), _chan(w[layer + ".b"]))
    v = torch.where(v >= 0, v, v * torch.tensor(0.1, dtype=torch.float32))
    inv = torch.tensor(_inv(s_out), dtype=torch.float32)
    return v * inv, ((acc * _chan(w[layer + ".factor"])).abs() + _chan(w[layer + ".b"]).abs()) * inv


def int8_epilogue(acc, w, layer: str) -> torch.Tensor:
    """fmaf(acc, factor, bias) -> leaky(0.1) -> quantize_s8(v, 1/s_out) (int8_kernels.cuh:47-50)."""
    t = int8_pre_round(acc, w, layer)[0]
    return torch.clamp(torch.round(t), -127, 127)


def int8_acc(x: torch.Tensor, w, layer: str) -> torch.Tensor:
    """INT32 accumulator (exact, as float32: |acc| <= 127 * 127 * 288 < 2^24) of an INT8 layer."""
    return _conv64(x, w[layer + ".wq"], 2 if layer.startswith("bottleneck") else 1)


def int8_layer(x: torch.Tensor, w, layer: str) -> torch.Tensor:
    return int8_epilogue(int8_acc(x, w, layer), w, layer)


def refine(work: torch.Tensor, w) -> torch.Tensor:
    """fp16(leaky(fl32(acc + bias))), acc the 18-step K=16 chain (9 taps x 2 channel halves), with the
    FP32 ``.bias`` (SrcPyrNativeFp16Refine.cuh:425-466 accumulate, 472-475 epilogue)."""
    return f16(M.leaky(fp16_chain(work, w["refine.w"]) + _chan(w["refine.b"])))


def tail(dec: torch.Tensor, w) -> torch.Tensor:
    """fp16(fl32(acc + fp16(bias))), acc the 4-step K=16 chain over the 64 refine channels
    (SrcPyrNativeFp16Refine.cuh:494-538; bias rounded on the host, SrcPyrCudaRuntime.cu:2999-3006)."""
    return f16(fp16_chain(dec, w["tail.w"]) + _chan(f16(w["tail.b"])))


def controller(src: torch.Tensor, w: Mapping[str, object], precision: str,
               record: Dict[str, torch.Tensor] | None = None) -> torch.Tensor:
    """Packed FP16 coefficients [B,64,Hp/2,Wp/2] under the given precision policy.

    ``src`` is the padded source (values already FP16-representable for the
    GPU configs).  ``record`` (optional) receives the intermediate tensors:
    features, skip, low0..low4 (E4M3 values / INT8 codes / FP16 values),
    work, refine, meta.
    """
    rec = record if record is not None else {}
    if precision == "fp16":
        # FP16 policy: the project GEMM runs on FP32-accurate operands (features and weights
        # split into FP16 hi + lo on the GPU); its output is stored in FP16 like every activation.
        feat = F.pixel_unshuffle(M.rgb_to_feature8(src, w), 2)
        wp = w.get("project.w32", w["project.w"])
        skip = f16(M.leaky(_conv64(feat, wp) + _chan(w["project.b"])))
    else:
        feat = features(src, w)
        skip = project(feat, w)
    rec["features"], rec["skip"] = feat, skip
    if precision == "fp16":
        low = f16(M.leaky(_conv64(F.pixel_unshuffle(skip, 2), w["compress.w"]) + _chan(w["compress.b"])))
        rec["low0"] = low
        for i in range(4):
            low = f16(M.leaky(_conv64(low, w[f"bottleneck{i}.w"], groups=2) + _chan(w[f"bottleneck{i}.b"])))
            rec[f"low{i + 1}"] = low
        e = f16(M.leaky(_conv64(low, w["expand.w"]) + _chan(w["expand.b"])))
        work = f16(F.pixel_shuffle(e, 2) + skip)
    elif precision in ("mixed", "int8"):
        layer_fn, x = (fp8_layer, fp8_compress_input(skip, w)) if precision == "mixed" else (int8_layer, int8_input(skip, w))
        rec["compress_in"] = x
        low = layer_fn(x, w, "compress")
        rec["low0"] = low
        for i in range(4):
            low = layer_fn(low, w, f"bottleneck{i}")
            rec[f"low{i + 1}"] = low
        q = layer_fn(low, w, "expand")
        rec["expand_out"] = q
        work = expand_residual(q, _scales(w, "expand")[1], skip)
    else:
        raise ValueError(f"unknown precision {precision!r}")
    rec["work"] = work
    dec = refine(work, w)
    rec["refine"] = dec
    meta = tail(dec, w)
    rec["meta"] = meta
    return meta


# FP16 value of 0.05 (0x2A66 = 0.04998779296875): the slope the quantized policies' head clamps with.
H005 = float(np.float16(0.05))


def coefficient_clamp_fp16(t: torch.Tensor) -> torch.Tensor:
    """Clamped coefficient rounded to FP16, as the head of the quantized policies computes it.

    c = a for |a| <= 2, else sign(a) * min(rne16((|a| - 2) * fp16(0.05) + 2), 2.5): one rounding
    of an FP16 fused multiply-add (|a| - 2 is exact in FP16 for |a| > 2; the float64 product of two
    11-bit significands and the sum with 2 are exact, so ``.half()`` is that single rounding).
    +-inf -> +-2.5, NaN stays NaN.  The reference clamp (aeisu/reconstruction.py:15-17,
    ``model.coefficient_clamp``) is FP32; this value is within half an FP16 ulp of c plus
    (0.05 - fp16(0.05)) (|a| - 2) of it, and equal to it for |a| <= 2.
    """
    a = t.half().double()
    m = a.abs()
    soft = torch.clamp(((m - 2) * H005 + 2).half().double(), max=2.5)
    c = torch.where(m <= 2, m, soft)
    c = torch.where(torch.isnan(a), a, torch.copysign(c, a))
    return c.float()


def head(src: torch.Tensor, meta: torch.Tensor, w, out_dtype=torch.float16, clamp=None) -> torch.Tensor:
    """FP32 reconstruction on FP16 coefficients, clamp [0,1], round to ``out_dtype``.

    ``clamp``: the coefficient clamp (default the reference's FP32 ``coefficient_clamp``, which the
    emulated deployments use; ``coefficient_clamp_fp16`` restates the quantized policies' GPU head).
    """
    out = M.reconstruct(src.float(), meta.float(), w["base"].float(), w["basis"].float(), clamp)
    return out.clamp(0, 1).to(out_dtype).float()


def forward(src: torch.Tensor, w, precision: str, out_dtype=torch.float16,
            record: Dict[str, torch.Tensor] | None = None) -> torch.Tensor:
    """Whole padded frame -> clipped 2x frame under ``precision``."""
    meta = controller(src, w, precision, record)
    return head(src, meta, w, out_dtype)
