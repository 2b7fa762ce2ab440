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
  SrcPyrNativeFp8Conv.cuh:459-471,590-596 (bottlenecks),
  SrcPyrNativeFp8Expand.cuh:233-237,280-302 (expand + skip add),
  SrcPyrNativeFp16Refine.cuh:472-475,494-538 (refine + tail),
  adaptive/AdaptiveReconstruction.cuh:288-417 (head).
* ``int8`` -- the reference conventional INT8/FP16 policy: symmetric INT8
  activations with ``quantize_s8`` and INT32 accumulation, ``acc*factor+bias``
  epilogues (optimized/shader/src/int8_kernels.cuh:2-62,159-201), expand
  output ``fp16(q*s_out + skip)`` (int8_kernels.cuh:52-57).  Project, refine
  and tail use the same FP16/FP32-accumulate arithmetic as ``mixed`` (the
  reference uses HFMA2 partial sums and a Winograd refine,
  fusion_kernels.cu:125-190,249-351; this build keeps FP32 accumulation).

Parity status: the reference ships no Python for the FP8/INT8 emulations, so
this file is pinned by (a) the exact E4M3 / INT8 rounding functions (pinned
in ``oracle.quant``), (b) its FP16 policy agreeing with the FP32 oracle to
well under 1e-3, and (c) the reference's statistical gates: Mixed-vs-FP16
output PSNR >= 35 dB (SrcPyrRuntimeTest.cpp:454-457).  Layer-by-layer
bit-exactness against the reference's CUDA kernels is parity unpinned.
"""
from __future__ import annotations

from typing import Dict, Mapping

import numpy as np
import torch
from torch.nn import functional as F

from . import model as M
from .quant import e4m3_decode, e4m3_round_t, f16, fmaf, quantize_s8

LAYERS = ("project", "compress", "bottleneck0", "bottleneck1", "bottleneck2",
          "bottleneck3", "expand", "refine", "tail")


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
    """INT8/FP16 weights from the shader_precision_v1 payload (Appendix of the artifact)."""
    w: Dict[str, object] = dict(_analysis_from_vector(record["analysis_parameters"].numpy()))
    for layer in ("project", "refine", "tail"):
        w[layer + ".w"] = record["half_weights"][layer].float()
        w[layer + ".b"] = record["half_biases"][layer].float()
    for layer in ("compress", "bottleneck0", "bottleneck1", "bottleneck2", "bottleneck3", "expand"):
        w[layer + ".wq"] = record["int8_weights"][layer].float()
        w[layer + ".factor"] = record["int8_factors"][layer].float()
        w[layer + ".b"] = record["int8_biases"][layer].float()
    w["act"] = torch.as_tensor(record["activation_scales"], dtype=torch.float32)
    w["base"], w["basis"] = record["base"].float(), record["bank"].float()
    return w


def _conv64(x: torch.Tensor, w: torch.Tensor, groups: int = 1) -> torch.Tensor:
    """Convolution accumulated in float64 then rounded once to float32."""
    return F.conv2d(x.double(), w.double(), padding=w.shape[-1] // 2, groups=groups).float()


def _chan(v: torch.Tensor) -> torch.Tensor:
    return v.view(1, -1, 1, 1)


def _inv(s) -> float:
    """float32(1) / float32(s): the host-side reciprocal of SrcPyrCudaRuntime.cu:4403."""
    return float(np.float32(1.0) / np.float32(s))


def features(src: torch.Tensor, w: Mapping[str, object]) -> torch.Tensor:
    """FP16-rounded packed analysis features [B,32,Hp/2,Wp/2] (channel = c*4 + phase)."""
    return f16(F.pixel_unshuffle(M.rgb_to_feature8(src, w), 2))


def project(feat: torch.Tensor, w) -> torch.Tensor:
    """FP16 skip = fp16(leaky(W16 . feat + b)) (SrcPyrCudaRuntime.cu:2568-2583)."""
    acc = _conv64(feat, w["project.w"]) + _chan(w["project.b"])
    return f16(M.leaky(acc))


def _fp8_epilogue(acc, w, layer, s_in, s_out) -> torch.Tensor:
    """fmaf(acc, s_in*wscale, bias_fp8) -> leaky -> e4m3(v * 1/s_out)."""
    scale = (torch.tensor(float(s_in), dtype=torch.float32) * w[layer + ".ws"].float())
    v = fmaf(acc, _chan(scale), _chan(w[layer + ".b8"]))
    v = torch.where(v < 0, v * _chan(w[layer + ".prelu"]), v)
    return e4m3_round_t(v * torch.tensor(_inv(s_out), dtype=torch.float32))


def _int8_epilogue(acc, w, layer, s_out) -> torch.Tensor:
    """fmaf(acc, factor, bias) -> leaky(0.1) -> quantize_s8(v, 1/s_out) (integer-valued float)."""
    v = fmaf(acc, _chan(w[layer + ".factor"]), _chan(w[layer + ".b"]))
    v = torch.where(v >= 0, v, v * torch.tensor(0.1, dtype=torch.float32))
    return quantize_s8(v, _inv(s_out))


def controller(src: torch.Tensor, w: Mapping[str, object], precision: str,
               record: Dict[str, torch.Tensor] | None = None) -> torch.Tensor:
    """Packed FP16 coefficients [B,64,Hp/2,Wp/2] under the given precision policy.

    ``src`` is the padded source (values already FP16-representable for the
    GPU configs).  ``record`` (optional) receives the intermediate tensors.
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
    act = w.get("act")
    if precision == "fp16":
        low = f16(M.leaky(_conv64(F.pixel_unshuffle(skip, 2), w["compress.w"]) + _chan(w["compress.b"])))
        rec["low0"] = low
        for i in range(4):
            low = f16(M.leaky(_conv64(low, w[f"bottleneck{i}.w"], groups=2) + _chan(w[f"bottleneck{i}.b"])))
            rec[f"low{i + 1}"] = low
        e = f16(M.leaky(_conv64(low, w["expand.w"]) + _chan(w["expand.b"])))
        work = f16(F.pixel_shuffle(e, 2) + skip)
    elif precision == "mixed":
        x = e4m3_round_t(F.pixel_unshuffle(skip, 2) * torch.tensor(_inv(act[1]), dtype=torch.float32))
        low = _fp8_epilogue(_conv64(x, w["compress.w8"]), w, "compress", act[1], act[2])
        rec["low0"] = low
        for i in range(4):
            acc = _conv64(low, w[f"bottleneck{i}.w8"], groups=2)
            low = _fp8_epilogue(acc, w, f"bottleneck{i}", act[i + 2], act[i + 3])
            rec[f"low{i + 1}"] = low
        q = _fp8_epilogue(_conv64(low, w["expand.w8"]), w, "expand", act[6], act[7])
        work = f16(fmaf(F.pixel_shuffle(q, 2), float(act[7]), skip))
    elif precision == "int8":
        x = quantize_s8(F.pixel_unshuffle(skip, 2), _inv(act[1]))
        low = _int8_epilogue(_conv64(x, w["compress.wq"]), w, "compress", act[2])
        rec["low0"] = low
        for i in range(4):
            acc = _conv64(low, w[f"bottleneck{i}.wq"], groups=2)
            low = _int8_epilogue(acc, w, f"bottleneck{i}", act[i + 3])
            rec[f"low{i + 1}"] = low
        q = _int8_epilogue(_conv64(low, w["expand.wq"]), w, "expand", act[7])
        work = f16(fmaf(F.pixel_shuffle(q, 2), float(act[7]), skip))
    else:
        raise ValueError(f"unknown precision {precision!r}")
    rec["work"] = work
    dec = f16(M.leaky(_conv64(work, w["refine.w"]) + _chan(w["refine.b"])))
    rec["refine"] = dec
    meta = f16(_conv64(dec, w["tail.w"]) + _chan(f16(w["tail.b"])))
    rec["meta"] = meta
    return meta


def head(src: torch.Tensor, meta: torch.Tensor, w, out_dtype=torch.float16) -> torch.Tensor:
    """FP32 reconstruction on FP16 coefficients, clamp [0,1], round to ``out_dtype``."""
    out = M.reconstruct(src.float(), meta.float(), w["base"].float(), w["basis"].float())
    return out.clamp(0, 1).to(out_dtype).float()


def forward(src: torch.Tensor, w, precision: str, out_dtype=torch.float16,
            record: Dict[str, torch.Tensor] | None = None) -> torch.Tensor:
    """Whole padded frame -> clipped 2x frame under ``precision``."""
    meta = controller(src, w, precision, record)
    return head(src, meta, w, out_dtype)
