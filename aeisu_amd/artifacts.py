"""SPYR8F8 artifact writer and converters for the released AEISU weight files.

The native runtime consumes one container format, SPYR8F8 (reference layout:
optimized/native/src/neural/srcpyr/SrcPyrModel.cpp:37-81, 243-470), so that
no pickle parsing happens in C++.  This module turns every released weight
file into that container:

* folded FP32 checkpoints (``weights/*.pt``, aeisu/runtime.py:35-56) ->
  FP16 artifact: ``<layer>.weight_fp16`` (OIHW), ``.bias``, ``.prelu`` for the
  nine deployed layers, ``adaptive_basis`` = project_basis(basis_raw)
  (aeisu/reconstruction.py:8-12), ``adaptive_base``, ``analysis_stencil``;
* the shader INT8 checkpoint (``shader_precision_v1``,
  optimized/shader/runtime.py:34-53) -> INT8 artifact: the FP16 project /
  refine / tail plus ``<layer>.weight_i8`` (data type 6, an extension of the
  reference's type table), ``.int8_factor`` and ``.bias`` for the six integer
  layers, and its INT8 ``activation_scales``;
* existing SPYR8F8 files (the Mixed FP8 artifacts) are passed through as-is.

Layer names follow the reference artifact: project, compress,
bottleneck0..3 (= cat(bottleneck_270_a{i+1}, bottleneck_270_b{i+1}) along the
output axis, groups of 32), expand, refine, tail.
"""
from __future__ import annotations

import hashlib
import struct
from pathlib import Path
from typing import Dict, List, Tuple

import numpy as np
import torch

ARCHITECTURE = "aif16x5_learnedrgb4dir8_s32_parallel32x4_learnedbase_oc25_v1"
HEADER_SIZE, DESC_SIZE, CHECKSUM_OFFSET, ALIGN = 512, 80, 184, 64
DT_E4M3, DT_F16, DT_F32, DT_I8 = 1, 2, 3, 6
LAYOUT_SCALAR, LAYOUT_VECTOR, LAYOUT_OIHW, LAYOUT_BASIS = 0, 1, 2, 4
LAYERS = ("project", "compress", "bottleneck0", "bottleneck1", "bottleneck2", "bottleneck3",
          "expand", "refine", "tail")
FOLDED_NAMES = {"project": "project_540", "compress": "compress_270", "expand": "expand_270",
                "refine": "refine_540", "tail": "metadata_head"}
_DTYPES = {DT_E4M3: np.uint8, DT_F16: np.float16, DT_F32: np.float32, DT_I8: np.int8}


def project_basis(raw: torch.Tensor, scale: float = 0.5) -> torch.Tensor:
    """Zero-DC, L1 = scale basis, [16,4,25] -> [25,16,4] (aeisu/reconstruction.py:8-12)."""
    raw = raw.float()
    centred = raw - raw.mean(dim=-1, keepdim=True)
    norm = centred.abs().sum(dim=-1, keepdim=True).clamp_min(1e-6)
    return (centred * (scale / norm)).permute(2, 0, 1).contiguous()


def write(tensors: List[Tuple[str, int, int, np.ndarray]], edge_phase_max_shift: float = 0.0,
          edge_gate_gain: float = 0.0) -> bytes:
    """Serialise (name, dtype code, layout code, array) records into a SPYR8F8 blob.

    Layout (SrcPyrModel.cpp:37-81): 512-byte header, one 80-byte descriptor per tensor,
    payload from the first 64-byte boundary after the descriptors, every tensor at a
    64-byte aligned offset in record order, file size padded to a multiple of 64 bytes;
    SHA-256 of the file with its checksum field zeroed stored at byte 184.
    """
    count = len(tensors)
    toc_bytes = count * DESC_SIZE
    payload = -(-(HEADER_SIZE + toc_bytes) // ALIGN) * ALIGN
    offsets, cursor = [], payload
    for _, _, _, arr in tensors:
        offsets.append(cursor)
        cursor = -(-(cursor + arr.nbytes) // ALIGN) * ALIGN
    size = cursor                                   # the file is padded to the alignment too
    blob = bytearray(size)
    dims = (8, 32, 32, 64, 4, 64, 2, 1, 1, 2, 1, count, ALIGN, DESC_SIZE)
    struct.pack_into("<8sIIII64s14I2f4Q", blob, 0, b"SPYR8F8\0", 1, HEADER_SIZE, 0x01020304, 0,
                     ARCHITECTURE.encode(), *dims, edge_phase_max_shift, edge_gate_gain, size, HEADER_SIZE,
                     toc_bytes, payload)
    for i, ((name, dtype, layout, arr), off) in enumerate(zip(tensors, offsets)):
        arr = np.ascontiguousarray(arr, dtype=_DTYPES[dtype])
        if len(name.encode()) >= 32 or arr.ndim == 0 or arr.ndim > 4:
            raise ValueError(f"cannot store tensor {name!r} with shape {arr.shape}")
        shape = list(arr.shape) + [0] * (4 - arr.ndim)
        struct.pack_into("<32sIII4IQQ4s", blob, HEADER_SIZE + i * DESC_SIZE, name.encode(), dtype, layout,
                         arr.ndim, *shape, off, arr.nbytes, b"\0\0\0\0")
        blob[off:off + arr.nbytes] = arr.tobytes()
    digest = hashlib.sha256(bytes(blob)).digest()        # checksum field is still zero here
    blob[CHECKSUM_OFFSET:CHECKSUM_OFFSET + 32] = digest
    return bytes(blob)


def _vec(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).reshape(-1)


def _analysis_vector(get) -> np.ndarray:
    """24 analysis constants in SrcPyrArchitecture.h:42-51 order."""
    return np.concatenate([_vec(get("analysis_rgb_basis")), _vec(get("analysis_rgb_mix")),
                           _vec(get("analysis_dx_rows")), _vec(get("analysis_dy_cols")),
                           _vec(get("analysis_diag45")), _vec(get("analysis_diag135"))])


def _common(records, analysis, base, basis) -> None:
    records += [("adaptive_basis", DT_F32, LAYOUT_BASIS, np.asarray(basis, np.float32)),
                ("precision_guards", DT_F32, LAYOUT_VECTOR, np.zeros(2, np.float32)),
                ("adaptive_base", DT_F32, LAYOUT_BASIS, np.asarray(base, np.float32)),
                ("analysis_stencil", DT_F32, LAYOUT_VECTOR, analysis)]


def _prelu(layer: str, cout: int) -> np.ndarray:
    return np.full(cout, 1.0 if layer == "tail" else 0.1, np.float32)


def state_tensors(payload) -> Dict[str, torch.Tensor]:
    """Tensor state dict of a checkpoint payload (aeisu/runtime.py:35-42)."""
    if isinstance(payload, dict):
        for key in ("model", "model_state_dict", "state_dict"):
            if isinstance(payload.get(key), dict):
                return payload[key]
        if payload and all(torch.is_tensor(v) for v in payload.values()):
            return payload
    raise ValueError("Checkpoint does not contain a tensor state dictionary")


def folded_to_fp16(payload) -> bytes:
    """FP16 SPYR8F8 blob from a folded FP32 checkpoint payload."""
    state = {k: v.detach().float() for k, v in state_tensors(payload).items()}
    if any(".rep_low_u" in k for k in state):
        raise ValueError("training checkpoints must be folded first (export.py)")
    scale = float(payload.get("basis_l1_scale", 0.5)) if isinstance(payload, dict) else 0.5
    records: List[Tuple[str, int, int, np.ndarray]] = []
    for layer in LAYERS:
        if layer.startswith("bottleneck"):
            i = int(layer[-1]) + 1
            w = torch.cat((state[f"bottleneck_270_a{i}.weight"], state[f"bottleneck_270_b{i}.weight"]))
            b = torch.cat((state[f"bottleneck_270_a{i}.bias"], state[f"bottleneck_270_b{i}.bias"]))
        else:
            w, b = state[FOLDED_NAMES[layer] + ".weight"], state[FOLDED_NAMES[layer] + ".bias"]
        records += [(f"{layer}.weight_fp16", DT_F16, LAYOUT_OIHW, w.half().numpy()),
                    (f"{layer}.bias", DT_F32, LAYOUT_VECTOR, b.numpy()),
                    (f"{layer}.prelu", DT_F32, LAYOUT_VECTOR, _prelu(layer, w.shape[0])),
                    # kept at full precision: the FP32 policy runs them as they are, and the FP16
                    # policy splits the project weights into FP16 hi + lo operands
                    (f"{layer}.weight_fp32", DT_F32, LAYOUT_OIHW, w.numpy())]
    basis = project_basis(state["basis_raw"], scale).numpy()
    _common(records, _analysis_vector(lambda k: state[k].numpy()), state["base_kernel"].numpy(), basis)
    return write(records)


def int8_to_blob(record) -> bytes:
    """INT8 SPYR8F8 blob from the ``shader_precision_v1`` payload."""
    if record.get("format") != "shader_precision_v1":
        raise ValueError("not a shader_precision_v1 INT8 checkpoint")
    records: List[Tuple[str, int, int, np.ndarray]] = [
        ("activation_scales", DT_F32, LAYOUT_VECTOR, _vec(record["activation_scales"]))]
    for layer in LAYERS:
        if layer in record["half_weights"]:
            w = record["half_weights"][layer]
            records += [(f"{layer}.weight_fp16", DT_F16, LAYOUT_OIHW, w.half().numpy()),
                        (f"{layer}.bias", DT_F32, LAYOUT_VECTOR, _vec(record["half_biases"][layer]))]
        else:
            w = record["int8_weights"][layer]
            records += [(f"{layer}.weight_i8", DT_I8, LAYOUT_OIHW, w.to(torch.int8).numpy()),
                        (f"{layer}.int8_factor", DT_F32, LAYOUT_VECTOR, _vec(record["int8_factors"][layer])),
                        (f"{layer}.bias", DT_F32, LAYOUT_VECTOR, _vec(record["int8_biases"][layer]))]
        records.append((f"{layer}.prelu", DT_F32, LAYOUT_VECTOR, _prelu(layer, w.shape[0])))
    _common(records, _vec(record["analysis_parameters"]), record["base"].float().numpy(),
            record["bank"].float().numpy())
    return write(records)


def read_tensors(blob: bytes) -> Dict[str, np.ndarray]:
    """Name -> array view of a SPYR8F8 blob (no validation; the C++ loader validates)."""
    count = struct.unpack_from("<I", blob, 132)[0]
    out = {}
    for i in range(count):
        name, dtype, _, rank, *rest = struct.unpack_from("<32sIII4IQQ4s", blob, HEADER_SIZE + i * DESC_SIZE)
        shape, off, nbytes = tuple(rest[:4])[:rank], rest[4], rest[5]
        arr = np.frombuffer(blob, dtype=_DTYPES[dtype], count=int(np.prod(shape)), offset=off)
        out[name.split(b"\0", 1)[0].decode()] = arr.reshape(shape)
    return out


def read_records(blob: bytes) -> Tuple[List[Tuple[str, int, int, np.ndarray]], Dict[str, float]]:
    """Ordered (name, dtype, layout, array) records and the edge-phase header fields of a
    SPYR8F8 blob, such that ``write(records, **header) == blob`` for a well-formed file."""
    count = struct.unpack_from("<I", blob, 132)[0]
    shift, gain = struct.unpack_from("<2f", blob, 144)
    records = []
    for i in range(count):
        name, dtype, layout, rank, *rest = struct.unpack_from("<32sIII4IQQ4s", blob, HEADER_SIZE + i * DESC_SIZE)
        shape, off = tuple(rest[:4])[:rank], rest[4]
        arr = np.frombuffer(blob, dtype=_DTYPES[dtype], count=int(np.prod(shape)), offset=off).reshape(shape)
        records.append((name.split(b"\0", 1)[0].decode(), dtype, layout, arr.copy()))
    return records, {"edge_phase_max_shift": shift, "edge_gate_gain": gain}


def load_blob(path) -> Tuple[bytes, str]:
    """(SPYR8F8 blob, natural precision) for any released weight file.

    Natural precision: "fp16" for folded checkpoints, "mixed" for SPYR8F8
    artifacts carrying FP8 weights, "int8" for the shader INT8 checkpoint.
    """
    path = Path(path)
    data = path.read_bytes()
    if data[:8] == b"SPYR8F8\0":
        names = read_tensors(data)
        return data, ("mixed" if "compress.weight_fp8" in names else
                      "int8" if "compress.weight_i8" in names else "fp16")
    payload = torch.load(path, map_location="cpu", weights_only=True)
    if isinstance(payload, dict) and payload.get("format") == "shader_precision_v1":
        return int8_to_blob(payload), "int8"
    return folded_to_fp16(payload), "fp16"
