"""CPU checks of the C ABI library and the artifact writer (no GPU compute).

* libaeisu_amd.so loads and exports every function declared in include/aeisu_amd.h.
* The SPYR8F8 writer's output is read back by the independent oracle reader.
* Artifact validation in the C++ loader (SrcPyrModel.cpp:257-422 semantics)
  rejects corrupted inputs before any HIP call, with AEISU_ERR_ARTIFACT.
"""
from __future__ import annotations

import ctypes
import re
import struct

import numpy as np
import pytest
import torch

from aeisu_amd import _lib as L
from aeisu_amd import artifacts as A
from oracle import model as M
from oracle import spyr8f8
from tests._util import ROOT, WEIGHTS


def header_functions():
    text = (ROOT / "include" / "aeisu_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aeisu_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    names = header_functions()
    assert len(names) >= 19
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(L.SIGNATURES), "ctypes signatures and header disagree"
    assert lib.aeisu_version().startswith(b"aeisu_amd")


def header_constants():
    """`#define AEISU_<NAME> <integer>` lines of the public header."""
    text = (ROOT / "include" / "aeisu_amd.h").read_text()
    out = {}
    for name, value in re.findall(r"^#define (AEISU_[A-Z0-9_]+)\s+\(?(-?\d+)u?\)?", text, flags=re.M):
        out[name] = int(value)
    return out


def test_binding_constants_match_header():
    """Status codes, precision policies and flags of the ctypes binding are the header's values."""
    h = header_constants()
    for name in ("AEISU_ERR_INVALID_ARGUMENT", "AEISU_ERR_ARTIFACT", "AEISU_ERR_HIP", "AEISU_ERR_STATE",
                 "AEISU_ERR_NONFINITE"):
        assert getattr(L, name) == h[name], name
    assert L.PRECISION == {"fp16": h["AEISU_PRECISION_FP16"], "mixed": h["AEISU_PRECISION_MIXED"],
                           "int8": h["AEISU_PRECISION_INT8"], "mixed-fp8mma": h["AEISU_PRECISION_MIXED_FP8MMA"],
                           "fp32": h["AEISU_PRECISION_FP32"]}
    flags = {k[len("AEISU_"):]: v for k, v in h.items() if k.startswith("AEISU_FLAG_")}
    assert len(flags) >= 5
    for name, value in flags.items():
        assert getattr(L, name) == value, name
    assert len(set(flags.values())) == len(flags) and all(v & (v - 1) == 0 for v in flags.values())


def _create(blob: bytes, precision: str):
    h = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(blob, len(blob))
    rc = L.lib().aeisu_create_from_memory(buf, len(blob), L.PRECISION[precision], ctypes.byref(h))
    msg = L.lib().aeisu_last_error().decode()
    if rc == L.AEISU_OK:
        L.lib().aeisu_destroy(h)
    return rc, msg


def _rewrite(blob: bytes, fn):
    """Apply fn to the tensor dict of a blob and serialise it again (valid checksum)."""
    t = A.read_tensors(blob)
    recs = []
    for name, arr in t.items():
        arr = fn(name, np.array(arr))
        if arr is None:
            continue
        dt = {np.dtype("float16"): A.DT_F16, np.dtype("float32"): A.DT_F32, np.dtype("uint8"): A.DT_E4M3,
              np.dtype("int8"): A.DT_I8}[arr.dtype]
        lay = A.LAYOUT_BASIS if name.startswith("adaptive") else (A.LAYOUT_OIHW if arr.ndim == 4 else A.LAYOUT_VECTOR)
        recs.append((name, dt, lay, arr))
    return A.write(recs)


@pytest.fixture(scope="module")
def blobs():
    return {
        "fp16": A.load_blob(WEIGHTS / "aeisu_area.pt")[0],
        "mixed": (WEIGHTS / "aeisu_area_mixed_fp8.bin").read_bytes(),
        "int8": A.load_blob(WEIGHTS / "aeisu_int8_fp16.pt")[0],
    }


@pytest.mark.parametrize("prec,src", [("fp16", "fp16"), ("mixed", "mixed"), ("int8", "int8"), ("fp16", "mixed"),
                                      ("mixed-fp8mma", "mixed"), ("fp32", "fp16")])
def test_valid_artifacts_pass_validation(blobs, prec, src):
    rc, msg = _create(blobs[src], prec)
    # a CPU-only box fails only at the first HIP call, after validation succeeded
    assert rc == L.AEISU_OK or (rc == L.AEISU_ERR_HIP and "hip" in msg.lower()), msg


def test_fp32_policy_needs_fp32_weights(blobs):
    """FP32 runs every layer's FP32 weights: an FP8 artifact (no *.weight_fp32) is rejected during
    validation, before any HIP call, naming the first missing tensor."""
    rc, msg = _create(blobs["mixed"], "fp32")
    assert rc == L.AEISU_ERR_ARTIFACT and "project.weight_fp32" in msg, msg
    no_refine = _rewrite(blobs["fp16"], lambda name, a: None if name == "refine.weight_fp32" else a)
    rc, msg = _create(no_refine, "fp32")
    assert rc == L.AEISU_ERR_ARTIFACT and "refine.weight_fp32" in msg, msg


def test_writer_round_trip_with_oracle_reader(blobs):
    art = spyr8f8.read(blobs["fp16"])
    state = M.load_folded(WEIGHTS / "aeisu_area.pt")
    t = art["tensors"]
    assert np.array_equal(t["project.weight_fp16"], state["project_540.weight"].half().numpy())
    assert np.array_equal(t["project.weight_fp32"], state["project_540.weight"].numpy())
    # every layer's FP32 weights travel for the FP32 policy
    assert np.array_equal(t["expand.weight_fp32"], state["expand_270.weight"].numpy())
    assert np.array_equal(t["bottleneck1.weight_fp32"], torch.cat((state["bottleneck_270_a2.weight"],
                                                                   state["bottleneck_270_b2.weight"])).numpy())
    assert np.array_equal(t["bottleneck3.bias"], torch.cat((state["bottleneck_270_a4.bias"],
                                                             state["bottleneck_270_b4.bias"])).numpy())
    assert np.array_equal(t["adaptive_basis"], state["basis"].numpy())
    i8 = spyr8f8.read(blobs["int8"])["tensors"]
    rec = torch.load(WEIGHTS / "aeisu_int8_fp16.pt", map_location="cpu", weights_only=True)
    assert np.array_equal(i8["expand.weight_i8"], rec["int8_weights"]["expand"].numpy())
    assert np.array_equal(i8["tail.weight_fp16"], rec["half_weights"]["tail"].numpy())


@pytest.mark.parametrize("case,expect", [
    ("checksum", "checksum mismatch"),
    ("truncated", "inconsistent SPYR8 header"),
    ("magic", "magic/version/endian/flags"),
    ("short", "smaller than its header"),
    ("reserved", "header extension"),
])
def test_corrupted_container_rejected(blobs, case, expect):
    b = bytearray(blobs["mixed"])
    if case == "checksum":
        b[-5] ^= 0x40
    elif case == "truncated":
        b = b[:-64]
    elif case == "magic":
        b[0] = ord("X")
    elif case == "short":
        b = b[:100]
    elif case == "reserved":
        b[400] = 1
    rc, msg = _create(bytes(b), "mixed")
    assert rc == L.AEISU_ERR_ARTIFACT and expect in msg, msg


@pytest.mark.parametrize("case,prec,expect", [
    ("nan_basis", "mixed", "Nonfinite adaptive basis"),
    ("dc_basis", "mixed", "zero-DC/L1"),
    ("nan_base", "mixed", "Nonfinite adaptive learned base"),
    ("prelu", "mixed", "unsupported per-channel slope"),
    ("shape", "mixed", "wrong type or shape: refine.weight_fp16"),
    ("missing_fp8", "mixed", "missing SPYR8 tensor: compress.weight_fp8"),
    ("scale", "mixed", "invalid activation scale"),
    ("fp16_only", "mixed", "missing SPYR8 tensor: activation_scales"),
])
def test_semantic_validation(blobs, case, prec, expect):
    base = blobs["fp16"] if case == "fp16_only" else blobs["mixed"]

    def edit(name, arr):
        if case == "nan_basis" and name == "adaptive_basis":
            arr[3, 2, 1] = np.nan
        if case == "dc_basis" and name == "adaptive_basis":
            arr[0, 5, 0] += 0.01
        if case == "nan_base" and name == "adaptive_base":
            arr[7, 1] = np.inf
        if case == "prelu" and name == "expand.prelu":
            arr[3] = 0.2
        if case == "shape" and name == "refine.weight_fp16":
            arr = arr[:, :, :1, :1].copy()
        if case == "missing_fp8" and name == "compress.weight_fp8":
            return None
        if case == "scale" and name == "activation_scales":
            arr[4] = 0.0
        return arr

    rc, msg = _create(_rewrite(base, edit), prec)
    assert rc == L.AEISU_ERR_ARTIFACT and expect in msg, msg


def test_argument_validation_without_device():
    lib = L.lib()
    assert lib.aeisu_configure(None, 1, 8, 8, 0, 0, 0, 0) == L.AEISU_ERR_INVALID_ARGUMENT
    assert b"null runtime" in lib.aeisu_last_error()
    h = ctypes.c_void_p()
    assert lib.aeisu_create_from_memory(b"x", 1, 99, ctypes.byref(h)) == L.AEISU_ERR_INVALID_ARGUMENT
    assert lib.aeisu_create_from_file(b"/nonexistent/model.bin", 2, ctypes.byref(h)) == L.AEISU_ERR_ARTIFACT
    assert lib.aeisu_intermediate_bytes(None, 0) == 0 and lib.aeisu_persistent_bytes(None) == 0
    assert lib.aeisu_create_sibling(None, ctypes.byref(h)) == L.AEISU_ERR_INVALID_ARGUMENT and not h.value
    assert lib.aeisu_shares_weights(None, None) == 0
    assert lib.aeisu_startup_report(None, None, 0) == 0
    assert lib.aeisu_upscale_noalloc(None, 1, 8, 8, 0, 0, None, None, None) == L.AEISU_ERR_INVALID_ARGUMENT


def test_header_layout_constants():
    b = (WEIGHTS / "aeisu_area_mixed_fp8.bin").read_bytes()
    assert b[:8] == b"SPYR8F8\0" and struct.unpack_from("<I", b, 16)[0] == 0x01020304
    ours = A.load_blob(WEIGHTS / "aeisu_area.pt")[0]
    assert ours[:24] == b[:8] + struct.pack("<IIII", 1, 512, 0x01020304, 0)
    assert ours[24:88] == b[24:88]                                   # architecture id
    assert ours[88:132] == b[88:132]                                 # 11 dimension fields before the count
