"""Independent SPYR8F8 artifact reader -- TEST INFRASTRUCTURE ONLY.

Follows the reference loader optimized/native/src/neural/srcpyr/SrcPyrModel.cpp:
header layout 37-68, descriptor layout 70-81, validation 243-353, tensor
requirements 355-470.  It is deliberately separate from the product's C++
parser and Python writer so that the tests can compare the two.

Pinning: Appendix-B identities against the folded FP32 checkpoints
(fp16(weight) == weight_fp16, biases equal, analysis tensors equal,
base_kernel == adaptive_base, project_basis(basis_raw) ~= adaptive_basis).
"""
from __future__ import annotations

import hashlib
import struct
from typing import Dict

import numpy as np

HEADER_SIZE = 512
DESC_SIZE = 80
CHECKSUM_OFFSET = 184
_HEADER = struct.Struct("<8sIIII64s14I2f4Q32s")       # 216 bytes before the reserved tail
_DESC = struct.Struct("<32sIII4IQQ4s")
DTYPES = {1: np.uint8, 2: np.float16, 3: np.float32,    # 1 = e4m3fn codes
          6: np.int8}                                   # 6 = INT8 (this build's extension for the INT8 policy)
LAYER_NAMES = ("project", "compress", "bottleneck0", "bottleneck1", "bottleneck2",
               "bottleneck3", "expand", "refine", "tail")


def read(data: bytes) -> Dict[str, object]:
    if len(data) < HEADER_SIZE:
        raise ValueError("artifact smaller than its header")
    f = _HEADER.unpack_from(data, 0)
    magic, version, header_size, endian, flags, arch = f[:6]
    (logical, packed, c540, c270, layers, tail, scale, fp8fmt, act_layout,
     weight_layout, scale_conv, count, align, desc_size) = f[6:20]
    edge_shift, edge_gain = f[20:22]
    file_size, toc_off, toc_bytes, payload_off = f[22:26]
    checksum = f[26]
    if magic != b"SPYR8F8\0" or version != 1 or header_size != HEADER_SIZE or \
            endian != 0x01020304 or flags != 0:
        raise ValueError("unsupported SPYR8 magic/version/endian/flags")
    if any(data[_HEADER.size:HEADER_SIZE]):
        raise ValueError("nonzero header extension bytes")
    if file_size != len(data) or toc_off != HEADER_SIZE or toc_bytes != count * DESC_SIZE \
            or desc_size != DESC_SIZE or align != 64:
        raise ValueError("inconsistent header")
    zeroed = bytearray(data)
    zeroed[CHECKSUM_OFFSET:CHECKSUM_OFFSET + 32] = bytes(32)
    if hashlib.sha256(zeroed).digest() != checksum:
        raise ValueError("checksum mismatch")
    tensors: Dict[str, np.ndarray] = {}
    for i in range(count):
        name, dtype, layout, rank, s0, s1, s2, s3, off, nbytes, _ = \
            _DESC.unpack_from(data, toc_off + i * DESC_SIZE)
        name = name.split(b"\0", 1)[0].decode()
        shape = (s0, s1, s2, s3)[:rank]
        arr = np.frombuffer(data, dtype=DTYPES[dtype], count=int(np.prod(shape)), offset=off)
        tensors[name] = arr.reshape(shape).copy()
    return {
        "architecture": arch.split(b"\0", 1)[0].decode(),
        "dims": dict(logical=logical, packed=packed, c540=c540, c270=c270, layers=layers,
                     tail=tail, scale=scale, fp8=fp8fmt),
        "tensors": tensors,
    }


def read_file(path) -> Dict[str, object]:
    with open(path, "rb") as fh:
        return read(fh.read())
