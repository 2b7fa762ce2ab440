"""Number-format emulation for the FP8 / INT8 deployments -- TEST INFRASTRUCTURE ONLY.

* OCP FP8 E4M3 ("e4m3fn"): 1 sign, 4 exponent (bias 7), 3 mantissa bits,
  no infinities, code 0x7F/0xFF = NaN, largest finite 448.  The reference
  converts with saturate-to-finite, round-to-nearest-even
  (``__nv_fp8_e4m3(float)``, used in
  optimized/native/src/neural/srcpyr/SrcPyrNativeFp8Compress.cuh:104-105,233-235).
  The encoder here follows the OCP 8-bit floating point specification v1.0
  directly: scale to the binade quantum, round half to even, saturate.
* Symmetric INT8 (optimized/shader/src/int8_kernels.cuh:2-4):
  q = clamp(rint(v * inv_scale), -127, 127) with rint = round half to even.

Pinning: the E4M3 decoder is checked against the artifact's codes times
``weight_scale`` versus the FP32 checkpoint, the encoder against the decoder
over every code and every midpoint between adjacent codes (ties must land on
the even code), and both against ``torch.float8_e4m3fn`` for in-range values.
"""
from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0


def e4m3_decode_table() -> np.ndarray:
    """float32 value of each of the 256 codes (NaN for 0x7F, 0xFF)."""
    out = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * man * 2.0 ** -9
        else:
            out[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return out


_DECODE = e4m3_decode_table()


def e4m3_decode(codes) -> np.ndarray:
    return _DECODE[np.asarray(codes, dtype=np.uint8)]


def e4m3_round(x) -> np.ndarray:
    """Round float32 values to the nearest E4M3 value (RNE, saturating). Returns float32."""
    v = np.asarray(x, dtype=np.float32).astype(np.float64)
    mag = np.abs(v)
    # exponent of the binade, floor(log2|v|), subnormal range pinned at -6
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where((mag > 0) & np.isfinite(mag), mag, 1.0)))
    e = np.maximum(e, -6.0)
    quantum = np.exp2(e - 3.0)
    q = np.round(mag / quantum) * quantum        # np.round is half-to-even; division exact
    q = np.minimum(q, E4M3_MAX)
    q = np.where(np.isinf(mag), E4M3_MAX, q)      # SATFINITE: +-inf -> +-448
    out = np.copysign(q, v)
    out = np.where(np.isnan(v), np.nan, out)
    return out.astype(np.float32)


def e4m3_encode(x) -> np.ndarray:
    """Codes (uint8) of e4m3_round(x)."""
    r = e4m3_round(x)
    table = _DECODE[:0x7F]                       # positive finite codes 0..126 (monotone)
    mag = np.abs(r)
    codes = np.searchsorted(table, mag).astype(np.uint8)
    codes = np.where(np.signbit(r), codes | 0x80, codes).astype(np.uint8)
    return np.where(np.isnan(r), np.uint8(0x7F), codes).astype(np.uint8)


def e4m3_round_t(x: torch.Tensor) -> torch.Tensor:
    """Torch wrapper of e4m3_round (CPU)."""
    return torch.from_numpy(e4m3_round(x.detach().cpu().numpy().astype(np.float32)))


def f16(x: torch.Tensor) -> torch.Tensor:
    """Round to FP16 (RNE) and return float32."""
    return x.to(torch.float16).to(torch.float32)


def quantize_s8(v: torch.Tensor, inv_scale: float) -> torch.Tensor:
    """clamp(rint(v * inv_scale), -127, 127) in float32 arithmetic (int8_kernels.cuh:2-4)."""
    prod = (v.to(torch.float32) * torch.tensor(inv_scale, dtype=torch.float32))
    return torch.clamp(torch.round(prod), -127, 127)   # torch.round: half to even


def fmaf(a: torch.Tensor, b, c) -> torch.Tensor:
    """float32 fused multiply-add emulated in float64 (one rounding to float32)."""
    a64 = a.to(torch.float64)
    b64 = torch.as_tensor(b, dtype=torch.float32).to(torch.float64)
    c64 = torch.as_tensor(c, dtype=torch.float32).to(torch.float64)
    return (a64 * b64 + c64).to(torch.float32)
