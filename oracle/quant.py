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

import math

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
    return e4m3_round_t(torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))).numpy()


def e4m3_round_t(x: torch.Tensor) -> torch.Tensor:
    """Round float32 values to the nearest E4M3 value (RNE, saturating), on float32 bit patterns.

    Normal E4M3 range (|x| >= 2^-6): keep 3 of the 23 mantissa bits, round half to even on the
    bit pattern (a carry out of the mantissa steps the exponent, as RNE requires).  Below 2^-6 the
    quantum is fixed at 2^-9: x * 2^9 is exact, torch.round is half to even.  Then saturate to
    +-448 (values from 464 up would round to the NaN code 0x7F).
    """
    x = x.detach().to(torch.float32).cpu()
    x = torch.clamp(x, -1024.0, 1024.0).contiguous()    # keeps the bit arithmetic below float32 max
    bits = x.view(torch.int32)
    bias = ((bits >> 20) & 1) + 0x7FFFF
    normal = ((bits + bias) & ~0xFFFFF).view(torch.float32)
    sub = torch.round(x * 512.0) / 512.0
    out = torch.where(x.abs() < 2.0 ** -6, sub, normal)
    out = torch.clamp(out, -E4M3_MAX, E4M3_MAX)
    return torch.where(torch.isnan(x), x, out)


def e4m3_round_by_quantum(x) -> np.ndarray:
    """Second, independent formulation of e4m3_round (binade quantum from log2, float64), used
    to cross-check the bit-pattern version."""
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


def f16(x: torch.Tensor) -> torch.Tensor:
    """Round to FP16 (RNE) and return float32."""
    return x.to(torch.float16).to(torch.float32)


def quantize_s8(v: torch.Tensor, inv_scale: float) -> torch.Tensor:
    """clamp(rint(v * inv_scale), -127, 127) in float32 arithmetic (int8_kernels.cuh:2-4)."""
    prod = (v.to(torch.float32) * torch.tensor(inv_scale, dtype=torch.float32))
    return torch.clamp(torch.round(prod), -127, 127)   # torch.round: half to even


def round_f32(s: torch.Tensor, err: torch.Tensor) -> torch.Tensor:
    """float32 RNE of the exact value s + err, where s is float64 and |err| <= ulp64(s)/2.

    Rounding s alone is right unless s sits exactly on a float32 midpoint and
    err breaks the tie (the float64 sum already rounded once); then the exact
    value lies on err's side of the midpoint.
    """
    r = s.to(torch.float32)
    r64 = r.to(torch.float64)
    up = torch.nextafter(r, torch.full_like(r, math.inf))
    dn = torch.nextafter(r, torch.full_like(r, -math.inf))
    at_up_mid = s == (r64 + up.to(torch.float64)) / 2
    at_dn_mid = s == (r64 + dn.to(torch.float64)) / 2
    r = torch.where(at_up_mid & (err > 0), up, r)
    return torch.where(at_dn_mid & (err < 0), dn, r)


def fmaf(a: torch.Tensor, b, c) -> torch.Tensor:
    """float32 fused multiply-add a*b + c with one rounding (C fmaf / v_fma_f32).

    a*b of two float32 values is exact in float64 (48 significant bits); the
    float64 sum with c is split into its rounded value and exact error
    (Knuth's TwoSum) so that the final float32 rounding is the correct one.
    """
    a64 = torch.as_tensor(a, dtype=torch.float32).to(torch.float64)
    b64 = torch.as_tensor(b, dtype=torch.float32).to(torch.float64)
    c64 = torch.as_tensor(c, dtype=torch.float32).to(torch.float64)
    p = a64 * b64
    c64 = c64.expand_as(p)
    s = p + c64
    r = s.to(torch.float32)
    # Only a float64 sum lying exactly on a float32 midpoint can round the wrong way: its low
    # 29 mantissa bits are 1 followed by 28 zeros (float32-normal range; smaller values take the
    # general path too).
    mid = (s.contiguous().view(torch.int64) & 0x1FFFFFFF) == 0x10000000
    mid |= (s != 0) & (s.abs() < 2.0 ** -125)
    if bool(mid.any()):
        sm, pm, cm = s[mid], p[mid], c64[mid]
        bb = sm - pm
        err = (pm - (sm - bb)) + (cm - bb)
        r = r.clone()
        r[mid] = round_f32(sm, err)
    return r
