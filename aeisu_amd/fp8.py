"""OCP FP8 E4M3 ("e4m3fn") codec used by the artifact writer and the calibrator.

Format: 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities, 0x7F/0xFF are
NaN, largest finite 448 (code 0x7E), subnormal quantum 2^-9.  Encoding rounds to
nearest even and saturates to +-448, the conversion the reference deployment uses for
its weights and activations (`__nv_fp8_e4m3(float)`, SATFINITE; the artifact's codes
of optimized/native/weights/adaptive_fp8.bin decode with this table).

The encoder works on the float32 bit pattern: normal values round their 23-bit
mantissa to 3 bits with a round-half-even bias, subnormal values (|x| < 2^-6) are
integer multiples of 2^-9 rounded with numpy's half-even rint.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def _decode_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for code in range(256):
        e, m = (code >> 3) & 0xF, code & 0x7
        mag = m * 2.0 ** -9 if e == 0 else (1.0 + m / 8.0) * 2.0 ** (e - 7)
        t[code] = -mag if code & 0x80 else mag
    t[0x7F] = t[0xFF] = np.nan
    return t


DECODE = _decode_table()


def decode(codes) -> np.ndarray:
    """uint8 codes -> float32 values."""
    return DECODE[np.asarray(codes, dtype=np.uint8)]


def encode(x) -> np.ndarray:
    """float values -> uint8 E4M3 codes (round to nearest even, saturate to +-448, NaN -> 0x7F)."""
    v = np.asarray(x, dtype=np.float32)
    bits = v.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    mag_bits = bits & np.uint32(0x7FFFFFFF)
    mag = mag_bits.view(np.float32)
    # normal range: keep 3 mantissa bits, round half to even on the 20 dropped bits
    lsb = (mag_bits >> 20) & np.uint32(1)
    rounded = (mag_bits + np.uint32(0x7FFFF) + lsb) & np.uint32(0xFFF00000)
    exp = (rounded >> 23).astype(np.int64) - 127 + 7
    man = ((rounded >> 20) & np.uint32(7)).astype(np.int64)
    normal_code = (exp << 3) | man
    # subnormal range: multiples of 2^-9 (q = 8 is the smallest normal, code 0x08)
    with np.errstate(invalid="ignore", over="ignore"):          # NaN / inf lanes are replaced below
        sub_code = np.rint(np.minimum(mag.astype(np.float64), 1.0) * 512.0).astype(np.int64)
    code = np.where(mag < 2.0 ** -6, sub_code, normal_code)
    code = np.where(code > 0x7E, 0x7E, code)                 # saturate (also catches +inf)
    out = code.astype(np.uint8) | sign
    return np.where(np.isnan(v), np.uint8(0x7F), out).astype(np.uint8)


def round_e4m3(x) -> np.ndarray:
    """Nearest E4M3 value as float32."""
    return decode(encode(x))
