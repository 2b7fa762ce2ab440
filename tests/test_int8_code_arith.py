"""The INT8 code arithmetic of the fused body (common.hpp s8_code_word, pack_low_bytes4), restated
in float32 numpy and checked against the definition it replaces, quant_s8 = clamp(rint(x), -127, 127)
with rint rounding half to even (the reference's quantize_s8, optimized/shader/src/int8_kernels.cuh:2-4).

The device computes fmed3(x, -127, 127) + 1.5 * 2^23 in FP32 and keeps the low byte of the sum's bit
pattern.  numpy's float32 addition rounds to nearest even like v_add_f32, so the restatement is the
device arithmetic.  Inputs: every float32 pattern whose low 11 mantissa bits are zero in [-300, 300],
every half-integer k + 0.5 and its two float32 neighbours for |k| <= 300, signed zeros, subnormals and
infinities.  A planted variant that rounds half away from zero must fail.
"""
import numpy as np

MAGIC = np.float32(12582912.0)          # 1.5 * 2^23


def _inputs() -> np.ndarray:
    lim = np.float32(300.0)
    hi = int(np.array(lim, np.float32).view(np.uint32))
    pos = (np.arange(0, hi + 1, 2048, dtype=np.uint64).astype(np.uint32)).view(np.float32)
    halves = np.arange(-300, 301, dtype=np.float32) + np.float32(0.5)
    near = np.concatenate([np.nextafter(halves, np.float32(np.inf)), np.nextafter(halves, np.float32(-np.inf)), halves])
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 1.1754942e-38, 126.5, 127.5, -127.5, 128.0],
                       dtype=np.float32)
    x = np.concatenate([pos, -pos, near, special]).astype(np.float32)
    return x


def _reference_codes(x: np.ndarray) -> np.ndarray:
    q = np.clip(np.rint(x.astype(np.float64)), -127, 127).astype(np.int64)   # rint: half to even
    return (q & 0xFF).astype(np.uint8)


def _device_codes(x: np.ndarray, magic: np.float32 = MAGIC) -> np.ndarray:
    clamped = np.minimum(np.maximum(x, np.float32(-127.0)), np.float32(127.0)).astype(np.float32)
    s = (clamped + magic).astype(np.float32)
    return (s.view(np.uint32) & 0xFF).astype(np.uint8)


def _pack_low_bytes4(a, b, c, d) -> np.ndarray:
    """v_perm_b32(b, a, 0x0c0c0400) | v_perm_b32(d, c, 0x04000c0c): low bytes a..d into bytes 0..3."""
    lo = (a & 0xFF) | ((b & 0xFF) << 8)
    hi = ((c & 0xFF) << 16) | ((d & 0xFF) << 24)
    return (lo | hi).astype(np.uint32)


def test_magic_add_equals_clamped_rint():
    x = _inputs()
    assert x.size > 1_000_000
    np.testing.assert_array_equal(_device_codes(x), _reference_codes(x))


def test_word_is_biased_twos_complement():
    """The whole sum is 0x4B400000 + q, so the low byte is q in two's complement."""
    x = np.arange(-127, 128, dtype=np.float32)
    s = (x + MAGIC).astype(np.float32).view(np.uint32).astype(np.int64)
    np.testing.assert_array_equal(s - 0x4B400000, np.arange(-127, 128))


def test_packing_matches_pack_s8x4():
    rng = np.random.default_rng(7)
    q = rng.integers(-127, 128, size=(4, 1000))
    words = [(np.float32(v) + MAGIC).astype(np.float32).view(np.uint32) for v in q.astype(np.float32)]
    packed = _pack_low_bytes4(*[w.astype(np.uint64) for w in words])
    expect = ((q[0] & 255) | ((q[1] & 255) << 8) | ((q[2] & 255) << 16) | ((q[3] & 255) << 24)).astype(np.uint32)
    np.testing.assert_array_equal(packed, expect)


def test_planted_half_away_rounding_is_caught():
    x = _inputs()
    away = (np.clip(np.sign(x) * np.floor(np.abs(x.astype(np.float64)) + 0.5), -127, 127).astype(np.int64) & 0xFF)
    assert (away.astype(np.uint8) != _device_codes(x)).any()
