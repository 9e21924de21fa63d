"""The group-wise quantization convention (no reference code exists for it:
sl-precision is absent, so the layout is parity-unpinned against it).

Pinned here by: hand-computed known answers, the closed-form round-trip bound
|w - dequant| <= scale / 2, the special cases (all-zero group, the largest
magnitude maps to +-qmax exactly, half-way rounding away from zero), and
bit-exact agreement between two independent implementations — the numpy
product quantizer and the C oracle.
"""
import numpy as np
import pytest

import oracle
from starlight_amd import quant
from starlight_amd.ir import QuantFormat


def test_int4_and_int8_known_answer():
    # amax = 7 -> scale 1; 3.5 rounds half away to 4; -1.4 -> -1.
    w = np.array([[7.0, -7.0, 3.5, -1.4]], np.float32)
    words, scales = quant.quantize(w, 4, QuantFormat.INT4)
    assert scales.tolist() == [[1.0]]
    # nibbles: 7 -> 0x7, -7 -> 0x9, 4 -> 0x4, -1 -> 0xF; bytes 0x97, 0xF4
    assert words.tolist() == [0x0000F497]
    w8 = np.array([[127.0, -127.0, 63.5, -25.4]], np.float32)
    words8, scales8 = quant.quantize(w8, 4, QuantFormat.INT8)
    assert scales8.tolist() == [[1.0]]
    assert words8.tolist() == [0xE740_817F]  # bytes 0x7F, 0x81, 0x40, 0xE7


def test_half_way_rounding_is_away_from_zero():
    v = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 0.49999997, -0.49999997], np.float32)
    assert quant.round_half_away(v).tolist() == [1, -1, 2, -2, 3, -3, 0, 0]


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
def test_special_cases(fmt):
    qmax = quant.QMAX[fmt]
    w = np.zeros((3, 256), np.float32)
    w[1, :128] = np.linspace(-0.3, 0.2, 128)
    w[2, 130] = -5.0
    words, scales = quant.quantize(w, 128, fmt)
    codes = quant.unpack_codes(words, 3, 256, fmt)
    assert np.all(scales[0] == 0) and np.all(codes[0] == 0)          # all-zero groups
    assert np.all(codes[1, 128:] == 0) and scales[1, 1] == 0
    assert codes[1, 0] == -qmax                                       # max |w| -> -qmax exactly
    assert codes[2, 130] == -qmax and np.count_nonzero(codes[2]) == 1
    assert np.all(np.abs(codes) <= qmax)                              # never -8 / -128


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
@pytest.mark.parametrize("n,k,group", [(1, 128, 128), (5, 256, 64), (7, 384, 128), (3, 34, 2)])
def test_numpy_and_c_oracle_agree_bit_exactly(fmt, n, k, group):
    rng = np.random.default_rng(n * 1000 + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    words, scales = quant.quantize(w, group, fmt)
    bits = 4 if fmt == QuantFormat.INT4 else 8
    payload, oscales = oracle.quantize_groupwise(w, n, k, group, bits)
    assert np.array_equal(scales, oscales)
    raw = words.view(np.uint8)[: payload.size]
    assert np.array_equal(raw, payload.ravel())
    assert np.array_equal(quant.unpack_codes(words, n, k, fmt), oracle.unpack_codes(payload, n, k, bits))
    assert np.array_equal(quant.dequantize(words, scales, n, k, group, fmt),
                          oracle.dequantize_groupwise(payload, oscales, n, k, group, bits))


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
def test_round_trip_error_is_at_most_half_a_step(fmt):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    words, scales = quant.quantize(w, 128, fmt)
    back = quant.dequantize(words, scales, 64, 512, 128, fmt)
    step = np.repeat(scales, 128, axis=1)
    assert np.all(np.abs(back.astype(np.float64) - w) <= step * 0.5 * (1 + 1e-6))


def test_every_int4_code_round_trips_through_the_packing():
    codes = np.arange(-8, 8, dtype=np.int8).reshape(2, 8)
    words = quant.pack_codes(codes, QuantFormat.INT4)
    assert np.array_equal(quant.unpack_codes(words, 2, 8, QuantFormat.INT4), codes)
    raw = words.view(np.uint8)
    assert raw[0] == ((-7 & 0xF) << 4 | (-8 & 0xF)) and raw[7] == (7 << 4 | 6)
