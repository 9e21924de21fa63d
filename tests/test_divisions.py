"""The q-GEMV's multiply-shift divisions are exact over the ranges its
launcher lets through (starlight_amd/csrc/kernels/qgemv_fused.hip, Args and
magic16 / run4_of): checked exhaustively against integer division.

The kernel replaces run-time divisions by per-launch values with
  n / d == (n * ceil(2^16 / d)) >> 16          (32-bit product)
  f / r == mulhi32(f, ceil(2^32 / r))
and the launcher bounds every numerator and divisor:
  * i / len, i a lane index (< 64), len = superblocks per wave (<= 64);
  * e / m, e an output element of a block (< 4096 = per_cap * 16 * m), m <= 16;
  * run / (k / 256), run = float4 index / 64 (< 128, m * k <= 32768), k / 256 <= 128;
  * f / run4, f a launch-time scale float4 (< 16384), run4 = 4 * sb_total * gps >= 8.
"""
import numpy as np


def magic16(d):
    return (65536 + d - 1) // d


def test_magic16_lane_over_len():
    n = np.arange(64, dtype=np.uint64)
    for d in range(1, 65):
        assert np.array_equal((n * magic16(d)) >> 16, n // d), d


def test_magic16_element_over_m():
    e = np.arange(4096, dtype=np.uint64)
    for m in range(1, 17):
        assert np.array_equal((e * magic16(m)) >> 16, e // m), m


def test_magic16_run_over_k256():
    run = np.arange(128, dtype=np.uint64)
    for d in range(1, 129):
        assert np.array_equal((run * magic16(d)) >> 16, run // d), d


def test_magic16_products_fit_32_bits():
    # the kernel multiplies in 32-bit registers
    assert 63 * magic16(1) < 2**32 and 4095 * magic16(1) < 2**32 and 127 * magic16(1) < 2**32


def test_mulhi_scale_run():
    f = np.arange(16384, dtype=np.uint64)
    for r in range(8, 4097):
        mg = ((1 << 32) + r - 1) // r
        assert mg < 2**32
        assert np.array_equal((f * mg) >> 32, f // r), r


def test_magic16_fails_outside_the_ranges():
    # the bounds are needed: one more row (m = 17) breaks e / m at e = 4096,
    # and a numerator past 2^15 breaks d = 3
    assert ((4096 * magic16(17)) >> 16) != 4096 // 17
    assert ((32768 * magic16(3)) >> 16) != 32768 // 3
