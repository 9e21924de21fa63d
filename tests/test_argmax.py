"""The engine's greedy choice (sl_engine_first_argmax, host code, no GPU):
the first index of the largest value with strict >, exactly as one
sequential scan from index 0 gives it, including NaNs (never taken past
index 0; a NaN at index 0 is kept) and -inf."""
import ctypes

import numpy as np
import pytest

from starlight_amd import device as dev


def scan(v):
    best, bv = 0, v[0]
    for j in range(1, len(v)):
        if v[j] > bv:
            best, bv = j, v[j]
    return best


def argmax(v):
    lib = dev.load_library()
    fn = lib.sl_engine_first_argmax
    fn.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_size_t]
    fn.restype = ctypes.c_uint32
    a = np.ascontiguousarray(v, np.float32)
    return int(fn(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), a.size))


def test_nan_at_a_lane_start_does_not_hide_the_block_maximum():
    # blocks of 256 reduced over 16 lanes: index 256 starts lane 0 of the
    # second block; the true maximum sits later in the same lane
    v = np.zeros(1024, np.float32)
    v[256] = np.nan
    v[256 + 16 * 5] = 3.0
    assert argmax(v) == scan(v) == 256 + 80


def test_nan_first_is_kept_and_later_nans_are_skipped():
    v = np.arange(600, dtype=np.float32)
    v[0] = np.nan
    assert argmax(v) == scan(v) == 0
    v = np.arange(600, dtype=np.float32)
    v[599] = np.nan
    assert argmax(v) == scan(v) == 598


@pytest.mark.parametrize("n", [1, 2, 255, 256, 257, 511, 4096 + 17, 32000])
def test_matches_the_sequential_scan(n):
    r = np.random.default_rng(n)
    for trial in range(20):
        v = r.standard_normal(n).astype(np.float32)
        if trial % 3 == 0:
            v[r.integers(0, n, max(1, n // 50))] = np.nan
        if trial % 4 == 1:
            v[r.integers(0, n, max(1, n // 50))] = np.float32(np.max(v[~np.isnan(v)]) if np.any(~np.isnan(v)) else 1)
        if trial % 5 == 2:
            v[:] = -np.inf
            v[r.integers(0, n)] = np.inf if n > 1 else -np.inf
        assert argmax(v) == scan(v), trial
