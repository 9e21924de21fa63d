"""The device's dequantized weights, bit for bit.

Every quantized MatMulNT path reads the private tile copy the device builds
at bind time, and unpacking and dequantization must be bit-exact against
the oracle. An activation row that is a unit vector e_k makes each kernel
return column k of its dequantized weight, and on every path that column is
exact:

 * decode GEMVs (m <= 16): x = 1.0 becomes the integer X = 2^21 (three int8
   limbs 0, 0, 32), the limb-times-code products are exact in i32, and the
   group's f32 combination is q * 2^25 (INT4 operands are 16 q) times a
   power of two, then one fma with the scale: q * s rounded once, plus
   exact zeros from every other group;
 * the prefill GEMM (m > 16): hi = 2^14 and lo = 0, so hi * q is exact in
   fp16 products with f32 sums, times the scale (one rounding), times the
   power of two 2^-14;
 * the VALU fallbacks of the row-major layout: q * 1.0 summed with zeros,
   times the scale.

So MatMulNT(I_K[k0:k0+m], W) through the C ABI, for k0 = 0, m, 2m, ...,
writes W' transposed, and it must equal oracle.dequantize_groupwise
(f32(q) * s, one multiply) exactly. The weights are ~N(0, 0.02), quantized
by the oracle's C routine (bit-identical to starlight_amd.quant, pinned in
tests/test_quant.py).

Which kernels the m values reach (launch_qmatmul, launch_qgemv_fused):
k = 4096: m = 1, 4 the fused GEMV with all limbs in one MFMA row block;
m = 8 the fused GEMV with one MFMA per limb; m = 16 the k-sliced fused GEMV
plus the slice sum; m = 512 the activation split and the fp16 matrix-core
GEMM. k = 14336: m = 1 the fused GEMV with 16 waves; m = 4 the split-K
matrix-core GEMV and its reduction; m = 8, 16 the k-sliced fused GEMV;
m = 512 the matrix-core GEMM with k cut into slices. The small shapes reach
the matrix-core GEMV for k not a multiple of 256, a partial last tile, and
the row-major layout's VALU GEMV and tiled GEMM.
"""
import numpy as np
import pytest

import oracle
from starlight_amd.ir import BufferRef, Op, QuantFormat, Value

pytestmark = pytest.mark.gpu

_IDENTITY = {}  # k -> (device, buffer) of I_k
_OUT = {}       # element count -> (device, buffer, host NaN fill)


def identity(hip, k):
    hit = _IDENTITY.get(k)
    if hit is None or hit[0] is not hip:
        hit = (hip, hip.upload_new_f32(np.eye(k, dtype=np.float32)))
        _IDENTITY[k] = hit
    return hit[1]


def out_buffer(hip, count):
    """An output buffer of `count` floats, refilled with NaN on every call
    so that an element no launch writes cannot pass."""
    hit = _OUT.get(count)
    if hit is None or hit[0] is not hip:
        hit = (hip, hip.allocate_f32(count, 256), np.full(count, np.nan, np.float32))
        _OUT[count] = hit
    hip.upload_f32(hit[1], hit[2])
    return hit[1]


def bound_weight(hip, n, k, fmt, group, seed):
    """Quantizes w ~N(0, 0.02) [n, k], uploads and binds it; returns the
    payload's BufferRef, its Value and the oracle's dequantized [n, k]."""
    bits = 4 if fmt == QuantFormat.INT4 else 8
    w = (np.random.default_rng(seed).standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    payload, scales = oracle.quantize_groupwise(w, n, k, group, bits)
    raw = payload.reshape(-1)
    raw = np.concatenate([raw, np.zeros((-raw.size) % 4, np.uint8)])
    words = raw.view("<u4").astype(np.uint32)
    pb = hip.upload_new_u32(words)
    sb = hip.upload_new_f32(scales)
    hip.bind_quantized(pb, sb, fmt, group, n, k)
    deq = oracle.dequantize_groupwise(payload, scales, n, k, group, bits)
    return BufferRef(pb, 0, words.size), Value.quantized([n, k], fmt, group), deq


def dequantized_columns(hip, wref, wval, n, k, m):
    """W' transposed [k, n], one MatMulNT of m unit rows per dispatch."""
    eye, out = identity(hip, k), out_buffer(hip, k * n)
    assert k % m == 0
    for k0 in range(0, k, m):
        hip.dispatch(Op.matmul_nt(), [BufferRef(eye, k0 * k, m * k), wref],
                     [Value.f32([1, m, k]), wval], [BufferRef(out, k0 * n, m * n)], [Value.f32([1, m, n])])
    return hip.read_f32(out, k * n).reshape(k, n)


def assert_bit_exact(got, want, what):
    bad = np.argwhere(got != want)
    assert bad.size == 0, (f"{what}: {len(bad)} elements differ, first at column {bad[0][0]}, row {bad[0][1]}: "
                           f"{got[tuple(bad[0])]!r} vs {want[tuple(bad[0])]!r}")


@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
def test_dequantized_weights_bit_exact_at_benchmark_shapes(hip, n, k, fmt, group):
    wref, wval, deq = bound_weight(hip, n, k, fmt, group, seed=n + k + group + int(fmt))
    want = np.ascontiguousarray(deq.T)
    assert np.count_nonzero(want) > 0.8 * want.size
    for m in (1, 4, 8, 16, 512):
        got = dequantized_columns(hip, wref, wval, n, k, m)
        assert_bit_exact(got, want, f"m={m}")


@pytest.mark.parametrize("m", [1, 16, 64])
@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
@pytest.mark.parametrize("n,k,group", [(300, 384, 128),   # tile layout, k % 256 != 0, partial last tile
                                       (200, 192, 64),    # row-major layout (k % 128 != 0)
                                       (136, 256, 32)])   # row-major layout (group below 64)
def test_dequantized_weights_bit_exact_other_layouts(hip, n, k, group, fmt, m):
    wref, wval, deq = bound_weight(hip, n, k, fmt, group, seed=n + k + m)
    got = dequantized_columns(hip, wref, wval, n, k, m)
    assert_bit_exact(got, np.ascontiguousarray(deq.T), f"m={m}")
