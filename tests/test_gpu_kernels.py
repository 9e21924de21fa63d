"""GPU-vs-oracle parity of every operator at sizes beyond the reference's
unit tests: unaligned offsets, non-multiple-of-4 widths, the generic and the
vectorised kernel paths, decode/prefill attention, broadcast matmuls, and
group-quantized weights at the benchmark's shapes.

Inputs are seeded (numpy Generator or the reference LCG); expectations come
from the C oracle on the same inputs.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import assert_elementwise, assert_normwise, rel_l2
from starlight_amd import quant
from starlight_amd.device import DeviceError
from starlight_amd.ir import BufferRef, Op, QuantFormat, RopeVariant, Value, ValueRole

pytestmark = pytest.mark.gpu


def put(hip, data, pad=0):
    """Uploads `data` after `pad` leading zeros; returns (buffer, BufferRef)."""
    a = np.ascontiguousarray(data, dtype=np.float32).ravel()
    buf = hip.upload_new_f32(np.concatenate([np.zeros(pad, np.float32), a]))
    return buf, BufferRef(buf, pad, a.size)


def put_u32(hip, data):
    a = np.ascontiguousarray(data, dtype=np.uint32).ravel()
    buf = hip.upload_new_u32(a)
    return buf, BufferRef(buf, 0, a.size)


def out_buf(hip, n, pad=0):
    buf = hip.allocate_f32(n + pad, 256)
    return buf, BufferRef(buf, pad, n)


def read(hip, ref):
    full = hip.read_f32(ref.buffer, ref.offset + ref.len)
    return full[ref.offset:]


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------ elementwise --


@pytest.mark.parametrize("n,pad", [(1, 0), (7, 1), (33, 0), (4096, 0), (4099, 3), (1_000_003, 2)])
def test_elementwise_parity(hip, n, pad):
    r = rng(n)
    a = r.standard_normal(n).astype(np.float32) * 4
    b = r.standard_normal(n).astype(np.float32)
    _, ar = put(hip, a, pad)
    _, br = put(hip, b, 0)
    _, orf = out_buf(hip, n, pad)
    v = Value.f32([n])
    hip.dispatch(Op.add(), [ar, br], [v, v], [orf], [v])
    assert np.array_equal(read(hip, orf), oracle.add(a, b, n))
    hip.dispatch(Op.mul(), [ar, br], [v, v], [orf], [v])
    assert np.array_equal(read(hip, orf), oracle.mul(a, b, n))
    hip.dispatch(Op.scale_by(0.37), [ar], [v], [orf], [v])
    assert np.array_equal(read(hip, orf), oracle.scale(a, 0.37))
    hip.dispatch(Op.silu(), [ar], [v], [orf], [v])
    assert_elementwise(read(hip, orf), oracle.silu(a))


def test_silu_extremes(hip):
    x = np.array([-100.0, -10.0, 0.0, 10.0, 100.0, -88.7, 88.7, 1e-30], np.float32)
    _, xr = put(hip, x)
    _, orf = out_buf(hip, x.size)
    v = Value.f32([x.size])
    hip.dispatch(Op.silu(), [xr], [v], [orf], [v])
    assert_elementwise(read(hip, orf), oracle.silu(x))


# ------------------------------------------------------------------- norm --


@pytest.mark.parametrize("rows,hidden,pad", [(1, 1, 0), (3, 7, 1), (4, 16, 0), (2, 33, 0), (64, 4096, 0),
                                             (5, 5000, 0), (3, 8192, 0), (2, 12000, 0), (7, 256, 2)])
def test_rms_norm_parity(hip, rows, hidden, pad):
    r = rng(rows * 7 + hidden)
    x = r.standard_normal(rows * hidden).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(hidden)).astype(np.float32)
    _, xr = put(hip, x, pad)
    _, wr = put(hip, w)
    _, orf = out_buf(hip, rows * hidden, pad)
    hip.dispatch(Op.rms_norm(1e-5), [xr, wr], [Value.f32([rows, hidden]), Value.f32([hidden], ValueRole.PARAM)],
                 [orf], [Value.f32([rows, hidden])])
    got = read(hip, orf).reshape(rows, hidden)
    want = oracle.rms_norm(x, w, rows, hidden, 1e-5).reshape(rows, hidden)
    for i in range(rows):
        assert_normwise(got[i], want[i])


# ---------------------------------------------------------------- softmax --


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (6, 17), (64, 2048), (4, 3000), (2, 9000)])
def test_softmax_parity(hip, rows, cols):
    x = rng(rows + cols).standard_normal(rows * cols).astype(np.float32) * 3
    _, xr = put(hip, x)
    _, orf = out_buf(hip, x.size)
    v = Value.f32([rows, cols])
    hip.dispatch(Op.softmax(), [xr], [v], [orf], [v])
    got = read(hip, orf).reshape(rows, cols)
    want = oracle.softmax(x, rows, cols).reshape(rows, cols)
    for i in range(rows):
        assert_normwise(got[i], want[i])


@pytest.mark.parametrize("rows,seq,past", [(2, 2, 0), (12, 4, 1), (4, 1, 7), (6, 3, 2), (64, 32, 100),
                                           (8, 2, 9000), (16, 8, 4088)])
def test_softmax_causal_parity(hip, rows, seq, past):
    cols = past + seq
    x = rng(rows * 3 + past).standard_normal(rows * cols).astype(np.float32) * 3
    _, xr = put(hip, x)
    _, orf = out_buf(hip, x.size)
    v = Value.f32([rows, cols])
    hip.dispatch(Op.softmax_causal(), [xr], [v], [orf], [v], [seq, past])
    got = read(hip, orf).reshape(rows, cols)
    want = oracle.softmax_causal(x, rows, cols, seq, past).reshape(rows, cols)
    for i in range(rows):
        assert_normwise(got[i], want[i])
        assert np.all(got[i][want[i] == 0] == 0)


# ------------------------------------------------------------------- rope --


@pytest.mark.parametrize("variant", [RopeVariant.NEOX, RopeVariant.GPTJ])
@pytest.mark.parametrize("batch,heads,seq,hd,theta,rank3", [
    (1, 1, 1, 2, 10_000.0, False), (2, 3, 5, 4, 10_000.0, False), (2, 2, 4, 8, 500_000.0, False),
    (1, 2, 3, 10, 1_000_000.0, False), (1, 32, 512, 128, 500_000.0, False), (2, 1, 17, 64, 10_000.0, True),
    (1, 8, 3, 128, 500_000.0, False), (1, 1, 2, 128, 500_000.0, False), (1, 40, 2, 256, 10_000.0, False)])
def test_rope_parity(hip, variant, batch, heads, seq, hd, theta, rank3):
    r = rng(batch * 100 + seq)
    x = r.uniform(-2, 2, batch * heads * seq * hd).astype(np.float32)
    pos = (np.arange(batch * seq) * 3 + r.integers(0, 5, batch * seq)).astype(np.uint32)
    if seq == 3:
        pos = pos + 4090  # near the end of a 4096-position context
    _, xr = put(hip, x)
    _, pr = put_u32(hip, pos)
    _, orf = out_buf(hip, x.size)
    shape = [batch, seq, hd] if rank3 else [batch, heads, seq, hd]
    hip.dispatch(Op.rope(variant, theta), [xr, pr], [Value.f32(shape), Value.u32([batch, seq])], [orf],
                 [Value.f32(shape)])
    want = oracle.rope(x, pos, batch, heads, seq, hd, theta, "neox" if variant == RopeVariant.NEOX else "gptj")
    assert_elementwise(read(hip, orf), want)


# ----------------------------------------------------------------- layout --


# rows of one pass (<= 1024 float4 or floats per 256 threads), of several,
# and of a pass that ends inside a thread's four loads
@pytest.mark.parametrize("vocab,hidden,rows", [(10, 5, 3), (1, 1, 1), (4, 7, 0), (13, 9, 6), (1000, 4096, 37),
                                               (20, 2048, 4), (50, 8192, 3), (9, 6000, 2), (7, 1025, 2),
                                               (5, 4099, 3)])
def test_gather_parity(hip, vocab, hidden, rows):
    r = rng(vocab + rows)
    table = r.standard_normal(vocab * hidden).astype(np.float32)
    ids = r.integers(0, vocab, rows).astype(np.uint32)
    _, tr = put(hip, table)
    ib = hip.allocate_u32(max(rows, 1), 256)
    if rows:
        hip.upload_u32(ib, ids)
    _, orf = out_buf(hip, rows * hidden)
    hip.dispatch(Op.gather(), [tr, BufferRef(ib, 0, rows)],
                 [Value.f32([vocab, hidden], ValueRole.PARAM), Value.u32([rows])], [orf],
                 [Value.f32([rows, hidden])]) if rows else None
    if rows:
        assert np.array_equal(read(hip, orf), oracle.gather(table, ids, vocab, hidden, rows))


@pytest.mark.parametrize("batch,seq,hidden,seq_len", [(1, 1, 3, 1), (3, 5, 4, 5), (2, 4, 7, 2), (2, 64, 4096, 40),
                                                     (1, 1, 4096, 1), (1, 1, 2048, 1), (2, 3, 8192, 3),
                                                     (3, 2, 1030, 1), (2, 2, 6004, 2)])
def test_last_token_parity(hip, batch, seq, hidden, seq_len):
    x = rng(seq).standard_normal(batch * seq * hidden).astype(np.float32)
    _, xr = put(hip, x)
    _, orf = out_buf(hip, batch * hidden)
    hip.dispatch(Op.last_token(), [xr], [Value.f32([batch, seq, hidden])], [orf], [Value.f32([batch, hidden])],
                 [seq_len])
    assert np.array_equal(read(hip, orf), oracle.last_token(x, batch, seq, hidden, seq_len))


@pytest.mark.parametrize("batch,seq,heads,hd,pad", [(1, 1, 1, 2, 0), (2, 3, 4, 4, 0), (2, 5, 3, 6, 1),
                                                    (1, 4, 2, 8, 0), (1, 100, 32, 128, 0), (2, 7, 8, 128, 2)])
def test_split_merge_parity(hip, batch, seq, heads, hd, pad):
    x = rng(seq * heads).standard_normal(batch * seq * heads * hd).astype(np.float32)
    _, xr = put(hip, x, pad)
    _, sr = out_buf(hip, x.size, pad)
    _, mr = out_buf(hip, x.size)
    hip.dispatch(Op.split_heads(heads, hd), [xr], [Value.f32([batch, seq, heads * hd])], [sr],
                 [Value.f32([batch, heads, seq, hd])])
    split = read(hip, sr)
    assert np.array_equal(split, oracle.split_heads(x, batch, seq, heads, hd))
    hip.dispatch(Op.merge_heads(heads, hd), [sr], [Value.f32([batch, heads, seq, hd])], [mr],
                 [Value.f32([batch, seq, heads * hd])])
    assert np.array_equal(read(hip, mr), x)


# -------------------------------------------------------------- attention --

ATT_SHAPES = [
    # batch, layers, layer, heads, kv_heads, seq, past_len, head_dim, max_seq
    (1, 1, 0, 2, 2, 3, 0, 4, 4),
    (2, 1, 0, 2, 2, 1, 3, 8, 6),
    (2, 2, 1, 4, 2, 2, 2, 8, 5),
    (2, 1, 0, 2, 1, 1, 5, 2, 7),
    (1, 1, 0, 6, 3, 2, 1, 4, 4),
    (1, 1, 0, 3, 1, 1, 2, 4, 3),
    (1, 2, 1, 32, 8, 1, 1000, 128, 1100),   # 8B-shaped decode step
    (1, 1, 0, 32, 8, 1, 300, 64, 512),      # 1B-shaped decode step
    (1, 1, 0, 32, 8, 1, 1500, 64, 2048),    # 1B-shaped: 32 partials of 64 positions, 8-key tiles
    (1, 1, 0, 32, 8, 1, 3990, 64, 4096),    # head_dim 64 at 4096 positions: 64 partials, four per merge thread
    (8, 1, 0, 32, 8, 1, 77, 128, 128),      # batch-8 decode
    (1, 1, 0, 32, 8, 100, 0, 128, 128),     # prefill, tiled path
    (1, 2, 0, 32, 8, 70, 30, 64, 128),      # chunked prefill after a prefix, tiled path
    (2, 1, 0, 4, 4, 20, 5, 96, 32),         # prefill through the split path (head_dim 96)
    (1, 1, 0, 4, 2, 3, 0, 256, 8),          # head_dim 256
    (1, 1, 0, 4, 1, 4, 10, 64, 16),         # 16 query rows per KV head (largest fused decode tile)
    (1, 1, 0, 8, 2, 1, 4095, 128, 4096),    # decode of the last position of a 4096 context
    (1, 1, 0, 8, 8, 1, 0, 128, 8),          # first token: one visible key
    (3, 1, 0, 6, 2, 2, 33, 32, 40),         # batch 3, GQA 3, two-token chunk
    (1, 1, 0, 32, 8, 1, 8000, 128, 8192),   # 64 key partitions, several tiles per wave
    (1, 1, 0, 16, 16, 1, 700, 64, 16384),   # MHA, partitions capped, long max_seq
    (1, 1, 0, 32, 4, 1, 200, 128, 256),     # 8 query rows per KV head
    (1, 1, 0, 16, 1, 1, 50, 128, 64),       # 16 query rows per KV head, head_dim 128
    (1, 1, 0, 4, 2, 1, 77, 192, 100),       # head_dim 192
    (2, 1, 0, 8, 2, 3, 40, 64, 64),         # three-token chunk through the decode kernel
    (2, 1, 0, 8, 8, 16, 3, 128, 32),        # prefill kernel: batch 2, MHA, 16 queries after a prefix
    (1, 1, 0, 16, 2, 65, 0, 64, 80),        # prefill kernel: 8 query heads per KV head, a 1-query tail tile
    (1, 1, 0, 32, 8, 1024, 0, 128, 1024),   # prefill kernel at the 8B shape, 1024 tokens
]


@pytest.mark.parametrize("shape", ATT_SHAPES)
def test_causal_attention_parity(hip, shape):
    B, L, layer, H, Hkv, S, past, D, max_seq = shape
    r = rng(sum(shape))
    q = r.uniform(-1, 1, B * H * S * D).astype(np.float32)
    k = r.uniform(-1, 1, B * Hkv * S * D).astype(np.float32)
    v = r.uniform(-1, 1, B * Hkv * S * D).astype(np.float32)
    cache = r.uniform(-1, 1, B * L * 2 * max_seq * Hkv * D).astype(np.float32)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    _, qr = put(hip, q)
    _, kr = put(hip, k)
    _, vr = put(hip, v)
    cb, cr = put(hip, cache)
    _, orf = out_buf(hip, q.size)
    hip.dispatch(Op.causal_attention(layer, H, Hkv, D, scale), [qr, kr, vr, cr],
                 [Value.f32([B, H, S, D]), Value.f32([B, Hkv, S, D]), Value.f32([B, Hkv, S, D]),
                  Value.f32([B, L, 2, max_seq, Hkv, D], ValueRole.STATE)], [orf], [Value.f32([B, H, S, D])], [past])
    want_out, want_cache = oracle.causal_attention(q, k, v, cache, B, L, layer, H, Hkv, S, past, D, max_seq, scale)
    got = read(hip, orf).reshape(B * H * S, D)
    want = want_out.reshape(B * H * S, D)
    for i in range(B * H * S):
        assert_normwise(got[i], want[i])
    assert np.array_equal(read(hip, cr), want_cache)


def test_kv_append_parity(hip):
    B, L, layer, Hkv, D, max_seq, past, S = 2, 3, 2, 8, 128, 64, 10, 5
    r = rng(3)
    k = r.standard_normal(B * Hkv * S * D).astype(np.float32)
    v = r.standard_normal(B * Hkv * S * D).astype(np.float32)
    cache = r.standard_normal(B * L * 2 * max_seq * Hkv * D).astype(np.float32)
    _, kr = put(hip, k)
    _, vr = put(hip, v)
    _, cr = put(hip, cache)
    hip.dispatch(Op.kv_append(layer), [kr, vr, cr],
                 [Value.f32([B, Hkv, S, D]), Value.f32([B, Hkv, S, D]),
                  Value.f32([B, L, 2, max_seq, Hkv, D], ValueRole.STATE)], [], [], [past])
    assert np.array_equal(read(hip, cr), oracle.kv_append(k, v, cache, B, L, layer, Hkv, D, max_seq, past, S))


# ----------------------------------------------------------------- matmul --


@pytest.mark.parametrize("nt", [True, False])
@pytest.mark.parametrize("a_shape,b_shape", [
    ((1, 1), (1, 1)), ((2, 3, 5), (2, 7, 5)), ((3, 4, 7), (5, 7)), ((1, 4, 9), (3, 6, 9)), ((64, 256), (300, 256)),
    ((2, 130, 70), (2, 65, 70)), ((2, 0, 4), (3, 4)), ((1, 2, 0), (3, 0)),
    # k % 4 == 0 and m >= 32: the f32 matrix-core kernel (128x128 tiles,
    # k staged 16 at a time): ragged m and n, a k tail, batch broadcast, NN
    # rows of B with n % 4 == 0 (and != 0: the VALU kernel)
    ((2, 130, 68), (2, 65, 68)), ((1, 257, 132), (3, 132, 132)), ((32, 512), (1000, 512)),
    ((2, 96, 20), (2, 36, 20)), ((4, 33, 4), (4, 129, 4)), ((256, 1024), (1536, 1024))])
def test_matmul_parity(hip, nt, a_shape, b_shape):
    r = rng(sum(a_shape) + sum(b_shape))
    if not nt:
        b_shape = b_shape[:-2] + (b_shape[-1], b_shape[-2])
    a = r.uniform(-1, 1, int(np.prod(a_shape))).astype(np.float32)
    b = r.uniform(-1, 1, int(np.prod(b_shape))).astype(np.float32)
    m, k = a_shape[-2], a_shape[-1]
    n = b_shape[-2] if nt else b_shape[-1]
    ba, bb = int(np.prod(a_shape[:-2])), int(np.prod(b_shape[:-2]))
    batch = max(ba, bb) if min(ba, bb) > 0 else 0
    out_shape = (batch if len(a_shape) > 2 or len(b_shape) > 2 else None, m, n)
    out_shape = tuple(d for d in out_shape if d is not None)
    _, ar = put(hip, a)
    _, br = put(hip, b)
    ob, orf = out_buf(hip, int(np.prod(out_shape)))
    hip.upload_f32(ob, np.full(int(np.prod(out_shape)), 5.0, np.float32)) if np.prod(out_shape) else None
    hip.dispatch(Op.matmul_nt() if nt else Op.matmul_nn(), [ar, br], [Value.f32(a_shape), Value.f32(b_shape)],
                 [orf], [Value.f32(out_shape)])
    fn = oracle.matmul_nt if nt else oracle.matmul_nn
    want = np.concatenate([
        fn(a.reshape(ba, -1)[i if ba > 1 else 0], b.reshape(bb, -1)[i if bb > 1 else 0], 1, m, k, n)
        for i in range(batch)]) if batch and m and n else np.zeros(int(np.prod(out_shape)), np.float32)
    got = read(hip, orf)
    if batch == 0:
        return  # an empty batch writes nothing (device.rs:1370-1372)
    if k == 0:
        assert np.all(got == 0)
        return
    for i in range(batch * m):
        assert_normwise(got.reshape(-1, n)[i], want.reshape(-1, n)[i])


# ------------------------------------------------------ quantized matmul --


def quant_weight(hip, w, fmt, group):
    n, k = w.shape
    words, scales = quant.quantize(w, group, fmt)
    pb = hip.upload_new_u32(words)
    sb = hip.upload_new_f32(scales)
    hip.bind_quantized(pb, sb, fmt, group, n, k)
    deq = quant.dequantize(words, scales, n, k, group, fmt)
    return BufferRef(pb, 0, words.size), Value.quantized([n, k], fmt, group), deq


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
@pytest.mark.parametrize("m,n,k,group", [(1, 256, 512, 128), (1, 300, 384, 128), (8, 256, 512, 128),
                                         (3, 64, 4096, 128), (17, 128, 256, 128), (64, 96, 512, 64),
                                         (2, 33, 130, 2), (1, 1024, 4096, 128), (2, 512, 1024, 128),
                                         (4, 48, 2048, 256), (12, 160, 1024, 128), (16, 64, 512, 64),
                                         (1, 4096, 14336, 128), (5, 17, 896, 128),
                                         # 16384 < m * k <= 32768: the fused GEMV with 16 waves per block
                                         (8, 256, 4096, 128), (2, 128, 14336, 128), (16, 96, 2048, 64),
                                         (6, 100, 4096, 256)])
def test_quantized_matmul_parity(hip, fmt, m, n, k, group):
    r = rng(m * n + k)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = r.standard_normal(m * k).astype(np.float32)
    wr, wv, deq = quant_weight(hip, w, fmt, group)
    _, ar = put(hip, a)
    _, orf = out_buf(hip, m * n)
    hip.dispatch(Op.matmul_nt(), [ar, wr], [Value.f32([1, m, k]), wv], [orf], [Value.f32([1, m, n])])
    want = oracle.matmul_nt(a, deq, 1, m, k, n)
    got = read(hip, orf).reshape(m, n)
    for i in range(m):
        assert_normwise(got[i], want.reshape(m, n)[i])


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
@pytest.mark.parametrize("m,n,k", [(1, 96, 4096), (4, 64, 2048), (8, 80, 4096), (3, 48, 14336)])
def test_quantized_gemv_extreme_activations(hip, fmt, m, n, k):
    """The GEMV's activation limbs take each 256-element chunk's exponent
    from its largest |x|: rows here are all zero, around 1e-33 (the chunk's
    scale 2^(22 - E) is not a normal float, so it is applied in two steps),
    around 1e25, and rows whose chunks span twelve orders of magnitude."""
    r = rng(m * 7 + n + k)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = r.standard_normal((m, k)).astype(np.float32)
    chunk_mag = 10.0 ** (np.arange(k // 256) % 13 - 6.0)
    kinds = ["zero", "tiny", "huge", "spread"]
    for i in range(m):
        kind = kinds[i % 4]
        if kind == "zero":
            a[i] = 0.0
        elif kind == "tiny":
            a[i] *= np.float32(1e-33)
        elif kind == "huge":
            a[i] *= np.float32(1e25)
        else:
            a[i] *= np.repeat(chunk_mag, 256).astype(np.float32)
    wr, wv, deq = quant_weight(hip, w, fmt, 128)
    _, ar = put(hip, a.ravel())
    _, orf = out_buf(hip, m * n)
    hip.dispatch(Op.matmul_nt(), [ar, wr], [Value.f32([1, m, k]), wv], [orf], [Value.f32([1, m, n])])
    want = oracle.matmul_nt(a.ravel(), deq, 1, m, k, n).reshape(m, n)
    got = read(hip, orf).reshape(m, n)
    for i in range(m):
        if kinds[i % 4] == "zero":
            np.testing.assert_array_equal(got[i], np.zeros(n, np.float32))
        else:
            assert_normwise(got[i], want[i])


@pytest.mark.parametrize("m", [1, 4, 8])
def test_rms_norm_then_quantized_projections_fuse(hip, m):
    """RmsNorm and two MatMulNT reading its output run as one fused GEMV with
    the norm as its prologue (at m = 8 and k = 4096, 16 waves per block and
    two partial sums per lane in the norm's reduction); the norm output is
    still written."""
    k, n1, n2 = 4096, 512, 256
    r = rng(70 + m)
    x = r.standard_normal(m * k).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)
    w1 = (r.standard_normal((n1, k)) * 0.02).astype(np.float32)
    w2 = (r.standard_normal((n2, k)) * 0.02).astype(np.float32)
    r1, v1, d1 = quant_weight(hip, w1, QuantFormat.INT4, 128)
    r2, v2, d2 = quant_weight(hip, w2, QuantFormat.INT4, 128)
    _, xr = put(hip, x)
    _, gr = put(hip, gamma)
    _, nr = out_buf(hip, m * k)
    _, o1 = out_buf(hip, m * n1)
    _, o2 = out_buf(hip, m * n2)
    xv = Value.f32([1, m, k])
    before = hip.stats()
    hip.dispatch(Op.rms_norm(1e-5), [xr, gr], [xv, Value.f32([k], ValueRole.PARAM)], [nr], [xv])
    hip.dispatch(Op.matmul_nt(), [nr, r1], [xv, v1], [o1], [Value.f32([1, m, n1])])
    hip.dispatch(Op.matmul_nt(), [nr, r2], [xv, v2], [o2], [Value.f32([1, m, n2])])
    hip.synchronize()
    assert hip.stats()["fused_commands"] - before["fused_commands"] == 3
    normed = oracle.rms_norm(x, gamma, m, k, 1e-5)
    got_n = read(hip, nr).reshape(m, k)
    for i in range(m):
        assert_normwise(got_n[i], normed.reshape(m, k)[i])
    for orf, deq, n in ((o1, d1, n1), (o2, d2, n2)):
        want = oracle.matmul_nt(normed, deq, 1, m, k, n).reshape(m, n)
        got = read(hip, orf).reshape(m, n)
        for i in range(m):
            assert_normwise(got[i], want[i])


@pytest.mark.parametrize("fmt,m,n,k,group", [(QuantFormat.INT4, 17, 100, 128, 128), (QuantFormat.INT8, 130, 257, 512, 64),
                                              (QuantFormat.INT4, 300, 512, 1024, 256),
                                              (QuantFormat.INT8, 200, 96, 2048, 128),
                                              (QuantFormat.INT4, 512, 512, 4096, 128),
                                              (QuantFormat.INT4, 40, 64, 384, 32),
                                              (QuantFormat.INT8, 33, 200, 384, 128),
                                              (QuantFormat.INT4, 272, 11008, 256, 128)])
def test_quantized_matmul_many_rows_on_matrix_cores(hip, fmt, m, n, k, group):
    """m > 16: the fp16 matrix-core path on split activations. Rows span nine
    orders of magnitude (each is split against its own maximum) and row 0 is
    all zeros. The shapes reach each block form: k in two slices of 128-row
    blocks (small grids whose half k is a whole number of groups and 128-k
    superblocks), 64-row blocks with 64-k stages (k 128, 384 at group 128) or
    32-k stages (group 32), and 128-row blocks (more than 256 of them)."""
    r = rng(m + n + k + group)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    mag = (10.0 ** r.uniform(-6, 3, m)).astype(np.float32)
    a = (r.standard_normal((m, k)).astype(np.float32) * mag[:, None]).astype(np.float32)
    a[0] = 0.0
    wr, wv, deq = quant_weight(hip, w, fmt, group)
    _, ar = put(hip, a.ravel())
    _, orf = out_buf(hip, m * n)
    hip.dispatch(Op.matmul_nt(), [ar, wr], [Value.f32([1, m, k]), wv], [orf], [Value.f32([1, m, n])])
    want = oracle.matmul_nt(a.ravel(), deq, 1, m, k, n).reshape(m, n)
    got = read(hip, orf).reshape(m, n)
    np.testing.assert_array_equal(got[0], np.zeros(n, np.float32))
    for i in range(1, m):
        assert_normwise(got[i], want[i])
    # the split keeps about 22 bits per element: far inside the bound
    worst = max(rel_l2(got[i], want[i]) for i in range(1, m))
    assert worst <= 2e-5, worst


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
def test_quantized_gemv_benchmark_shapes(hip, fmt, n, k):
    r = rng(n + k)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    a = r.standard_normal(k).astype(np.float32)
    wr, wv, deq = quant_weight(hip, w, fmt, 128)
    _, ar = put(hip, a)
    _, orf = out_buf(hip, n)
    hip.dispatch(Op.matmul_nt(), [ar, wr], [Value.f32([1, k]), wv], [orf], [Value.f32([1, n])])
    want = oracle.matmul_nt(a, deq, 1, 1, k, n)
    assert_normwise(read(hip, orf), want)


def test_quantized_payload_reupload_refreshes_codes(hip):
    n, k = 64, 256
    r = rng(11)
    w1 = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    w2 = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    wr, wv, _ = quant_weight(hip, w1, QuantFormat.INT4, 128)
    words2, scales2 = quant.quantize(w2, 128, QuantFormat.INT4)
    hip.upload_u32(wr.buffer, words2)
    sb = hip.upload_new_f32(scales2)
    hip.bind_quantized(wr.buffer, sb, QuantFormat.INT4, 128, n, k)
    a = r.standard_normal(k).astype(np.float32)
    _, ar = put(hip, a)
    _, orf = out_buf(hip, n)
    hip.dispatch(Op.matmul_nt(), [ar, wr], [Value.f32([1, k]), wv], [orf], [Value.f32([1, n])])
    want = oracle.matmul_nt(a, quant.dequantize(words2, scales2, n, k, 128, QuantFormat.INT4), 1, 1, k, n)
    assert_normwise(read(hip, orf), want)


def test_quantized_scale_reupload_refreshes_tile_scales(hip):
    # Scales uploaded again into the bound buffer must reach the decode GEMV
    # (which reads a tile-ordered copy of them) without a new bind.
    n, k = 96, 512
    r = rng(12)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    words, scales = quant.quantize(w, 128, QuantFormat.INT4)
    pb = hip.upload_new_u32(words)
    sb = hip.upload_new_f32(scales)
    hip.bind_quantized(pb, sb, QuantFormat.INT4, 128, n, k)
    scales2 = (scales * r.uniform(0.5, 2.0, scales.shape)).astype(np.float32)
    hip.upload_f32(sb, scales2)
    a = r.standard_normal(k).astype(np.float32)
    _, ar = put(hip, a)
    _, orf = out_buf(hip, n)
    hip.dispatch(Op.matmul_nt(), [ar, BufferRef(pb, 0, words.size)],
                 [Value.f32([1, k]), Value.quantized([n, k], QuantFormat.INT4, 128)], [orf], [Value.f32([1, n])])
    want = oracle.matmul_nt(a, quant.dequantize(words, scales2, n, k, 128, QuantFormat.INT4), 1, 1, k, n)
    assert_normwise(read(hip, orf), want)


# ------------------------------------------------------------- composites --


@pytest.mark.parametrize("quantized", [False, True])
@pytest.mark.parametrize("rows,hidden,inter", [(1, 1, 1), (3, 5, 7), (2, 8, 4), (4, 6, 13), (1, 256, 688),
                                               (5, 512, 1024), (1, 4096, 14336), (16, 512, 768)])
def test_swiglu_parity(hip, quantized, rows, hidden, inter):
    if quantized and (hidden % 128 or inter % 128):
        pytest.skip("group size 128 needs hidden and inter multiples of 128")
    r = rng(rows + hidden + inter)
    x = r.uniform(-1, 1, rows * hidden).astype(np.float32)
    g = (r.standard_normal((inter, hidden)) * 0.1).astype(np.float32)
    u = (r.standard_normal((inter, hidden)) * 0.1).astype(np.float32)
    d = (r.standard_normal((hidden, inter)) * 0.1).astype(np.float32)
    _, xr = put(hip, x)
    if quantized:
        fmt = QuantFormat.INT8 if rows == 16 else QuantFormat.INT4
        gr, gv, g = quant_weight(hip, g, fmt, 128)
        ur, uv, u = quant_weight(hip, u, fmt, 128)
        dr, dv, d = quant_weight(hip, d, fmt, 128)
    else:
        gr, ur, dr = put(hip, g)[1], put(hip, u)[1], put(hip, d)[1]
        gv = uv = Value.f32([inter, hidden], ValueRole.PARAM)
        dv = Value.f32([hidden, inter], ValueRole.PARAM)
    _, orf = out_buf(hip, rows * hidden)
    hip.dispatch(Op.swiglu(), [xr, gr, ur, dr], [Value.f32([rows, hidden]), gv, uv, dv], [orf],
                 [Value.f32([rows, hidden])])
    want = oracle.swiglu(x, g, u, d, rows, hidden, inter).reshape(rows, hidden)
    got = read(hip, orf).reshape(rows, hidden)
    for i in range(rows):
        assert_normwise(got[i], want[i])


@pytest.mark.parametrize("quantized", [False, True])
@pytest.mark.parametrize("rows,hidden,out_f", [(1, 1, 1), (3, 7, 5), (2, 33, 17), (4, 256, 384), (1, 4096, 1024),
                                               (3, 512, 640),
                                               # the fused GEMV's prologue at 2, 4 and 8 float4 of
                                               # activations per thread (its runs' sums reduced together)
                                               (2, 4096, 512), (8, 4096, 256), (1, 8192, 256),
                                               # rows ending inside a thread's runs, and runs past the input
                                               (3, 4096, 256), (6, 4096, 128), (12, 2048, 256),
                                               # many rows: the norm inside the q-GEMM's activation split
                                               # (up to 8192 wide), or on its own past that
                                               (64, 4096, 256), (40, 2048, 384), (100, 8192, 128),
                                               (33, 12288, 128)])
def test_rms_norm_matmul_parity(hip, quantized, rows, hidden, out_f):
    if quantized and hidden % 128:
        pytest.skip("group size 128 needs hidden multiple of 128")
    r = rng(rows + hidden)
    x = r.uniform(-2, 2, rows * hidden).astype(np.float32)
    wt = r.uniform(0.5, 1.5, hidden).astype(np.float32)
    w = (r.standard_normal((out_f, hidden)) * 0.1).astype(np.float32)
    _, xr = put(hip, x)
    _, wtr = put(hip, wt)
    if quantized:
        wr, wv, w = quant_weight(hip, w, QuantFormat.INT8, 128)
    else:
        wr = put(hip, w)[1]
        wv = Value.f32([out_f, hidden], ValueRole.PARAM)
    _, orf = out_buf(hip, rows * out_f)
    hip.dispatch(Op.rms_norm_matmul(1e-5), [xr, wtr, wr],
                 [Value.f32([rows, hidden]), Value.f32([hidden], ValueRole.PARAM), wv], [orf],
                 [Value.f32([rows, out_f])])
    want = oracle.rms_norm_matmul(x, wt, w, rows, hidden, out_f, 1e-5).reshape(rows, out_f)
    got = read(hip, orf).reshape(rows, out_f)
    for i in range(rows):
        assert_normwise(got[i], want[i])


@pytest.mark.parametrize("rows,hidden,out_f", [(64, 4096, 256), (17, 2048, 128), (48, 8192, 64)])
def test_rms_norm_matmul_int4_many_rows(hip, rows, hidden, out_f):
    """RmsNormMatMul on INT4 weights at more than 16 rows: the norm inside the
    q-GEMM's activation split. Normwise per row against the oracle (1e-4)."""
    r = rng(rows * 3 + hidden)
    x = r.uniform(-2, 2, rows * hidden).astype(np.float32)
    wt = r.uniform(0.5, 1.5, hidden).astype(np.float32)
    w = (r.standard_normal((out_f, hidden)) * 0.1).astype(np.float32)
    _, xr = put(hip, x)
    _, wtr = put(hip, wt)
    wr, wv, w = quant_weight(hip, w, QuantFormat.INT4, 128)
    _, orf = out_buf(hip, rows * out_f)
    hip.dispatch(Op.rms_norm_matmul(1e-5), [xr, wtr, wr],
                 [Value.f32([rows, hidden]), Value.f32([hidden], ValueRole.PARAM), wv], [orf],
                 [Value.f32([rows, out_f])])
    want = oracle.rms_norm_matmul(x, wt, w, rows, hidden, out_f, 1e-5).reshape(rows, out_f)
    got = read(hip, orf).reshape(rows, out_f)
    for i in range(rows):
        assert_normwise(got[i], want[i])
