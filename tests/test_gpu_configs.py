"""The benchmark configurations against the oracle, at the sizes the
benchmark runs them (or, for whole models, two layers of the same shapes).

 * Prefill of more than 16 tokens runs the matrix-core GEMM and the tiled
   prefill attention inside a fused submission; it is submitted three times
   so the second is captured as a HIP graph and the third replays it.
 * 8B-shaped batch-8 decode, INT8 weights through the engine.
 * Engine steps are teacher-forced: both engines take the oracle's greedy
   ids, so every step's logits are compared on identical inputs
   (1e-4 normwise per row), and the GPU's greedy id must equal the oracle's
   unless the oracle's top-2 gap is below 1e-4 * ||logits||_2.
 * Kernel-level: the [128256 x 4096] lm_head GEMV, the q-matmul at its full
   shapes for M = 8 and M = 512, and the elementwise / reduction
   microbenchmark at full size.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import assert_elementwise, assert_normwise
from models import Pair
from starlight_amd.graph import LlamaConfig
from starlight_amd.ir import BufferRef, Op, QuantFormat, RopeVariant, Value, ValueRole

pytestmark = pytest.mark.gpu


def shape_1b(fmt, layers=2):
    return LlamaConfig(layers=layers, hidden=2048, heads=32, kv_heads=8, head_dim=64, ffn=8192, vocab=32000,
                       theta=500_000.0, quant=fmt)


def shape_8b(fmt, layers=2, vocab=32000):
    return LlamaConfig(layers=layers, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=vocab,
                       theta=500_000.0, quant=fmt)


# ----------------------------------------------------------------- engine --


@pytest.mark.parametrize("model", ["1b", "8b"])
@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
def test_prefill_beyond_16_tokens_captured_and_replayed(hip, model, fmt):
    """A 40-token prompt (not a multiple of 16 or 64) through two layers:
    the prefill submission runs on the matrix cores and the tiled prefill
    attention, as one eager run, one graph capture and one graph replay, each
    with the oracle's logits; then 4 teacher-forced decode steps."""
    cfg = shape_1b(fmt) if model == "1b" else shape_8b(fmt)
    pair = Pair(hip, cfg, batch=1, prompt_len=40, max_seq=64, seed=20)
    try:
        before = hip.stats()
        ids = pair.prefill(repeats=3)
        mid = hip.stats()
        assert mid["graph_captures"] >= before["graph_captures"] + 1
        assert mid["graph_replays"] >= before["graph_replays"] + 1
        steps = pair.decode(ids, 4)
        assert len(steps) == 4
        after = hip.stats()
        assert after["fused_commands"] > mid["fused_commands"]
    finally:
        pair.close()


def test_8b_shaped_batch8_decode(hip):
    """Eight sequences of the 8B shapes (two layers, INT4 g128): an 8 x 12
    token prefill (96 rows on the matrix cores), then 6 teacher-forced decode
    steps of 8 rows, every row's logits and greedy id checked."""
    cfg = shape_8b(QuantFormat.INT4)
    pair = Pair(hip, cfg, batch=8, prompt_len=12, max_seq=32, seed=21)
    try:
        ids = pair.prefill()
        before = hip.stats()
        pair.decode(ids, 6)
        after = hip.stats()
        assert after["graph_replays"] >= before["graph_replays"] + 3
        assert pair.mismatched_ids <= 1
    finally:
        pair.close()


def test_8b_shaped_int8_decode(hip):
    """The INT8 variant of the 8B shapes through the engine: 8-token prefill,
    8 teacher-forced decode steps (fused and graph-replayed)."""
    cfg = shape_8b(QuantFormat.INT8)
    pair = Pair(hip, cfg, batch=1, prompt_len=8, max_seq=32, seed=22)
    try:
        ids = pair.prefill()
        before = hip.stats()
        pair.decode(ids, 8)
        after = hip.stats()
        assert after["graph_replays"] >= before["graph_replays"] + 5
        assert after["fused_commands"] > before["fused_commands"]
    finally:
        pair.close()


# ----------------------------------------------------------------- kernels --


def quantized(hip, w, fmt, group=128):
    n, k = w.shape
    bits = 4 if fmt == QuantFormat.INT4 else 8
    payload, scales = oracle.quantize_groupwise(w, n, k, group, bits)
    raw = payload.ravel()
    raw = np.concatenate([raw, np.zeros((-raw.size) % 4, np.uint8)])
    words = raw.view("<u4")
    pb = hip.upload_new_u32(words)
    sb = hip.upload_new_f32(scales)
    hip.bind_quantized(pb, sb, fmt, group, n, k)
    deq = oracle.dequantize_groupwise(payload, scales, n, k, group, bits)
    return BufferRef(pb, 0, words.size), Value.quantized([n, k], fmt, group), deq


def run_qmatmul(hip, fmt, m, n, k, seed):
    r = np.random.default_rng(seed)
    w = (r.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    a = r.standard_normal(m * k, dtype=np.float32)
    wr, wv, deq = quantized(hip, w, fmt)
    ab = hip.upload_new_f32(a)
    ob = hip.allocate_f32(m * n, 256)
    hip.dispatch(Op.matmul_nt(), [BufferRef(ab, 0, a.size), wr], [Value.f32([1, m, k]), wv],
                 [BufferRef(ob, 0, m * n)], [Value.f32([1, m, n])])
    got = hip.read_f32(ob, m * n).reshape(m, n)
    want = oracle.matmul_nt(a, deq, 1, m, k, n).reshape(m, n)
    for i in range(m):
        assert_normwise(got[i], want[i])


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
def test_lm_head_gemv_128256_rows(hip, fmt):
    """The 8B lm_head, [128256 x 4096] g128, at M = 1 (8016 row tiles)."""
    run_qmatmul(hip, fmt, 1, 128256, 4096, 31)


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("m", [8, 512])
def test_qmatmul_full_shapes(hip, fmt, n, k, m):
    """The q-matmul microbenchmark shapes at M = 8 (decode, small batch) and
    M = 512 (prefill GEMM), every row against dequantize-then-matmul_nt."""
    run_qmatmul(hip, fmt, m, n, k, 32 + m + n // 1024)


def test_rms_norm_full_4096x4096(hip):
    r = np.random.default_rng(40)
    rows = hidden = 4096
    x = r.standard_normal(rows * hidden, dtype=np.float32)
    w = (1 + 0.1 * r.standard_normal(hidden)).astype(np.float32)
    xb, wb, ob = hip.upload_new_f32(x), hip.upload_new_f32(w), hip.allocate_f32(x.size, 256)
    v = Value.f32([rows, hidden])
    hip.dispatch(Op.rms_norm(1e-5), [BufferRef(xb, 0, x.size), BufferRef(wb, 0, hidden)],
                 [v, Value.f32([hidden], ValueRole.PARAM)], [BufferRef(ob, 0, x.size)], [v])
    got = hip.read_f32(ob, x.size).reshape(rows, hidden)
    want = oracle.rms_norm(x, w, rows, hidden, 1e-5).reshape(rows, hidden)
    err = np.linalg.norm((got - want).astype(np.float64), axis=1) / np.linalg.norm(want.astype(np.float64), axis=1)
    assert err.max() <= 1e-4, err.max()


def test_softmax_full_32x2048x2048(hip):
    """Scaled scores (x / sqrt(128)) over 65,536 rows of 2,048."""
    r = np.random.default_rng(41)
    rows, cols = 32 * 2048, 2048
    x = (r.standard_normal(rows * cols, dtype=np.float32) * np.float32(1 / math.sqrt(128))).astype(np.float32)
    xb, ob = hip.upload_new_f32(x), hip.allocate_f32(x.size, 256)
    v = Value.f32([32, 2048, 2048])
    hip.dispatch(Op.softmax(), [BufferRef(xb, 0, x.size)], [v], [BufferRef(ob, 0, x.size)], [v])
    got = hip.read_f32(ob, x.size).reshape(rows, cols)
    want = oracle.softmax(x, rows, cols).reshape(rows, cols)
    err = np.linalg.norm((got - want).astype(np.float64), axis=1) / np.linalg.norm(want.astype(np.float64), axis=1)
    assert err.max() <= 1e-4, err.max()


@pytest.mark.parametrize("variant", [RopeVariant.NEOX, RopeVariant.GPTJ])
def test_rope_full_4096_tokens(hip, variant):
    """RoPE (theta 500000) on [1, 32, 4096, 128], positions 0..4095: every
    element within 1e-6 relative."""
    r = np.random.default_rng(42)
    B, H, S, D = 1, 32, 4096, 128
    x = r.standard_normal(B * H * S * D, dtype=np.float32)
    pos = np.arange(S, dtype=np.uint32)
    xb, pb, ob = hip.upload_new_f32(x), hip.upload_new_u32(pos), hip.allocate_f32(x.size, 256)
    v = Value.f32([B, H, S, D])
    hip.dispatch(Op.rope(variant, 500_000.0), [BufferRef(xb, 0, x.size), BufferRef(pb, 0, S)],
                 [v, Value.u32([B, S])], [BufferRef(ob, 0, x.size)], [v])
    name = "neox" if variant == RopeVariant.NEOX else "gptj"
    assert_elementwise(hip.read_f32(ob, x.size), oracle.rope(x, pos, B, H, S, D, 500_000.0, name))


def test_add_and_silu_mul_full_4096x14336(hip):
    """The residual add (bit-exact) and SiLU(gate) * up, which the device
    runs as one fused pass (per element within 1e-6)."""
    r = np.random.default_rng(43)
    n = 4096 * 14336
    a = r.standard_normal(n, dtype=np.float32)
    b = r.standard_normal(n, dtype=np.float32)
    ab, bb = hip.upload_new_f32(a), hip.upload_new_f32(b)
    tb, ob = hip.allocate_f32(n, 256), hip.allocate_f32(n, 256)
    v = Value.f32([4096, 14336])
    A, Bf, T, O = (BufferRef(x, 0, n) for x in (ab, bb, tb, ob))
    hip.dispatch(Op.add(), [A, Bf], [v, v], [O], [v])
    assert np.array_equal(hip.read_f32(ob, n), oracle.add(a, b, n))
    before = hip.stats()
    hip.dispatch(Op.silu(), [A], [v], [T], [v])
    hip.dispatch(Op.mul(), [T, Bf], [v, v], [O], [v])
    hip.dispatch(Op.scale_by(1.0), [Bf], [v], [T], [v])  # t is dead after the Mul
    hip.synchronize()
    assert hip.stats()["fused_commands"] - before["fused_commands"] == 2
    assert_elementwise(hip.read_f32(ob, n), oracle.mul(oracle.silu(a), b, n))
