"""Pins the C oracle against the reference's own kernel tests.

Every case below uses the seeds, shapes, input ranges, f64 oracles and the
mixed abs/rel tolerance of the corresponding `#[test]` in
crates/backends/backend-cpu/src/reference/*.rs (file:line in each docstring).
The f64 oracles are written here with numpy in float64 — vectorised, not the
scalar loop order the restatement uses — so a dropped term, swapped operand
or wrong index in the C code fails them.
"""
import math

import numpy as np
import pytest

from conftest import assert_close
from oracle import Lcg, OracleError


def f64(a):
    return np.asarray(a, dtype=np.float64)


# ---------------------------------------------------------------- LCG ------


def test_lcg_matches_an_independent_integer_restatement():
    """reference/mod.rs:118-148: state = state*6364136223846793005 + 1442695040888963407
    (mod 2^64); next_u32 = state >> 33; uniform = low + (high-low)*f32(u/u32::MAX)."""
    state = 7
    lcg = Lcg(7)
    for _ in range(1000):
        state = (state * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        assert lcg.next_u32() == state >> 33
    lcg = Lcg(3)
    state = 3
    vals = lcg.fill(500, -2.0, 2.0)
    for v in vals:
        state = (state * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        unit = np.float32((state >> 33) / 4294967295.0)
        expect = np.float32(np.float32(-2.0) + np.float32(np.float32(4.0) * unit))
        assert v == expect
    assert vals.min() >= -2.0 and vals.max() <= 2.0


# -------------------------------------------------------------- matmul -----


def _nt64(a, b, batch, m, k, n):
    return np.einsum("bmk,bnk->bmn", f64(a).reshape(batch, m, k), f64(b).reshape(batch, n, k))


def _nn64(a, b, batch, m, k, n):
    return np.einsum("bmk,bkn->bmn", f64(a).reshape(batch, m, k), f64(b).reshape(batch, k, n))


@pytest.mark.parametrize("seed,shape", [(1, (1, 1, 1, 1)), (2, (2, 3, 5, 7)), (3, (2, 4, 9, 6))])
def test_matmul_nt_matches_f64_oracle(oracle, seed, shape):
    """matmul.rs:191-196."""
    batch, m, k, n = shape
    lcg = Lcg(seed)
    a = lcg.fill(batch * m * k, -1.0, 1.0)
    b = lcg.fill(batch * n * k, -1.0, 1.0)
    assert_close(oracle.matmul_nt(a, b, batch, m, k, n), _nt64(a, b, batch, m, k, n))


@pytest.mark.parametrize("seed,shape", [(11, (1, 1, 1, 1)), (12, (3, 4, 7, 5)), (13, (2, 5, 3, 9))])
def test_matmul_nn_matches_f64_oracle(oracle, seed, shape):
    """matmul.rs:198-204."""
    batch, m, k, n = shape
    lcg = Lcg(seed)
    a = lcg.fill(batch * m * k, -1.0, 1.0)
    b = lcg.fill(batch * k * n, -1.0, 1.0)
    assert_close(oracle.matmul_nn(a, b, batch, m, k, n), _nn64(a, b, batch, m, k, n))


def test_matmul_accepts_empty_dimensions(oracle):
    """matmul.rs:206-228: empty batch / rows accepted; k == 0 writes zeros."""
    e = np.zeros(0, np.float32)
    oracle.matmul_nt(e, e, 0, 2, 3, 4)
    oracle.matmul_nn(e, e, 0, 2, 3, 4)
    oracle.matmul_nt(e, np.zeros(24, np.float32), 2, 0, 3, 4)
    oracle.matmul_nn(e, np.zeros(24, np.float32), 2, 0, 3, 4)
    assert np.array_equal(oracle.matmul_nt(e, e, 1, 2, 0, 3), np.zeros(6))
    assert np.array_equal(oracle.matmul_nn(e, e, 1, 2, 0, 3), np.zeros(6))


def test_matmul_rejects_wrong_lengths(oracle):
    """matmul.rs:230-257."""
    a = np.zeros(24, np.float32)
    b_nt = np.zeros(40, np.float32)
    b_nn = np.zeros(40, np.float32)
    for call in (
        lambda: oracle.matmul_nt(a[:-1], b_nt, 2, 3, 4, 5),
        lambda: oracle.matmul_nt(a, b_nt[:-1], 2, 3, 4, 5),
        lambda: oracle.matmul_nn(a, b_nn, 2, 3, 4, 5, out_len=29),
        lambda: oracle.matmul_nn(a, b_nn[:-1], 2, 3, 4, 5),
    ):
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == "LengthMismatch"


def test_matmul_reports_shape_overflow(oracle):
    """matmul.rs:259-266."""
    e = np.zeros(0, np.float32)
    with pytest.raises(OracleError) as err:
        oracle.matmul_nt(e, e, 2**64 - 1, 2, 1, 1, out_len=0)
    assert err.value.kind == "ShapeOverflow"


# ---------------------------------------------------------------- norm -----


def _rms64(x, w, rows, hidden, eps):
    x = f64(x).reshape(rows, hidden)
    inv = 1.0 / np.sqrt((x * x).sum(axis=1, keepdims=True) / hidden + float(np.float32(eps)))
    return x * inv * f64(w)[None, :]


@pytest.mark.parametrize("rows,hidden,eps,seed", [(1, 1, 1e-5, 1), (3, 7, 1e-6, 2), (4, 16, 1e-5, 3),
                                                  (2, 33, 1e-6, 4)])
def test_rms_norm_matches_f64_oracle(oracle, rows, hidden, eps, seed):
    """norm.rs:106-112."""
    lcg = Lcg(seed)
    x = lcg.fill(rows * hidden, -2.0, 2.0)
    w = lcg.fill(hidden, 0.5, 1.5)
    assert_close(oracle.rms_norm(x, w, rows, hidden, eps), _rms64(x, w, rows, hidden, eps))


def test_rms_norm_zero_rows_and_invalid_shapes(oracle):
    """norm.rs:114-144."""
    oracle.rms_norm(np.zeros(0), np.ones(4), 0, 4, 1e-5)
    with pytest.raises(OracleError) as err:
        oracle.rms_norm(np.zeros(0), np.zeros(0), 2, 0, 1e-5, out_len=0)
    assert err.value.kind == "InvalidShape"
    x, w = np.ones(8), np.ones(4)
    for call in (
        lambda: oracle.rms_norm(x, w[:3], 2, 4, 1e-5),
        lambda: oracle.rms_norm(x[:7], w, 2, 4, 1e-5),
        lambda: oracle.rms_norm(x, w, 2, 4, 1e-5, out_len=7),
    ):
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == "LengthMismatch"


# ------------------------------------------------------------- softmax -----


def _softmax64(x, rows, cols, visible=None):
    x = f64(x).reshape(rows, cols)
    out = np.zeros_like(x)
    for r in range(rows):
        v = cols if visible is None else visible[r]
        e = np.exp(x[r, :v] - x[r, :v].max())
        out[r, :v] = e / e.sum()
    return out


@pytest.mark.parametrize("seed,shape", [(1, (1, 1)), (2, (3, 5)), (3, (6, 17))])
def test_softmax_matches_f64_oracle(oracle, seed, shape):
    """softmax.rs:194-199."""
    rows, cols = shape
    x = Lcg(seed).fill(rows * cols, -4.0, 4.0)
    assert_close(oracle.softmax(x, rows, cols), _softmax64(x, rows, cols))


def test_softmax_is_stable_for_extreme_values(oracle):
    """softmax.rs:201-208."""
    x = np.array([1000.0, 999.0, -1000.0, 0.0], np.float32)
    out = oracle.softmax(x, 2, 2)
    assert_close(out, _softmax64(x, 2, 2))
    assert np.isfinite(out).all()


@pytest.mark.parametrize("seed,shape", [(11, (2, 2, 0)), (12, (12, 4, 1)), (13, (4, 1, 7)),
                                        (14, (6, 3, 2))])
def test_softmax_causal_matches_f64_oracle(oracle, seed, shape):
    """softmax.rs:210-220; masked columns must come back exactly zero."""
    rows, seq, past = shape
    cols = past + seq
    x = Lcg(seed).fill(rows * cols, -3.0, 3.0)
    visible = [past + r % seq + 1 for r in range(rows)]
    out = oracle.softmax_causal(x, rows, cols, seq, past)
    assert_close(out, _softmax64(x, rows, cols, visible))
    grid = out.reshape(rows, cols)
    for r in range(rows):
        assert np.all(grid[r, visible[r]:] == 0.0)


def test_softmax_rejects_invalid_shapes(oracle):
    """softmax.rs:222-254."""
    cases = [
        (lambda: oracle.softmax(np.zeros(0), 0, 4), "InvalidShape"),
        (lambda: oracle.softmax(np.zeros(0), 4, 0), "InvalidShape"),
        (lambda: oracle.softmax(np.zeros(5), 2, 3), "LengthMismatch"),
        (lambda: oracle.softmax_causal(np.zeros(6), 2, 3, 2, 0), "InvalidShape"),
        (lambda: oracle.softmax_causal(np.zeros(4), 2, 2, 0, 2), "InvalidShape"),
        (lambda: oracle.softmax_causal(np.zeros(6), 3, 2, 2, 0), "InvalidShape"),
        (lambda: oracle.softmax_causal(np.zeros(5), 2, 3, 2, 1), "LengthMismatch"),
    ]
    for call, kind in cases:
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == kind


# ---------------------------------------------------------------- rope -----


def _positions(lcg, batch, seq, past_offset):
    """rope.rs:148-154: past_offset + index*2 + below(5)."""
    return np.array([past_offset + i * 2 + lcg.below(5) for i in range(batch * seq)], np.uint32)


def _rope64(x, pos, batch, heads, seq, head_dim, theta, interleaved):
    x = f64(x).reshape(batch, heads, seq, head_dim)
    half = head_dim // 2
    pairs = np.arange(half, dtype=np.float64)
    inv = float(np.float32(theta)) ** (2.0 * pairs / head_dim)
    ang = f64(pos).reshape(batch, 1, seq, 1) / inv.reshape(1, 1, 1, half)
    s, c = np.sin(ang), np.cos(ang)
    if interleaved:
        a, b = x[..., 0::2], x[..., 1::2]
    else:
        a, b = x[..., :half], x[..., half:]
    ra, rb = a * c - b * s, a * s + b * c
    out = np.empty_like(x)
    if interleaved:
        out[..., 0::2], out[..., 1::2] = ra, rb
    else:
        out[..., :half], out[..., half:] = ra, rb
    return out


@pytest.mark.parametrize("seed,shape", [(1, (1, 1, 1, 2, 10_000.0)), (2, (2, 3, 5, 4, 10_000.0)),
                                        (3, (2, 2, 4, 8, 500_000.0)), (4, (1, 3, 3, 6, 10_000.0))])
def test_rope_neox_matches_f64_oracle(oracle, seed, shape):
    """rope.rs:238-248."""
    batch, heads, seq, hd, theta = shape
    lcg = Lcg(seed)
    x = lcg.fill(batch * heads * seq * hd, -2.0, 2.0)
    pos = _positions(lcg, batch, seq, 3)
    out = oracle.rope(x, pos, batch, heads, seq, hd, theta, "neox")
    assert_close(out, _rope64(x, pos, batch, heads, seq, hd, theta, False))


@pytest.mark.parametrize("seed,shape", [(11, (1, 1, 1, 2, 10_000.0)), (12, (2, 3, 5, 4, 10_000.0)),
                                        (13, (2, 2, 4, 8, 500_000.0)),
                                        (14, (1, 2, 3, 10, 1_000_000.0))])
def test_rope_gptj_matches_f64_oracle(oracle, seed, shape):
    """rope.rs:250-260."""
    batch, heads, seq, hd, theta = shape
    lcg = Lcg(seed)
    x = lcg.fill(batch * heads * seq * hd, -2.0, 2.0)
    pos = _positions(lcg, batch, seq, 1)
    out = oracle.rope(x, pos, batch, heads, seq, hd, theta, "gptj")
    assert_close(out, _rope64(x, pos, batch, heads, seq, hd, theta, True))


def test_rope_position_zero_is_identity_and_norm_is_preserved(oracle):
    """Closed forms: angle 0 leaves x unchanged bit-for-bit; a rotation keeps
    each pair's length (to f32 rounding)."""
    x = Lcg(5).fill(2 * 3 * 4 * 8, -2.0, 2.0)
    pos = np.zeros(2 * 4, np.uint32)
    assert np.array_equal(oracle.rope(x, pos, 2, 3, 4, 8, 10_000.0, "neox"), x)
    pos = np.arange(8, dtype=np.uint32) * 37
    out = oracle.rope(x, pos, 2, 3, 4, 8, 10_000.0, "neox").reshape(-1, 8)
    xi = f64(x).reshape(-1, 8)
    np.testing.assert_allclose(out[:, :4] ** 2 + out[:, 4:] ** 2, xi[:, :4] ** 2 + xi[:, 4:] ** 2,
                               rtol=1e-5)


def test_rope_rejects_invalid_shapes(oracle):
    """rope.rs:262-282."""
    x, pos = np.zeros(8), np.zeros(2, np.uint32)
    cases = [
        (lambda: oracle.rope(x, pos, 1, 1, 2, 3, 10_000.0, "neox"), "InvalidShape"),
        (lambda: oracle.rope(x, pos, 1, 1, 2, 0, 10_000.0, "gptj"), "InvalidShape"),
        (lambda: oracle.rope(x, pos[:1], 1, 1, 2, 4, 10_000.0, "neox"), "LengthMismatch"),
        (lambda: oracle.rope(x[:7], pos, 1, 1, 2, 4, 10_000.0, "gptj"), "LengthMismatch"),
    ]
    for call, kind in cases:
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == kind


# --------------------------------------------------------- elementwise -----


def _silu64(x):
    x = f64(x)
    return x / (1.0 + np.exp(-x))


@pytest.mark.parametrize("seed,length", [(1, 1), (2, 7), (3, 33)])
def test_silu_matches_f64_oracle(oracle, seed, length):
    """elementwise.rs:90-105."""
    x = Lcg(seed).fill(length, -8.0, 8.0)
    assert_close(oracle.silu(x), _silu64(x))


def test_silu_extremes(oracle):
    """elementwise.rs:101-104."""
    x = np.array([-100.0, -10.0, 0.0, 10.0, 100.0], np.float32)
    assert_close(oracle.silu(x), _silu64(x))


@pytest.mark.parametrize("seed,length", [(11, 0), (12, 1), (13, 5), (14, 33)])
def test_mul_add_scale_match_f64_oracle(oracle, seed, length):
    """elementwise.rs:107-143."""
    lcg = Lcg(seed)
    a = lcg.fill(length, -2.0, 2.0)
    b = lcg.fill(length, -2.0, 2.0)
    assert_close(oracle.mul(a, b, length), f64(a) * f64(b))
    assert_close(oracle.add(a, b, length), f64(a) + f64(b))
    assert_close(oracle.scale(a, -1.5), f64(a) * -1.5)


def test_elementwise_rejects_wrong_lengths(oracle):
    """elementwise.rs:145-169."""
    a = np.array([1.0, 2.0, 3.0], np.float32)
    b = np.array([4.0, 5.0, 6.0], np.float32)
    for call in (
        lambda: oracle.mul(a, b[:2], 3),
        lambda: oracle.mul(a[:2], b, 3),
        lambda: oracle.add(a, b, 3, out_len=2),
        lambda: oracle.add(a, b[:2], 3),
    ):
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == "LengthMismatch"
    e = np.zeros(0, np.float32)
    oracle.silu(e), oracle.scale(e, 2.0), oracle.mul(e, e, 0), oracle.add(e, e, 0)


# -------------------------------------------------------------- layout -----


@pytest.mark.parametrize("seed,shape", [(1, (10, 5, 3)), (2, (1, 1, 1)), (3, (4, 7, 0)),
                                        (4, (13, 9, 6))])
def test_gather_matches_f64_oracle(oracle, seed, shape):
    """layout.rs:287-296."""
    vocab, hidden, rows = shape
    lcg = Lcg(seed)
    table = lcg.fill(vocab * hidden, -1.0, 1.0)
    ids = np.array([lcg.below(vocab) for _ in range(rows)], np.uint32)
    expected = f64(table).reshape(vocab, hidden)[ids.astype(np.int64)]
    assert_close(oracle.gather(table, ids, vocab, hidden, rows), expected)


def test_gather_rejects_bad_ids_and_lengths(oracle):
    """layout.rs:298-318: a bad id is rejected before any write."""
    table = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    out = np.zeros(2, np.float32)
    with pytest.raises(OracleError) as err:
        oracle.gather(table, [4], 2, 2, 1, out=out)
    assert (err.value.kind, err.value.reason) == ("InvalidShape", "id out of range")
    assert np.array_equal(out, [0.0, 0.0])
    for call in (
        lambda: oracle.gather(table[:3], [0], 2, 2, 1),
        lambda: oracle.gather(table, [0, 1], 2, 2, 1, out=np.zeros(2, np.float32)),
        lambda: oracle.gather(table, [0], 2, 2, 1, out=np.zeros(1, np.float32)),
    ):
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == "LengthMismatch"


@pytest.mark.parametrize("seed,shape", [(11, (1, 1, 3, 1)), (12, (3, 5, 4, 5)), (13, (2, 4, 7, 2))])
def test_last_token_matches_f64_oracle(oracle, seed, shape):
    """layout.rs:320-327."""
    batch, seq, hidden, seq_len = shape
    inp = Lcg(seed).fill(batch * seq * hidden, -1.0, 1.0)
    expected = f64(inp).reshape(batch, seq, hidden)[:, seq_len - 1, :]
    assert_close(oracle.last_token(inp, batch, seq, hidden, seq_len), expected)


def test_last_token_rejects_bad_seq_len_and_lengths(oracle):
    """layout.rs:329-349."""
    inp = np.zeros(16, np.float32)
    cases = [
        (lambda: oracle.last_token(inp, 2, 4, 2, 0), "InvalidShape"),
        (lambda: oracle.last_token(inp, 2, 4, 2, 5), "InvalidShape"),
        (lambda: oracle.last_token(inp[:15], 2, 4, 2, 4), "LengthMismatch"),
        (lambda: oracle.last_token(inp, 2, 4, 2, 4, out_len=3), "LengthMismatch"),
    ]
    for call, kind in cases:
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == kind


@pytest.mark.parametrize("seed,shape", [(21, (1, 1, 1, 2)), (22, (2, 3, 4, 4)), (23, (2, 5, 3, 6)),
                                        (24, (1, 4, 2, 8))])
def test_split_and_merge_heads_match_f64_oracle(oracle, seed, shape):
    """layout.rs:351-361 (and the split∘merge identity of layout.rs:265-283)."""
    batch, seq, heads, hd = shape
    inp = Lcg(seed).fill(batch * seq * heads * hd, -1.0, 1.0)
    split = oracle.split_heads(inp, batch, seq, heads, hd)
    expected = f64(inp).reshape(batch, seq, heads, hd).transpose(0, 2, 1, 3)
    assert_close(split, expected)
    merged = oracle.merge_heads(split, batch, seq, heads, hd)
    assert_close(merged, f64(split).reshape(batch, heads, seq, hd).transpose(0, 2, 1, 3))
    assert np.array_equal(merged, inp)


def test_split_and_merge_reject_wrong_lengths(oracle):
    """layout.rs:363-383."""
    inp = np.zeros(16, np.float32)
    for call in (
        lambda: oracle.split_heads(inp[:15], 2, 2, 2, 2, out_len=16),
        lambda: oracle.split_heads(inp, 2, 2, 2, 2, out_len=15),
        lambda: oracle.merge_heads(inp[:15], 2, 2, 2, 2, out_len=16),
        lambda: oracle.merge_heads(inp, 2, 2, 2, 2, out_len=15),
    ):
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == "LengthMismatch"


# ----------------------------------------------------------- attention -----

ATT_FIELDS = ("batch", "layers", "layer", "heads", "kv_heads", "seq", "past_len", "head_dim", "max_seq")


def _kv_append64(k, v, cache, s):
    cache = f64(cache).reshape(s["batch"], s["layers"], 2, s["max_seq"], s["kv_heads"], s["head_dim"])
    kk = f64(k).reshape(s["batch"], s["kv_heads"], s["seq"], s["head_dim"])
    vv = f64(v).reshape(s["batch"], s["kv_heads"], s["seq"], s["head_dim"])
    t0, t1 = s["past_len"], s["past_len"] + s["seq"]
    cache[:, s["layer"], 0, t0:t1] = kk.transpose(0, 2, 1, 3)
    cache[:, s["layer"], 1, t0:t1] = vv.transpose(0, 2, 1, 3)
    return cache


def _attention64(q, k, v, cache0, s, scale):
    cache = _kv_append64(k, v, cache0, s)
    B, H, S, D = s["batch"], s["heads"], s["seq"], s["head_dim"]
    group = H // s["kv_heads"]
    qq = f64(q).reshape(B, H, S, D)
    out = np.zeros((B, H, S, D))
    for b in range(B):
        for h in range(H):
            kv = h // group
            for t in range(S):
                n = s["past_len"] + t + 1
                keys = cache[b, s["layer"], 0, :n, kv]
                vals = cache[b, s["layer"], 1, :n, kv]
                sc = keys @ qq[b, h, t] * float(np.float32(scale))
                p = np.exp(sc - sc.max())
                out[b, h, t] = (p / p.sum()) @ vals
    return out, cache


def _shape(*vals):
    return dict(zip(ATT_FIELDS, vals))


KV_CASES = [
    (1, _shape(1, 1, 0, 1, 1, 2, 0, 2, 4)),
    (2, _shape(2, 2, 1, 2, 2, 3, 2, 3, 5)),
    (3, _shape(1, 1, 0, 2, 2, 1, 0, 8, 1)),
    (4, _shape(1, 1, 0, 1, 1, 0, 2, 4, 4)),
]


def _kv_len(s):
    return s["batch"] * s["kv_heads"] * s["seq"] * s["head_dim"]


def _cache_len(s):
    return s["batch"] * s["layers"] * 2 * s["max_seq"] * s["kv_heads"] * s["head_dim"]


@pytest.mark.parametrize("seed,s", KV_CASES)
def test_kv_append_matches_f64_oracle(oracle, seed, s):
    """attention.rs:405-467."""
    lcg = Lcg(seed)
    k = lcg.fill(_kv_len(s), -1.0, 1.0)
    v = lcg.fill(_kv_len(s), -1.0, 1.0)
    cache = lcg.fill(_cache_len(s), -1.0, 1.0)
    out = oracle.kv_append(k, v, cache, s["batch"], s["layers"], s["layer"], s["kv_heads"],
                           s["head_dim"], s["max_seq"], s["past_len"], s["seq"])
    assert_close(out, _kv_append64(k, v, cache, s))


def test_kv_append_rejects_invalid_shapes(oracle):
    """attention.rs:469-507."""
    k = np.zeros(8, np.float32)
    v = np.zeros(8, np.float32)
    cache = np.zeros(24, np.float32)
    cases = [
        (lambda: oracle.kv_append(k[:-1], v, cache, 1, 1, 0, 1, 4, 3, 1, 2), "LengthMismatch"),
        (lambda: oracle.kv_append(k, v[:-1], cache, 1, 1, 0, 1, 4, 3, 1, 2), "LengthMismatch"),
        (lambda: oracle.kv_append(k, v, cache[:-1], 1, 1, 0, 1, 4, 3, 1, 2), "LengthMismatch"),
        (lambda: oracle.kv_append(k, v, cache, 1, 1, 1, 1, 4, 3, 1, 2), "InvalidShape"),
        (lambda: oracle.kv_append(k, v, cache, 1, 1, 0, 1, 4, 3, 2, 2), "InvalidShape"),
    ]
    for call, kind in cases:
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == kind


def test_kv_append_writes_documented_layout(oracle):
    """attention.rs:509-527: cache [1, 2, 2, 3, 1, 2], layer 1, past 1 → indices 14,15 / 20,21."""
    cache = oracle.kv_append([1.0, 2.0], [3.0, 4.0], np.zeros(24), 1, 2, 1, 1, 2, 3, 1, 1)
    assert list(cache[14:16]) == [1.0, 2.0]
    assert list(cache[20:22]) == [3.0, 4.0]
    assert np.count_nonzero(cache) == 4


def test_causal_attention_matches_hand_computed_decode(oracle):
    """attention.rs:529-542: one key, so the output is that key's value [3, 4]."""
    out, _ = oracle.causal_attention([1.0, 0.0], [1.0, 0.0], [3.0, 4.0], np.zeros(4), 1, 1, 0, 1, 1,
                                     1, 0, 2, 1, 1.0)
    assert_close(out, [3.0, 4.0])


ATT_CASES = [
    (11, _shape(1, 1, 0, 2, 2, 3, 0, 4, 4)),
    (12, _shape(2, 1, 0, 2, 2, 1, 3, 8, 6)),
    (13, _shape(2, 2, 1, 4, 2, 2, 2, 8, 5)),
    (14, _shape(2, 1, 0, 2, 1, 1, 5, 2, 7)),
    (15, _shape(1, 1, 0, 6, 3, 2, 1, 4, 4)),
    (16, _shape(1, 1, 0, 3, 1, 1, 2, 4, 3)),
]


def _run_attention(oracle, s, seed):
    lcg = Lcg(seed)
    qlen = s["batch"] * s["heads"] * s["seq"] * s["head_dim"]
    q = lcg.fill(qlen, -1.0, 1.0)
    k = lcg.fill(_kv_len(s), -1.0, 1.0)
    v = lcg.fill(_kv_len(s), -1.0, 1.0)
    cache = lcg.fill(_cache_len(s), -1.0, 1.0)
    scale = np.float32(1.0 / math.sqrt(s["head_dim"]))
    out, new_cache = oracle.causal_attention(q, k, v, cache, s["batch"], s["layers"], s["layer"],
                                             s["heads"], s["kv_heads"], s["seq"], s["past_len"],
                                             s["head_dim"], s["max_seq"], float(scale))
    return (q, k, v, cache, scale), out, new_cache


@pytest.mark.parametrize("seed,s", ATT_CASES)
def test_causal_attention_matches_f64_oracle(oracle, seed, s):
    """attention.rs:544-634 (MHA, decode, GQA 2x, MQA, GQA 6/3, MQA 3/1)."""
    (q, k, v, cache, scale), out, new_cache = _run_attention(oracle, s, seed)
    exp_out, exp_cache = _attention64(q, k, v, cache, s, scale)
    assert_close(out, exp_out)
    assert_close(new_cache, exp_cache)


def test_causal_attention_accepts_empty_sequence(oracle):
    """attention.rs:636-675."""
    s = _shape(1, 1, 0, 1, 1, 0, 2, 4, 4)
    cache = Lcg(21).fill(_cache_len(s), -1.0, 1.0)
    e = np.zeros(0, np.float32)
    out, new_cache = oracle.causal_attention(e, e, e, cache, 1, 1, 0, 1, 1, 0, 2, 4, 4, 0.5)
    assert out.size == 0
    assert np.array_equal(new_cache, cache)


def test_causal_attention_rejects_invalid_shapes(oracle):
    """attention.rs:677-787."""
    q = np.zeros(16, np.float32)
    k = np.zeros(16, np.float32)
    v = np.zeros(16, np.float32)
    cache = np.zeros(48, np.float32)

    def call(heads, kv_heads, layer, past, qq=q, cc=cache, out_len=None):
        return oracle.causal_attention(qq, k, v, cc, 1, 1, layer, heads, kv_heads, 2, past, 4, 3, 0.5,
                                       out_len=16 if out_len is None else out_len)

    cases = [
        (lambda: call(3, 2, 0, 1), "InvalidShape"),
        (lambda: call(0, 0, 0, 1), "InvalidShape"),
        (lambda: call(0, 1, 0, 1), "InvalidShape"),
        (lambda: call(2, 2, 1, 1), "InvalidShape"),
        (lambda: call(2, 2, 0, 2), "InvalidShape"),
        (lambda: call(2, 2, 0, 1, qq=q[:-1]), "LengthMismatch"),
        (lambda: call(2, 2, 0, 1, out_len=15), "LengthMismatch"),
        (lambda: call(2, 2, 0, 1, cc=cache[:-1]), "LengthMismatch"),
    ]
    for fn, kind in cases:
        with pytest.raises(OracleError) as err:
            fn()
        assert err.value.kind == kind


# -------------------------------------------------------------- swiglu -----


def _swiglu64(x, g, u, d, rows, hidden, inter):
    x = f64(x).reshape(rows, hidden)
    gate = x @ f64(g).reshape(inter, hidden).T
    up = x @ f64(u).reshape(inter, hidden).T
    h = gate / (1.0 + np.exp(-gate)) * up
    return h @ f64(d).reshape(hidden, inter).T


@pytest.mark.parametrize("rows,hidden,inter,seed", [(1, 1, 1, 1), (3, 5, 7, 2), (2, 8, 4, 3),
                                                    (4, 6, 13, 4)])
def test_swiglu_matches_f64_oracle(oracle, rows, hidden, inter, seed):
    """swiglu.rs:144-150."""
    lcg = Lcg(seed)
    x = lcg.fill(rows * hidden, -1.0, 1.0)
    g = lcg.fill(inter * hidden, -1.0, 1.0)
    u = lcg.fill(inter * hidden, -1.0, 1.0)
    d = lcg.fill(hidden * inter, -1.0, 1.0)
    assert_close(oracle.swiglu(x, g, u, d, rows, hidden, inter),
                 _swiglu64(x, g, u, d, rows, hidden, inter))


def test_swiglu_zero_rows_and_invalid_shapes(oracle):
    """swiglu.rs:152-200."""
    e = np.zeros(0, np.float32)
    oracle.swiglu(e, np.full(6, 0.5), np.full(6, 0.25), np.full(6, 0.75), 0, 3, 2)
    for h, i in ((0, 2), (2, 0)):
        with pytest.raises(OracleError) as err:
            oracle.swiglu(e, e, e, e, 0, h, i, out_len=0)
        assert err.value.kind == "InvalidShape"
    x, w = np.ones(4), np.ones(8)
    for call in (
        lambda: oracle.swiglu(x[:3], w, w, w, 2, 2, 4),
        lambda: oracle.swiglu(x, w[:7], w, w, 2, 2, 4),
        lambda: oracle.swiglu(x, w, w[:7], w, 2, 2, 4),
        lambda: oracle.swiglu(x, w, w, w[:7], 2, 2, 4),
        lambda: oracle.swiglu(x, w, w, w, 2, 2, 4, out_len=3),
    ):
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == "LengthMismatch"


# ------------------------------------------------------- rms_norm_matmul ---


@pytest.mark.parametrize("rows,hidden,out_f,eps,seed", [(1, 1, 1, 1e-5, 1), (3, 7, 5, 1e-6, 2),
                                                        (2, 33, 17, 1e-5, 3), (4, 16, 9, 1e-6, 4)])
def test_rms_norm_matmul_matches_f64_oracle(oracle, rows, hidden, out_f, eps, seed):
    """fused.rs:346-353."""
    lcg = Lcg(seed)
    x = lcg.fill(rows * hidden, -2.0, 2.0)
    wt = lcg.fill(hidden, 0.5, 1.5)
    w = lcg.fill(out_f * hidden, -1.0, 1.0)
    expected = _rms64(x, wt, rows, hidden, eps) @ f64(w).reshape(out_f, hidden).T
    assert_close(oracle.rms_norm_matmul(x, wt, w, rows, hidden, out_f, eps), expected)


def test_rms_norm_matmul_zero_rows_and_invalid_shapes(oracle):
    """fused.rs:355-401."""
    e = np.zeros(0, np.float32)
    oracle.rms_norm_matmul(e, [1.0, 0.5, 2.0], np.ones(6), 0, 3, 2, 1e-5)
    for h, o in ((0, 3), (4, 0)):
        with pytest.raises(OracleError) as err:
            oracle.rms_norm_matmul(e, e, e, 2, h, o, 1e-5, out_len=0)
        assert err.value.kind == "InvalidShape"
    x, wt, w = np.ones(8), np.ones(4), np.ones(12)
    for call in (
        lambda: oracle.rms_norm_matmul(x[:7], wt, w, 2, 4, 3, 1e-5),
        lambda: oracle.rms_norm_matmul(x, wt[:3], w, 2, 4, 3, 1e-5),
        lambda: oracle.rms_norm_matmul(x, wt, w[:11], 2, 4, 3, 1e-5),
        lambda: oracle.rms_norm_matmul(x, wt, w, 2, 4, 3, 1e-5, out_len=5),
    ):
        with pytest.raises(OracleError) as err:
            call()
        assert err.value.kind == "LengthMismatch"
    with pytest.raises(OracleError) as err:
        oracle.rms_norm_matmul(e, wt, w, 2**64 - 1, 4, 3, 1e-5, out_len=0)
    assert err.value.kind == "ShapeOverflow"
