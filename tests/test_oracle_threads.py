"""The oracle's threaded loops give the single-threaded results bit for bit:
each output element is still computed by one thread in the reference's
order (matmul.rs:29-59, attention.rs:129-219, swiglu.rs:40-84,
fused.rs:41-90)."""
import numpy as np
import pytest

import oracle


@pytest.fixture
def threads():
    before = oracle.get_threads()
    yield
    oracle.set_threads(before)


def both(fn):
    oracle.set_threads(1)
    one = fn()
    oracle.set_threads(8)
    many = fn()
    return one, many


def test_matmul_nt_and_nn_threads_bit_identical(threads):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 7, 33)).astype(np.float32)
    b = rng.standard_normal((3, 29, 33)).astype(np.float32)
    one, many = both(lambda: oracle.matmul_nt(a, b, 3, 7, 33, 29))
    assert one.tobytes() == many.tobytes()
    bn = rng.standard_normal((3, 33, 29)).astype(np.float32)
    one, many = both(lambda: oracle.matmul_nn(a, bn, 3, 7, 33, 29))
    assert one.tobytes() == many.tobytes()


def test_attention_threads_bit_identical(threads):
    rng = np.random.default_rng(1)
    B, L, H, Hkv, S, D, past, max_seq = 2, 2, 8, 2, 3, 16, 5, 12
    q = rng.standard_normal(B * H * S * D).astype(np.float32)
    k = rng.standard_normal(B * Hkv * S * D).astype(np.float32)
    v = rng.standard_normal(B * Hkv * S * D).astype(np.float32)
    cache = rng.standard_normal(B * L * 2 * max_seq * Hkv * D).astype(np.float32)

    def run():
        out, new = oracle.causal_attention(q, k, v, cache.copy(), B, L, 1, H, Hkv, S, past, D, max_seq, 0.25)
        return np.concatenate([out, new])

    one, many = both(run)
    assert one.tobytes() == many.tobytes()


def test_swiglu_and_rms_norm_matmul_threads_bit_identical(threads):
    rng = np.random.default_rng(2)
    rows, hidden, inter = 3, 24, 40
    x = rng.standard_normal(rows * hidden).astype(np.float32)
    wg = rng.standard_normal(inter * hidden).astype(np.float32)
    wu = rng.standard_normal(inter * hidden).astype(np.float32)
    wd = rng.standard_normal(hidden * inter).astype(np.float32)
    one, many = both(lambda: oracle.swiglu(x, wg, wu, wd, rows, hidden, inter))
    assert one.tobytes() == many.tobytes()
    g = rng.standard_normal(hidden).astype(np.float32)
    w = rng.standard_normal(inter * hidden).astype(np.float32)
    one, many = both(lambda: oracle.rms_norm_matmul(x, g, w, rows, hidden, inter, 1e-5))
    assert one.tobytes() == many.tobytes()
