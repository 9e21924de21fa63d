"""Paged KV cache on the CPU: the oracle's paged decode attention against the
contiguous reference attention (attention.rs:129-219, slr_causal_attention)
bit for bit, for pages in order, in shuffled order and for rows of different
lengths; its errors; and the host page pool (allocation, release, reuse).
"""
import numpy as np
import pytest

import oracle
from oracle import OracleError
from starlight_amd.paged import OutOfPages, PagePool

L, HKV, H, D, PS = 2, 2, 8, 64, 16


def contiguous_reference(q, k, v, cache, past, layer, max_seq):
    """One row (batch 1) through the contiguous oracle."""
    out, new = oracle.causal_attention(q, k, v, cache, 1, L, layer, H, HKV, 1, past, D, max_seq, 0.125)
    return out, new


def paged_from_contiguous(caches, tables, num_pages, pages_per_seq):
    """Scatters each row's contiguous cache [L, 2, max_seq, HKV, D] into the
    pages its table names."""
    pool = np.zeros((L, num_pages, 2, PS, HKV, D), np.float32)
    for row, (cache, table) in enumerate(zip(caches, tables)):
        c = cache.reshape(L, 2, pages_per_seq * PS, HKV, D)
        for pi, page in enumerate(table):
            pool[:, page] = c[:, :, pi * PS:(pi + 1) * PS]
    return pool


@pytest.mark.parametrize("order", ["identity", "shuffled"])
@pytest.mark.parametrize("lengths", [[0], [37], [16], [100, 5, 63]])
def test_paged_oracle_equals_the_contiguous_reference(order, lengths):
    r = np.random.default_rng(len(lengths) * 7 + sum(lengths))
    B = len(lengths)
    pages_per_seq = 8
    max_seq = pages_per_seq * PS
    num_pages = B * pages_per_seq + 3
    ids = np.arange(num_pages)
    if order == "shuffled":
        r.shuffle(ids)
    tables = ids[:B * pages_per_seq].reshape(B, pages_per_seq).astype(np.uint32)
    caches = [r.uniform(-1, 1, L * 2 * max_seq * HKV * D).astype(np.float32) for _ in range(B)]
    q = r.uniform(-1, 1, B * H * D).astype(np.float32)
    k = r.uniform(-1, 1, B * HKV * D).astype(np.float32)
    v = r.uniform(-1, 1, B * HKV * D).astype(np.float32)
    pool = paged_from_contiguous(caches, tables, num_pages, pages_per_seq)
    layer = 1
    out, new_pool = oracle.paged_attention_decode(q, k, v, pool.ravel(), tables.ravel(), np.array(lengths, np.uint32),
                                                  B, L, layer, num_pages, PS, pages_per_seq, H, HKV, D, 0.125)
    want_pool_rows = []
    for b, past in enumerate(lengths):
        want, new_cache = contiguous_reference(q[b * H * D:(b + 1) * H * D], k[b * HKV * D:(b + 1) * HKV * D],
                                               v[b * HKV * D:(b + 1) * HKV * D], caches[b], past, layer, max_seq)
        assert out[b * H * D:(b + 1) * H * D].tobytes() == want.tobytes()
        want_pool_rows.append(new_cache)
    assert new_pool.tobytes() == paged_from_contiguous(want_pool_rows, tables, num_pages, pages_per_seq).tobytes()
    # pages no table names are untouched
    unused = sorted(set(range(num_pages)) - set(tables.ravel().tolist()))
    np.testing.assert_array_equal(new_pool.reshape(pool.shape)[:, unused], pool[:, unused])


def test_paged_oracle_errors():
    pool = np.zeros(L * 4 * 2 * PS * HKV * D, np.float32)
    q = np.zeros(H * D, np.float32)
    kv = np.zeros(HKV * D, np.float32)
    with pytest.raises(OracleError, match="page id out of range"):
        oracle.paged_attention_decode(q, kv, kv, pool, np.array([9, 0], np.uint32), np.array([3], np.uint32), 1, L,
                                      0, 4, PS, 2, H, HKV, D, 1.0)
    with pytest.raises(OracleError, match="exceeds the row's block table"):
        oracle.paged_attention_decode(q, kv, kv, pool, np.array([0, 1], np.uint32), np.array([32], np.uint32), 1, L,
                                      0, 4, PS, 2, H, HKV, D, 1.0)
    q2, kv2 = np.zeros(2 * H * D, np.float32), np.zeros(2 * HKV * D, np.float32)
    with pytest.raises(OracleError, match="another row reads"):
        oracle.paged_attention_decode(q2, kv2, kv2, pool, np.array([0, 1, 1, 2], np.uint32),
                                      np.array([20, 3], np.uint32), 2, L, 0, 4, PS, 2, H, HKV, D, 1.0)


def test_page_pool_allocates_releases_and_reuses():
    pool = PagePool(num_pages=6, page_size=16, pages_per_seq=4, max_batch=3)
    a, b = pool.admit("a"), pool.admit("b")
    assert (a, b) == (0, 1)
    pool.set_length("a", 20)        # positions 0..20 -> 2 pages
    pool.set_length("b", 15)        # 0..15 -> 1 page
    assert pool.pages["a"] == [0, 1] and pool.pages["b"] == [2]
    t = pool.tables()
    assert t.shape == (3, 4) and list(t[0, :2]) == [0, 1] and t[1, 0] == 2
    assert list(pool.seq_lens()) == [20, 15, 0]
    pool.release("a")
    assert pool.admit("c") == 0     # the freed row
    pool.set_length("c", 40)        # 3 pages: the two freed ones first
    assert sorted(pool.pages["c"][:2]) == [0, 1]
    with pytest.raises(OutOfPages):
        pool.set_length("b", 63)    # needs 4 pages, 2 free: nothing is taken
    assert pool.pages["b"] == [2] and len(pool.free) == 2
    with pytest.raises(ValueError, match="exceeds the block table"):
        pool.set_length("c", 64)
    with pytest.raises(ValueError, match="already admitted"):
        pool.admit("b")
