"""sl_hip_paged_attention on the GPU against the oracle's paged decode
attention (itself equal bit for bit to the contiguous reference attention,
tests/test_paged.py): rows of different lengths in one batch, pages in
shuffled order, a continuous-batching run whose sequences leave and join
(pages released and reused), and the errors for a bad block table.

Attention outputs within 1e-4 normwise per (row, head); the page pool,
whose only change is the appended K/V rows, bit for bit.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import assert_normwise
from starlight_amd.device import DeviceError
from starlight_amd.ir import BufferRef, Op
from starlight_amd.paged import PagedKvCache, PagePool

pytestmark = pytest.mark.gpu

H, HKV, D, LAYERS = 32, 8, 128, 2
SCALE = float(np.float32(1.0 / math.sqrt(D)))


def upload(hip, a):
    b = hip.upload_new_f32(a)
    return BufferRef(b, 0, a.size)


def run_step(hip, cache, pool_host, layer, rng, batch, h=H, hkv=HKV, d=D):
    """One decode step on the GPU and the oracle; returns the oracle pool."""
    scale = float(np.float32(1.0 / math.sqrt(d)))
    q = rng.uniform(-1, 1, batch * h * d).astype(np.float32)
    k = rng.uniform(-1, 1, batch * hkv * d).astype(np.float32)
    v = rng.uniform(-1, 1, batch * hkv * d).astype(np.float32)
    out = hip.allocate_f32(batch * h * d, 256)
    cache.sync()
    cache.attention(Op.causal_attention(layer, h, hkv, d, scale), upload(hip, q), upload(hip, k), upload(hip, v),
                    BufferRef(out, 0, batch * h * d), batch)
    got = hip.read_f32(out, batch * h * d)
    p = cache.pool
    want, new_pool = oracle.paged_attention_decode(q, k, v, pool_host, p.tables()[:batch].ravel(),
                                                   p.seq_lens()[:batch], batch, LAYERS, layer, p.num_pages,
                                                   p.page_size, p.pages_per_seq, h, hkv, d, scale)
    for i in range(batch * h):
        assert_normwise(got[i * d:(i + 1) * d], want[i * d:(i + 1) * d])
    return new_pool


def test_mixed_lengths_shuffled_pages(hip):
    """Four rows at 0, 37, 100 and 1030 cached positions (8B decode shapes,
    16-position pages handed out in shuffled order)."""
    rng = np.random.default_rng(50)
    pool = PagePool(num_pages=4 * 80 + 8, page_size=16, pages_per_seq=80, max_batch=4)
    rng.shuffle(pool.free)
    cache = PagedKvCache(hip, LAYERS, HKV, D, pool)
    host = rng.uniform(-1, 1, cache.pool_elements).astype(np.float32)
    hip.upload_f32(cache.pool_buffer, host)
    for seq, n in enumerate([0, 37, 100, 1030]):
        pool.admit(seq)
        pool.set_length(seq, n)
    want_pool = run_step(hip, cache, host, 1, rng, 4)
    np.testing.assert_array_equal(hip.read_f32(cache.pool_buffer, cache.pool_elements), want_pool)


@pytest.mark.parametrize("lengths", [[0, 300, 550, 2040], [1500]])
def test_mixed_lengths_head_dim_64(hip, lengths):
    """The 1B decode geometry (32 query heads over 8 KV heads of 64, 8-key
    tiles, one partial per 64 positions of a row's 2048-position capacity up
    to the grid's cap): four rows at 0-2040 positions, and one row alone at
    1500 (32 partials)."""
    rng = np.random.default_rng(51 + len(lengths))
    b = len(lengths)
    pool = PagePool(num_pages=b * 128 + 8, page_size=16, pages_per_seq=128, max_batch=b)
    rng.shuffle(pool.free)
    cache = PagedKvCache(hip, LAYERS, 8, 64, pool)
    host = rng.uniform(-1, 1, cache.pool_elements).astype(np.float32)
    hip.upload_f32(cache.pool_buffer, host)
    for seq, n in enumerate(lengths):
        pool.admit(seq)
        pool.set_length(seq, n)
    want_pool = run_step(hip, cache, host, 0, rng, b, h=32, hkv=8, d=64)
    np.testing.assert_array_equal(hip.read_f32(cache.pool_buffer, cache.pool_elements), want_pool)


def test_continuous_batching_with_page_reuse(hip):
    """Eight steps: rows advance one position a step; after step 3 sequence 1
    leaves and a new one takes its row from position 0 with recycled pages;
    after step 5 a fourth row joins. Every step's outputs and the final pool
    match the oracle."""
    rng = np.random.default_rng(51)
    pool = PagePool(num_pages=40, page_size=16, pages_per_seq=12, max_batch=4)
    cache = PagedKvCache(hip, LAYERS, HKV, D, pool)
    host = rng.uniform(-1, 1, cache.pool_elements).astype(np.float32)
    hip.upload_f32(cache.pool_buffer, host)
    for seq, n in enumerate([5, 40, 17]):
        pool.admit(seq)
        pool.set_length(seq, n)
    next_seq = 3
    for step in range(8):
        batch = max(pool.rows.values()) + 1
        host = run_step(hip, cache, host, step % LAYERS, rng, batch)
        for seq in list(pool.rows):
            pool.set_length(seq, pool.lengths[seq] + 1)
        if step == 3:
            freed = list(pool.pages[1])
            pool.release(1)
            pool.admit(next_seq)
            pool.set_length(next_seq, 0)
            assert pool.pages[next_seq][0] in freed  # a recycled page
            next_seq += 1
        if step == 5:
            pool.admit(next_seq)
            pool.set_length(next_seq, 3)
            next_seq += 1
    np.testing.assert_array_equal(hip.read_f32(cache.pool_buffer, cache.pool_elements), host)


def test_rows_sharing_a_read_only_prefix_page(hip):
    """Rows 0 and 1 (40 positions each) share their first page, which both
    only read: allowed, and the shared page is left unchanged."""
    rng = np.random.default_rng(52)
    pool = PagePool(num_pages=12, page_size=16, pages_per_seq=4, max_batch=2)
    cache = PagedKvCache(hip, LAYERS, HKV, D, pool)
    host = rng.uniform(-1, 1, cache.pool_elements).astype(np.float32)
    hip.upload_f32(cache.pool_buffer, host)
    for seq in range(2):
        pool.admit(seq)
        pool.set_length(seq, 40)
    shared = pool.pages[0][0]
    pool.free.append(pool.pages[1][0])
    pool.pages[1][0] = shared
    new_pool = run_step(hip, cache, host, 0, rng, 2)
    got = hip.read_f32(cache.pool_buffer, cache.pool_elements)
    np.testing.assert_array_equal(got, new_pool)
    page = 2 * 16 * HKV * D
    for layer in range(LAYERS):
        base = (layer * pool.num_pages + shared) * page
        np.testing.assert_array_equal(got[base:base + page], host[base:base + page])


@pytest.mark.parametrize("case,message", [
    ("page_out_of_range", "page id out of range"),
    ("past_table", "paged KV length exceeds the row's block table"),
    ("shared_write", "a row appends into a page another row reads"),
    ("appends_into_read_page", "a row appends into a page another row reads"),
])
def test_bad_block_tables_are_rejected(hip, case, message):
    pool = PagePool(num_pages=8, page_size=16, pages_per_seq=2, max_batch=2)
    cache = PagedKvCache(hip, LAYERS, HKV, D, pool)
    for seq, n in enumerate([20, 3]):
        pool.admit(seq)
        pool.set_length(seq, n)
    tables, lens = pool.tables(), pool.seq_lens()
    if case == "page_out_of_range":
        tables[1, 0] = 8
    elif case == "past_table":
        lens[0] = 32
    elif case == "shared_write":       # both rows append into one page
        tables[1, 0] = tables[0, 1]
        lens[1] = 5
    else:                              # row 1 appends into row 0's first page
        tables[1, 0] = tables[0, 0]
    hip.upload_u32(cache.table_buffer, tables.ravel())
    hip.upload_u32(cache.lens_buffer, lens)
    q = upload(hip, np.zeros(2 * H * D, np.float32))
    kv = upload(hip, np.zeros(2 * HKV * D, np.float32))
    kv2 = upload(hip, np.zeros(2 * HKV * D, np.float32))
    out = hip.allocate_f32(2 * H * D, 256)
    with pytest.raises(DeviceError) as e:
        hip.paged_attention(Op.causal_attention(0, H, HKV, D, SCALE), q, kv, kv2, BufferRef(out, 0, 2 * H * D), 2,
                            cache.c_struct())
    assert e.value == DeviceError.execution(message)


def test_empty_batch_is_a_no_op(hip):
    """A batch of no rows validates its arguments and launches nothing:
    the page pool is unchanged."""
    pool = PagePool(num_pages=4, page_size=16, pages_per_seq=2, max_batch=2)
    cache = PagedKvCache(hip, LAYERS, HKV, D, pool)
    host = np.random.default_rng(51).uniform(-1, 1, cache.pool_elements).astype(np.float32)
    hip.upload_f32(cache.pool_buffer, host)
    cache.sync()
    empty = BufferRef(hip.allocate_f32(16, 256), 0, 0)
    out = BufferRef(hip.allocate_f32(16, 256), 0, 0)
    hip.paged_attention(Op.causal_attention(0, H, HKV, D, SCALE), empty, empty, empty, out, 0, cache.c_struct())
    hip.synchronize()
    np.testing.assert_array_equal(hip.read_f32(cache.pool_buffer, cache.pool_elements), host)
