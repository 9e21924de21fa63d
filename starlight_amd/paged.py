"""Paged KV cache: host-side page management and the device binding of
`sl_hip_paged_attention` (no reference counterpart: gaps G-17 paged KV
cache and G-18 per-request lengths, ARCH-0008:123-124).

A pool of `num_pages` pages, each holding `page_size` positions of every
layer's K and V ([layer][page][K, V][slot][kv_head][head_dim] on the
device). Sequences occupy batch rows; each row has a block table of
`pages_per_seq` page ids and a cached length. Pages are taken from a free
list as a sequence grows and returned when it leaves, so rows of different
lengths decode together and a finished sequence's pages serve the next one.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional

import numpy as np

from . import ir


class OutOfPages(Exception):
    """The pool has no free page for a sequence that grows."""


class PagePool:
    """Free list and block tables of a paged KV cache (host side)."""

    def __init__(self, num_pages: int, page_size: int, pages_per_seq: int, max_batch: int):
        self.num_pages, self.page_size, self.pages_per_seq, self.max_batch = num_pages, page_size, pages_per_seq, \
            max_batch
        self.free: List[int] = list(range(num_pages - 1, -1, -1))  # pop() hands out low ids first
        self.rows: Dict[object, int] = {}        # sequence id -> batch row
        self.pages: Dict[object, List[int]] = {}
        self.lengths: Dict[object, int] = {}

    def admit(self, seq) -> int:
        """Gives sequence `seq` a free batch row (length 0, no pages)."""
        if seq in self.rows:
            raise ValueError(f"sequence {seq!r} is already admitted")
        used = set(self.rows.values())
        row = next((r for r in range(self.max_batch) if r not in used), None)
        if row is None:
            raise ValueError("every batch row is in use")
        self.rows[seq], self.pages[seq], self.lengths[seq] = row, [], 0
        return row

    def reserve(self, seq, length: int) -> None:
        """Makes positions 0..length-1 of `seq` addressable, taking pages from
        the free list (OutOfPages, taking none, when too few are free)."""
        need = (length + self.page_size - 1) // self.page_size
        if need > self.pages_per_seq:
            raise ValueError(f"length {length} exceeds the block table ({self.pages_per_seq} pages)")
        pages = self.pages[seq]
        if need - len(pages) > len(self.free):
            raise OutOfPages(f"no free page for sequence {seq!r}")
        while len(pages) < need:
            pages.append(self.free.pop())

    def set_length(self, seq, length: int) -> None:
        self.reserve(seq, length + 1)  # the next step appends at position `length`
        self.lengths[seq] = length

    def release(self, seq) -> None:
        """Returns the sequence's pages to the free list and frees its row."""
        self.free.extend(reversed(self.pages.pop(seq)))
        del self.rows[seq], self.lengths[seq]

    def tables(self) -> np.ndarray:
        """[max_batch, pages_per_seq] u32 block tables (unused entries 0)."""
        t = np.zeros((self.max_batch, self.pages_per_seq), np.uint32)
        for seq, row in self.rows.items():
            p = self.pages[seq]
            t[row, :len(p)] = p
        return t

    def seq_lens(self) -> np.ndarray:
        """[max_batch] u32 cached lengths (0 for unused rows)."""
        n = np.zeros(self.max_batch, np.uint32)
        for seq, row in self.rows.items():
            n[row] = self.lengths[seq]
        return n


class CPagedKv(ctypes.Structure):
    """sl_paged_kv."""
    _fields_ = [("pool", ctypes.c_uint32), ("block_table", ctypes.c_uint32), ("seq_lens", ctypes.c_uint32),
                ("layers", ctypes.c_uint32), ("num_pages", ctypes.c_uint32), ("page_size", ctypes.c_uint32),
                ("pages_per_seq", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class PagedKvCache:
    """A PagePool bound to device buffers: the page pool (f32), the block
    tables and the lengths (u32, uploaded by `sync`)."""

    def __init__(self, device, layers: int, kv_heads: int, head_dim: int, pool: PagePool):
        self.device, self.pool = device, pool
        self.layers, self.kv_heads, self.head_dim = layers, kv_heads, head_dim
        self.pool_elements = layers * pool.num_pages * 2 * pool.page_size * kv_heads * head_dim
        self.pool_buffer = device.allocate_f32(self.pool_elements, 256)
        self.table_buffer = device.allocate_u32(pool.max_batch * pool.pages_per_seq, 256)
        self.lens_buffer = device.allocate_u32(pool.max_batch, 256)

    def sync(self) -> None:
        """Uploads the block tables and lengths of the pool's current state."""
        self.device.upload_u32(self.table_buffer, self.pool.tables().ravel())
        self.device.upload_u32(self.lens_buffer, self.pool.seq_lens())

    def c_struct(self) -> CPagedKv:
        p = self.pool
        return CPagedKv(self.pool_buffer, self.table_buffer, self.lens_buffer, self.layers, p.num_pages, p.page_size,
                        p.pages_per_seq, 0)

    def attention(self, op: ir.Op, q: ir.BufferRef, k_new: ir.BufferRef, v_new: ir.BufferRef,
                  out: ir.BufferRef, batch: Optional[int] = None) -> None:
        """sl_hip_paged_attention over rows 0..batch-1 at their current
        lengths (the highest admitted row + 1 by default). Every one of those
        rows must hold a sequence: each row appends its new K/V, so an empty
        row would write into the page its zeroed table names."""
        rows = set(self.pool.rows.values())
        if batch is None:
            batch = max(rows) + 1 if rows else 0
        missing = [r for r in range(batch) if r not in rows]
        if missing:
            raise ValueError(f"rows {missing} hold no sequence")
        self.device.paged_attention(op, q, k_new, v_new, out, batch, self.c_struct())

    def bind_state(self, state_buffer: int) -> None:
        """Binds a decode program's KV State buffer to this cache
        (sl_hip_bind_paged_state): its CausalAttention commands then read
        and append through the block tables at each row's own length."""
        self.device.bind_paged_state(state_buffer, self.c_struct())

    def store(self, seq, state_buffer: int, index: int, max_seq: int, length: int) -> None:
        """Copies positions [0, length) of batch index `index` of a
        contiguous KV State (a prefill program's) into `seq`'s pages, which
        must already be reserved (sl_hip_paged_store)."""
        self.sync()
        self.device.paged_store(self.c_struct(), self.pool.rows[seq], state_buffer, index, max_seq, self.kv_heads,
                                self.head_dim, length)


class ContinuousBatcher:
    """Continuous batching through the engine: the per-step calls a request
    scheduler makes (the scheduler itself, admission policy and sampling
    are the control plane's and not part of this backend).

    A batch-1 prefill engine runs each new prompt on its own contiguous KV
    State (padded to the compiled prompt length; LastToken takes the last
    real token), and the prompt's K/V rows are stored into the sequence's
    pages. A batch-`max_batch` decode engine, whose KV State is bound to the
    paged cache, then decodes every admitted sequence in one step at its own
    length: row b reads its seq_lens[b] cached positions and appends one.
    Rows without a sequence hold a placeholder with one page of its own, so
    every row's append has a page no other row reads; their logits are
    ignored.
    """

    def __init__(self, device, prefill_engine, prefill_state: int, prefill_max_seq: int, prompt_capacity: int,
                 decode_engine, decode_state: int, cache: PagedKvCache, vocab: int):
        self.device, self.cache, self.pool = device, cache, cache.pool
        self.prefill_engine, self.prefill_state = prefill_engine, prefill_state
        self.prefill_max_seq, self.prompt_capacity = prefill_max_seq, prompt_capacity
        self.decode_engine, self.vocab = decode_engine, vocab
        self.batch = self.pool.max_batch
        self._idle = {}  # row -> placeholder key
        for row in range(self.batch):
            self._park(row)
        self._tables = None
        cache.bind_state(decode_state)

    def _park(self, row: int) -> None:
        key = ("idle", row)
        assert self.pool.admit(key) == row
        self.pool.set_length(key, 0)
        self._idle[row] = key

    def sync(self) -> None:
        """Uploads the block tables (when they changed) and the lengths."""
        tables = self.pool.tables()
        if self._tables is None or not np.array_equal(tables, self._tables):
            self.device.upload_u32(self.cache.table_buffer, tables.ravel())
            self._tables = tables
        self.device.upload_u32(self.cache.lens_buffer, self.pool.seq_lens())

    def sequences(self) -> Dict[object, int]:
        """Active sequence -> batch row."""
        return {s: r for s, r in self.pool.rows.items() if not (isinstance(s, tuple) and s[:1] == ("idle",))}

    def admit(self, seq, prompt) -> np.ndarray:
        """Prefills `prompt` for a new sequence in a free row and returns the
        logits of its last token."""
        prompt = np.asarray(prompt, np.uint32)
        n = prompt.size
        if n == 0 or n > self.prompt_capacity:
            raise ValueError(f"prompt length {n} is outside 1..{self.prompt_capacity}")
        if not self._idle:
            raise ValueError("every batch row is in use")
        row = min(self._idle)
        self.pool.release(self._idle.pop(row))
        assert self.pool.admit(seq) == row
        try:
            self.pool.set_length(seq, n)
        except Exception:
            self.pool.release(seq)
            self._park(row)
            raise
        tokens = np.zeros(self.prompt_capacity, np.uint32)
        tokens[:n] = prompt
        logits = np.zeros(self.vocab, np.float32)
        self.prefill_engine.step(self.prefill_engine.PREFILL, tokens,
                                 np.arange(self.prompt_capacity, dtype=np.uint32), n, 0, logits)
        self.cache.store(seq, self.prefill_state, 0, self.prefill_max_seq, n)
        self._tables = None
        return logits

    def release(self, seq) -> None:
        """The sequence leaves: its pages return to the pool, its row idles."""
        row = self.pool.rows[seq]
        self.pool.release(seq)
        self._park(row)

    def step(self, tokens: Dict[object, int]) -> Dict[object, np.ndarray]:
        """One decode step of every active sequence: `tokens` maps each to
        its next input token; returns each one's logits. Every sequence's
        length grows by one."""
        active = self.sequences()
        if set(tokens) != set(active):
            raise ValueError("a decode step takes one token for every active sequence")
        ids = np.zeros(self.batch, np.uint32)
        for seq, row in active.items():
            ids[row] = tokens[seq]
        positions = self.pool.seq_lens().copy()  # each row's token sits at its cached length
        self.sync()
        logits = np.zeros(self.batch * self.vocab, np.float32)
        self.decode_engine.step(self.decode_engine.DECODE, ids, positions, 1, 0, logits)
        for key in list(self.pool.rows):
            self.pool.set_length(key, self.pool.lengths[key] + (0 if key in self._idle.values() else 1))
        rows = logits.reshape(self.batch, self.vocab)
        return {seq: rows[row].copy() for seq, row in active.items()}
