"""Continuous batching through the engine on the GPU, against the oracle
engine run one sequence at a time.

The decode program is the ordinary compiled llama-dense CommandBuffer at
batch 4; its KV State is bound to a paged cache (sl_hip_bind_paged_state),
so every CausalAttention of the fused, graph-replayed decode step reads
each row at its own length through the block tables. New prompts are
prefilled one at a time on a batch-1 prefill engine and stored into their
pages (sl_hip_paged_store). The run: four prompts of different lengths,
decode steps, then a sequence leaves and a new one takes its row (its freed
pages recycled) while the others keep decoding.

Each sequence has its own oracle engine (batch 1, its prompt at its exact
length, contiguous cache). Steps are teacher-forced: every row is fed the
oracle's greedy id, each active row's logits are compared at 1e-4 normwise,
and the GPU's greedy id must equal the oracle's unless the oracle's top-2
gap is below 1e-4 * ||logits||_2.
"""
import numpy as np
import pytest

import models
from conftest import assert_normwise
from oracle.cpu_device import OracleDevice
from starlight_amd import device as hipdevice
from starlight_amd import engine, graph, synth
from starlight_amd.graph import LlamaConfig
from starlight_amd.ir import QuantFormat, ValueRole
from starlight_amd.paged import ContinuousBatcher, PagedKvCache, PagePool

pytestmark = pytest.mark.gpu


def kv_value(lowered):
    return next(i for i, v in enumerate(lowered.ir.values) if v.role == ValueRole.STATE)


class OracleSequence:
    """One sequence on the oracle engine (batch 1, contiguous cache)."""

    def __init__(self, cdev, cbufs, cfg, prompt, max_seq):
        self.prompt, self.n, self.vocab = prompt, len(prompt), cfg.vocab
        pre = graph.lower_llama(cfg, 1, self.n, max_seq)
        dec = graph.lower_llama(cfg, 1, 1, max_seq)
        self.eng = engine.Engine(cdev, engine.compile_program(pre, cbufs), engine.compile_program(dec, cbufs), 1,
                                 max_seq)

    def prefill(self):
        out = np.zeros(self.vocab, np.float32)
        self.eng.step(self.eng.PREFILL, self.prompt, np.arange(self.n, dtype=np.uint32), self.n, 0, out)
        return out

    def decode(self, token):
        out = np.zeros(self.vocab, np.float32)
        self.eng.step(self.eng.DECODE, [token], [self.n], 1, self.n, out)
        self.n += 1
        return out


def check(got, want, mismatches):
    assert_normwise(got, want)
    if int(np.argmax(got)) != int(np.argmax(want)):
        assert models.near_tie(want), "greedy id differs without a near-tie"
        mismatches.append(1)
    return int(np.argmax(want))


CONFIGS = {
    "small": LlamaConfig(layers=2, hidden=512, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=512,
                         theta=500_000.0, quant=QuantFormat.INT4),
    "8b-shape-2-layers": LlamaConfig(layers=2, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336,
                                     vocab=32000, theta=500_000.0, quant=QuantFormat.INT4),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_continuous_batching_through_the_engine(hip, name):
    cfg = CONFIGS[name]
    B, cap, max_seq, page = 4, 64, 128, 16
    seed = 40
    caps = graph.DeviceCapabilities.from_c(hipdevice.capabilities())
    gb = models.upload(hip, cfg, seed)
    pre = graph.compile_for(graph.lower_llama(cfg, 1, cap, max_seq), caps)
    pre_dec = graph.compile_for(graph.lower_llama(cfg, 1, 1, max_seq), caps)
    peng = engine.NativeEngine(hip, engine.compile_program(pre, gb), engine.compile_program(pre_dec, gb), 1, max_seq)
    # the decode program's own cache holds 16 positions: it is bound to the pages
    dec = graph.compile_for(graph.lower_llama(cfg, B, 1, 16), caps)
    deng = engine.NativeEngine(hip, engine.compile_program(dec, gb), engine.compile_program(dec, gb), B, 16)
    pool = PagePool(num_pages=48, page_size=page, pages_per_seq=max_seq // page, max_batch=B)
    np.random.default_rng(seed).shuffle(pool.free)
    cache = PagedKvCache(hip, cfg.layers, cfg.kv_heads, cfg.head_dim, pool)
    batcher = ContinuousBatcher(hip, peng, peng.state_buffer(kv_value(pre)), max_seq, cap, deng,
                                deng.state_buffer(kv_value(dec)), cache, cfg.vocab)

    cdev = OracleDevice()
    cbufs = models.upload(cdev, cfg, seed)
    lengths = {"a": 20, "b": 37, "c": 5, "d": 50, "e": 29}
    prompts = {s: synth.prompt(cfg.vocab, n, seed + i) for i, (s, n) in enumerate(lengths.items())}
    oracles, nxt, mismatches = {}, {}, []

    def join(s):
        oracles[s] = OracleSequence(cdev, cbufs, cfg, prompts[s], max_seq)
        nxt[s] = check(batcher.admit(s, prompts[s]), oracles[s].prefill(), mismatches)

    before = hip.stats()
    for s in "abcd":
        join(s)
    for step in range(10):
        if step == 4:
            batcher.release("c")  # leaves; its row and pages go to "e"
            del nxt["c"]
            join("e")
        got = batcher.step(dict(nxt))
        for s, logits in got.items():
            nxt[s] = check(logits, oracles[s].decode(nxt[s]), mismatches)
    after = hip.stats()
    assert set(batcher.sequences()) == {"a", "b", "d", "e"}
    assert pool.lengths["a"] == 30 and pool.lengths["e"] == 35
    assert after["graph_replays"] > before["graph_replays"]  # decode steps replayed with per-row lengths
    assert len(mismatches) <= 1
    # three more steps in the engine's native loop (sl_engine_decode_rows):
    # greedy, each row from its own length, against the oracle's greedy ids
    rows = batcher.sequences()
    for s in rows:
        pool.reserve(s, pool.lengths[s] + 4)
    batcher.sync()
    first = np.zeros(B, np.uint32)
    starts = pool.seq_lens()
    for s, r in rows.items():
        first[r] = nxt[s]
    ids = deng.decode_rows(first, starts, cache.lens_buffer, 3)
    for s, r in rows.items():
        tok = nxt[s]
        for step in range(3):
            want = oracles[s].decode(tok)
            tok = int(np.argmax(want))
            if int(ids[step, r]) != tok:
                assert models.near_tie(want), f"sequence {s} step {step}: greedy id differs without a near-tie"
                break
    hip.bind_paged_state(deng.state_buffer(kv_value(dec)), None)
    peng.close()
    deng.close()


def test_paged_state_binding_errors(hip):
    """Commands on a bound State: more than one token per row and KvAppend
    are Unimplemented; a bad block table is an Execution error at dispatch
    (nothing logged); without the binding the same commands run on the
    contiguous State."""
    from starlight_amd.device import DeviceError
    from starlight_amd.ir import BufferRef, Op, Value
    H, Hkv, D, max_seq = 4, 2, 64, 16
    pool = PagePool(num_pages=4, page_size=16, pages_per_seq=2, max_batch=1)
    cache = PagedKvCache(hip, 1, Hkv, D, pool)
    pool.admit(0)
    pool.set_length(0, 3)
    cache.sync()
    state = hip.allocate_f32(1 * 1 * 2 * max_seq * Hkv * D, 256)
    sv = Value.f32([1, 1, 2, max_seq, Hkv, D], ValueRole.STATE)
    sref = BufferRef(state, 0, 2 * max_seq * Hkv * D)
    op = Op.causal_attention(0, H, Hkv, D, 0.125)

    def attention(seq):
        q, k = hip.allocate_f32(H * seq * D, 256), hip.allocate_f32(Hkv * seq * D, 256)
        v, out = hip.allocate_f32(Hkv * seq * D, 256), hip.allocate_f32(H * seq * D, 256)
        hip.dispatch(op, [BufferRef(q, 0, H * seq * D), BufferRef(k, 0, Hkv * seq * D),
                          BufferRef(v, 0, Hkv * seq * D), sref],
                     [Value.f32([1, H, seq, D]), Value.f32([1, Hkv, seq, D]), Value.f32([1, Hkv, seq, D]), sv],
                     [BufferRef(out, 0, H * seq * D)], [Value.f32([1, H, seq, D])], [0])

    cache.bind_state(state)
    with pytest.raises(DeviceError) as e:
        attention(2)
    assert e.value == DeviceError.unimplemented("a paged State takes one new token per row")
    k, v = hip.allocate_f32(Hkv * D, 256), hip.allocate_f32(Hkv * D, 256)
    with pytest.raises(DeviceError) as e:
        hip.dispatch(Op.kv_append(0), [BufferRef(k, 0, Hkv * D), BufferRef(v, 0, Hkv * D), sref],
                     [Value.f32([1, Hkv, 1, D]), Value.f32([1, Hkv, 1, D]), sv], [], [], [0])
    assert e.value == DeviceError.unimplemented("only CausalAttention reads a paged State on HipDevice")
    attention(1)
    hip.synchronize()
    hip.upload_u32(cache.table_buffer, np.array([7, 0], np.uint32))  # page 7 of a 4-page pool
    with pytest.raises(DeviceError) as e:
        attention(1)
    assert e.value == DeviceError.execution("page id out of range")
    hip.bind_paged_state(state, None)
    attention(2)
    hip.synchronize()
