"""End to end on the GPU: compiled llama-dense CommandBuffers driven through
the native engine and the HIP device, against the same programs on the CPU
oracle device.

Per-step logits must agree within 1e-4 normwise; greedy ids must be identical
except after a step where the oracle's top-2 logit gap is below
1e-4 * ||logits||_2 (a near-tie either side may resolve differently).
"""
import numpy as np
import pytest

from conftest import assert_normwise, rel_l2
from oracle.cpu_device import OracleDevice
from starlight_amd import engine, graph, synth
from starlight_amd.graph import LlamaConfig
from starlight_amd.ir import QuantFormat

from models import Pair
from test_engine_cpu import FIXTURE_EXPECTED

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ids", [(1, 2), (7,)])
def test_fixture_end_to_end_on_gpu(hip, ids):
    """distros/starlight-runtime/tests/end_to_end.rs:113-152, 184-217."""
    w = graph.fixture_weights()
    bufs = {name: hip.upload_new_f32(a) for name, a in w.items()}
    pre = engine.compile_program(graph.lower_fixture(len(ids)), bufs)
    dec = engine.compile_program(graph.lower_fixture(1), bufs)
    eng = engine.NativeEngine(hip, pre, dec, 1, 16)
    out = np.zeros(8, np.float32)
    eng.step(eng.PREFILL, ids, [], len(ids), 0, out)
    assert np.max(np.abs(out.astype(np.float64) - FIXTURE_EXPECTED[ids])) <= 1e-5


def run_both(hip, cfg: LlamaConfig, prompt_len: int, steps: int, max_seq: int, seed: int = 0):
    weights = synth.llama_weights(cfg, seed)
    prompt = synth.prompt(cfg.vocab, prompt_len, seed)

    gbufs = engine.upload_weights(hip, cfg, weights)
    gpu = engine.NativeEngine(hip, engine.compile_program(graph.lower_llama(cfg, 1, prompt_len, max_seq), gbufs),
                              engine.compile_program(graph.lower_llama(cfg, 1, 1, max_seq), gbufs), 1, max_seq)
    g_tokens, g_logits = gpu.generate(prompt, steps, cfg.vocab)

    cpu_dev = OracleDevice()
    cbufs = engine.upload_weights(cpu_dev, cfg, weights)
    cpu = engine.Engine(cpu_dev, engine.compile_program(graph.lower_llama(cfg, 1, prompt_len, max_seq), cbufs),
                        engine.compile_program(graph.lower_llama(cfg, 1, 1, max_seq), cbufs), 1, max_seq)
    c_tokens, c_logits = cpu.generate(prompt, steps, cfg.vocab)
    return g_tokens, g_logits, c_tokens, c_logits


def check_generation(g_tokens, g_logits, c_tokens, c_logits):
    for i in range(len(c_tokens)):
        assert_normwise(g_logits[i], c_logits[i])
        if g_tokens[i] != c_tokens[i]:
            top2 = np.sort(c_logits[i].astype(np.float64))[-2:]
            gap = top2[1] - top2[0]
            assert gap < 1e-4 * np.linalg.norm(c_logits[i]), f"greedy id differs at step {i} with gap {gap}"
            return i  # the sequences legitimately diverge after a near-tie
    return len(c_tokens)


def test_tiny_llama_prefill_32_then_32_greedy_steps(hip):
    """The tiny llama-dense configuration: 2 layers, hidden 256, 4x64 MHA,
    SwiGLU 688, vocab 1024, f32 weights N(0, 0.02) from seed 0."""
    g_tokens, g_logits, c_tokens, c_logits = run_both(hip, graph.TINY, 32, 32, 64)
    compared = check_generation(g_tokens, g_logits, c_tokens, c_logits)
    assert compared >= 8


def test_tiny_llama_teacher_forced_32_steps(hip):
    """The tiny configuration again, with both engines fed the oracle's
    greedy ids: all 32 decode steps' logits are compared."""
    pair = Pair(hip, graph.TINY, batch=1, prompt_len=32, max_seq=64, seed=0)
    try:
        assert len(pair.decode(pair.prefill(), 32)) == 32
    finally:
        pair.close()


@pytest.mark.parametrize("fmt", [QuantFormat.INT4, QuantFormat.INT8])
def test_1b_shaped_quantized_layers(hip, fmt):
    """The 1B-class shapes (hidden 2048, 32/8 heads x 64, SwiGLU 8192,
    vocab 32000, theta 500000) with group-quantized weights, two layers so the
    oracle finishes quickly: 8-token prefill, 8 teacher-forced decode steps,
    every step compared."""
    cfg = LlamaConfig(layers=2, hidden=2048, heads=32, kv_heads=8, head_dim=64, ffn=8192, vocab=32000,
                      theta=500_000.0, quant=fmt)
    pair = Pair(hip, cfg, batch=1, prompt_len=8, max_seq=32, seed=0)
    try:
        assert len(pair.decode(pair.prefill(), 8)) == 8
    finally:
        pair.close()


def test_kv_cache_matches_the_oracle_after_decode(hip):
    """After prefill + decode, the device KV cache equals the oracle's bit for
    bit up to the accumulated rounding of the projections (1e-4 normwise per
    layer slice), and positions beyond past_len stay zero."""
    cfg = graph.TINY
    weights = synth.llama_weights(cfg, 3)
    prompt = synth.prompt(cfg.vocab, 5, 3)
    max_seq = 16
    bufs = engine.upload_weights(hip, cfg, weights)
    pre_l, dec_l = graph.lower_llama(cfg, 1, 5, max_seq), graph.lower_llama(cfg, 1, 1, max_seq)
    gpu = engine.NativeEngine(hip, engine.compile_program(pre_l, bufs), engine.compile_program(dec_l, bufs), 1,
                              max_seq)
    gpu.generate(prompt, 2, cfg.vocab)
    kv_buf = gpu.state_buffer(pre_l.kv_cache)
    n = 1 * cfg.layers * 2 * max_seq * cfg.kv_heads * cfg.head_dim
    got = hip.read_f32(kv_buf, n).reshape(cfg.layers, 2, max_seq, -1)

    cdev = OracleDevice()
    cb = engine.upload_weights(cdev, cfg, weights)
    cpu = engine.Engine(cdev, engine.compile_program(pre_l, cb), engine.compile_program(dec_l, cb), 1, max_seq)
    cpu.generate(prompt, 2, cfg.vocab)
    want = cdev.f32[cpu.states[pre_l.kv_cache]].reshape(cfg.layers, 2, max_seq, -1)
    for l in range(cfg.layers):
        for kv in range(2):
            assert_normwise(got[l, kv, :7], want[l, kv, :7])
    assert np.all(got[:, :, 7:] == 0)


@pytest.mark.parametrize("fusion,graphs", [(False, False), (True, False), (False, True)])
def test_submission_options_keep_parity(hip, fusion, graphs):
    """Every combination of the submission options (fused launches, graph
    replay) gives the oracle's logits on the 1B-class INT4 shapes."""
    cfg = LlamaConfig(layers=2, hidden=2048, heads=32, kv_heads=8, head_dim=64, ffn=8192, vocab=32000,
                      theta=500_000.0, quant=QuantFormat.INT4)
    hip.set_options(fusion=fusion, graphs=graphs)
    try:
        pair = Pair(hip, cfg, batch=1, prompt_len=8, max_seq=32, seed=1)
        assert len(pair.decode(pair.prefill(), 4)) == 4
        pair.close()
    finally:
        hip.set_options()


def test_8b_shaped_decode_fuses_and_replays(hip):
    """The 8B decode shapes (hidden 4096, 32/8 heads x 128, SwiGLU 14336, INT4
    g128), two layers and a 32000 vocabulary so the oracle keeps up: 6-token
    prefill, 6 greedy steps. The decode submissions must run fused and, from
    the third step, as graph replays, with the oracle's logits every step."""
    cfg = LlamaConfig(layers=2, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=32000,
                      theta=500_000.0, quant=QuantFormat.INT4)
    before = hip.stats()
    g_tokens, g_logits, c_tokens, c_logits = run_both(hip, cfg, 6, 6, 64, seed=2)
    after = hip.stats()
    assert check_generation(g_tokens, g_logits, c_tokens, c_logits) >= 3
    assert after["fused_commands"] > before["fused_commands"]
    assert after["graph_captures"] > before["graph_captures"]
    assert after["graph_replays"] >= before["graph_replays"] + 3


def test_model_from_a_saved_checkpoint_on_gpu(hip, tmp_path):
    """A quantized Safetensors checkpoint (starlight_amd.formats) loaded and
    uploaded: the same ids and logits as the f32 weights quantized on upload,
    and the oracle device running the same loaded checkpoint agrees with the
    GPU (every step's logits within 1e-4 normwise, greedy ids equal except at
    a near-tie)."""
    from starlight_amd import formats
    cfg = LlamaConfig(layers=2, hidden=512, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=3000,
                      theta=500_000.0, quant=QuantFormat.INT4)
    weights = synth.llama_weights(cfg, 6)
    prompt = synth.prompt(cfg.vocab, 6, 6)
    path = str(tmp_path / "model.safetensors")
    formats.save(path, *formats.quantize_model(cfg, weights))

    def run(bufs):
        eng = engine.NativeEngine(hip, engine.compile_program(graph.lower_llama(cfg, 1, 6, 32), bufs),
                                  engine.compile_program(graph.lower_llama(cfg, 1, 1, 32), bufs), 1, 32)
        return eng.generate(prompt, 4, cfg.vocab)

    t_ref, l_ref = run(engine.upload_weights(hip, cfg, weights))
    t_ck, l_ck = run(formats.upload(hip, cfg, *formats.load(path)))
    np.testing.assert_array_equal(np.asarray(t_ck), np.asarray(t_ref))
    np.testing.assert_array_equal(np.asarray(l_ck), np.asarray(l_ref))
    # the oracle on the same loaded checkpoint
    cdev = OracleDevice()
    cb = formats.upload(cdev, cfg, *formats.load(path))
    cpu = engine.Engine(cdev, engine.compile_program(graph.lower_llama(cfg, 1, 6, 32), cb),
                        engine.compile_program(graph.lower_llama(cfg, 1, 1, 32), cb), 1, 32)
    c_tokens, c_logits = cpu.generate(prompt, 4, cfg.vocab)
    assert check_generation(t_ck, l_ck, c_tokens, c_logits) >= 3


def test_batched_decode_matches_a_step_loop(hip):
    """sl_engine_decode_batch: two sequences decoded together give the ids of
    a loop of engine steps with each row's first maximum taken by numpy."""
    cfg, B, prompt_len, steps, max_seq = graph.TINY, 2, 6, 5, 32
    weights = synth.llama_weights(cfg, 8)
    bufs = engine.upload_weights(hip, cfg, weights)
    prompts = np.concatenate([synth.prompt(cfg.vocab, prompt_len, 8 + b) for b in range(B)])
    positions = np.tile(np.arange(prompt_len, dtype=np.uint32), B)

    def fresh():
        eng = engine.NativeEngine(hip, engine.compile_program(graph.lower_llama(cfg, B, prompt_len, max_seq), bufs),
                                  engine.compile_program(graph.lower_llama(cfg, B, 1, max_seq), bufs), B, max_seq)
        logits = np.zeros(B * cfg.vocab, np.float32)
        eng.step(eng.PREFILL, prompts, positions, prompt_len, 0, logits)
        return eng, logits.reshape(B, cfg.vocab).argmax(axis=1).astype(np.uint32)

    eng, first = fresh()
    got = eng.decode_batch(first, prompt_len, steps)
    eng, cur = fresh()
    want = []
    logits = np.zeros(B * cfg.vocab, np.float32)
    for s in range(steps):
        past = prompt_len + s
        eng.step(eng.DECODE, cur, np.full(B, past, np.uint32), 1, past, logits)
        cur = logits.reshape(B, cfg.vocab).argmax(axis=1).astype(np.uint32)
        want.append(cur.copy())
    np.testing.assert_array_equal(got, np.stack(want))


def test_native_build_binds_scale_params_and_rejects_a_missing_one(hip):
    """sl_engine_build binds every quantized Param to its `<role>.__scales`
    Param from the program (ARCH-0006:147) and fails with Execution when
    one has no bound buffer."""
    from starlight_amd.device import DeviceError
    cfg = LlamaConfig(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=384,
                      theta=500_000.0, quant=QuantFormat.INT4)
    bufs = engine.upload_weights(hip, cfg, synth.llama_weights(cfg, 5))
    low = graph.lower_llama(cfg, 1, 1, 16)
    missing = {k: v for k, v in bufs.items() if k != "layers.0.attn.o.__scales"}
    with pytest.raises(DeviceError) as e:
        engine.NativeEngine(hip, engine.compile_program(low, missing), engine.compile_program(low, missing), 1, 16)
    assert e.value == DeviceError.execution("quantized Param has no bound scale Param")
    eng = engine.NativeEngine(hip, engine.compile_program(low, bufs), engine.compile_program(low, bufs), 1, 16)
    out = np.zeros(cfg.vocab, np.float32)
    eng.step(eng.DECODE, [3], [0], 1, 0, out)
    cdev = OracleDevice()
    cb = engine.upload_weights(cdev, cfg, synth.llama_weights(cfg, 5))
    cpu = engine.Engine(cdev, engine.compile_program(low, cb), engine.compile_program(low, cb), 1, 16)
    want = np.zeros(cfg.vocab, np.float32)
    cpu.step(cpu.DECODE, [3], [0], 1, 0, want)
    assert_normwise(out, want)


def test_native_step_errors_carry_their_own_message(hip):
    """Every failing engine call records its reason (the reference's step
    returns a typed StepError, ARCH-0007 §3.2): a step past the compiled
    capacity, an unknown mode and a wrong token count each raise Execution
    with their message, not the device's previous error, and a valid step
    still runs afterwards."""
    from starlight_amd.device import DeviceError
    from starlight_amd.ir import BufferRef, Op, Value
    cfg = LlamaConfig(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=384,
                      theta=500_000.0)
    bufs = engine.upload_weights(hip, cfg, synth.llama_weights(cfg, 6))
    eng = engine.NativeEngine(hip, engine.compile_program(graph.lower_llama(cfg, 1, 4, 16), bufs),
                              engine.compile_program(graph.lower_llama(cfg, 1, 1, 16), bufs), 1, 16)
    out = np.zeros(cfg.vocab, np.float32)
    # leave an unrelated error behind on the device first
    x = hip.upload_new_f32(np.zeros(8, np.float32))
    with pytest.raises(DeviceError):
        hip.dispatch(Op.add(), [BufferRef(x, 0, 8), BufferRef(x, 0, 4)], [Value.f32([8]), Value.f32([4])],
                     [BufferRef(x, 0, 8)], [Value.f32([8])])
    with pytest.raises(DeviceError) as e:
        eng.step(eng.DECODE, [3], [15], 1, 16, out)
    assert e.value == DeviceError.execution("step input exceeds the compiled capacity")
    with pytest.raises(DeviceError) as e:
        eng.step(7, [3], [0], 1, 0, out)
    assert e.value == DeviceError.execution("step mode is neither Prefill nor Decode")
    with pytest.raises(DeviceError) as e:
        eng.step(eng.DECODE, [3, 4], [0, 1], 1, 0, out)
    assert e.value == DeviceError.execution("step input exceeds the compiled capacity")
    eng.step(eng.PREFILL, [1, 2, 3, 4], [0, 1, 2, 3], 4, 0, out)
    assert np.isfinite(out).all()
    eng.close()
