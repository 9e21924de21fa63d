"""The restated engine step loop on the CPU oracle device: the runtime
fixture's end-to-end expectations (distros/starlight-runtime/tests/
end_to_end.rs:38-68, 102-111, 113-152, 184-217) and a tiny llama run."""
import numpy as np
import pytest

from oracle.cpu_device import OracleDevice
from starlight_amd import engine, graph, synth

# f64 closed forms of end_to_end.rs's expected_logits for the fixture weights.
FIXTURE_EXPECTED = {
    (1, 2): [-0.106132506, -0.098551613, -0.242588586, 0.181941439, 0.265331265, -0.106132506, -0.098551613,
             -0.242588586],
    (7,): [-0.158349585, -0.062208766, -0.19228164, 0.196051868, 0.216788123, -0.158349585, -0.062208766,
           -0.19228164],
}


def expected_fixture_logits(ids):
    """end_to_end.rs:38-68 in float64."""
    emb = (np.arange(32, dtype=np.float64) - 3.0) * 0.1
    norm = np.array([1.0, 0.5, 1.5, 0.75])
    lm = ((np.arange(32) % 5).astype(np.float64) - 2.0) * 0.1
    row = emb.reshape(8, 4)[ids[-1]]
    rms = row / np.sqrt((row * row).sum() / 4 + 1e-5) * norm
    return lm.reshape(8, 4) @ rms


def fixture_engine(device, seq):
    w = graph.fixture_weights()
    bufs = {name: device.upload_new_f32(a) for name, a in w.items()}
    pre = engine.compile_program(graph.lower_fixture(seq), bufs)
    dec = engine.compile_program(graph.lower_fixture(1), bufs)
    return engine.Engine(device, pre, dec, 1, 16)


@pytest.mark.parametrize("ids", [(1, 2), (7,)])
def test_fixture_matches_closed_form(ids):
    assert np.allclose(expected_fixture_logits(ids), FIXTURE_EXPECTED[ids], atol=1e-8)
    eng = fixture_engine(OracleDevice(), len(ids))
    out = np.zeros(8, np.float32)
    eng.step(engine.Engine.PREFILL, ids, [], len(ids), 0, out)
    assert np.max(np.abs(out.astype(np.float64) - FIXTURE_EXPECTED[ids])) <= 1e-5


def test_tiny_llama_runs_on_the_oracle_device():
    cfg = graph.TINY
    dev = OracleDevice()
    bufs = engine.upload_weights(dev, cfg, synth.llama_weights(cfg, 0))
    pre = engine.compile_program(graph.lower_llama(cfg, 1, 8, 16), bufs)
    dec = engine.compile_program(graph.lower_llama(cfg, 1, 1, 16), bufs)
    eng = engine.Engine(dev, pre, dec, 1, 16)
    tokens, logits = eng.generate(synth.prompt(cfg.vocab, 8, 0), 2, cfg.vocab)
    assert tokens.shape == (3,) and np.isfinite(logits).all()
    assert np.all(tokens < cfg.vocab)
