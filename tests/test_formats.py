"""Quantized checkpoints on disk (starlight_amd.formats): Safetensors with
the group-wise payload and scales as tensors and `starlight.quantization`
metadata. sl-precision, which defines such files for StarLight, is absent
from the reference tree, so the layout is this backend's own (parity
unpinned); these tests pin it against the payload convention of quant.py and
its independent nibble decoding, and run a model from a saved checkpoint."""
import json

import numpy as np
import pytest

from oracle.cpu_device import OracleDevice
from starlight_amd import engine, formats, graph, quant, synth
from starlight_amd.graph import LlamaConfig
from starlight_amd.ir import QuantFormat


def rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("fmt,group,n,k", [(QuantFormat.INT4, 128, 48, 256), (QuantFormat.INT4, 64, 7, 192),
                                           (QuantFormat.INT8, 128, 33, 384), (QuantFormat.INT4, 2, 3, 6)])
def test_round_trip_keeps_payload_scales_and_dense_tensors(tmp_path, fmt, group, n, k):
    r = rng(n + k)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    norm = r.standard_normal(k).astype(np.float32)
    q = formats.quantize_tensor(w, fmt, group)
    path = str(tmp_path / "ckpt.safetensors")
    formats.save(path, {"norm": norm}, {"proj": q})
    dense, quantized = formats.load(path)
    assert set(dense) == {"norm"} and set(quantized) == {"proj"}
    np.testing.assert_array_equal(dense["norm"], norm)
    got = quantized["proj"]
    assert (got.fmt, got.group, got.n, got.k) == (fmt, group, n, k)
    words, scales = quant.quantize(w, group, fmt)
    np.testing.assert_array_equal(got.words(), words)  # the device payload, bit for bit
    np.testing.assert_array_equal(got.scales, scales)
    np.testing.assert_array_equal(got.dequantize(), quant.dequantize(words, scales, n, k, group, fmt))

    from safetensors import safe_open
    with safe_open(path, framework="numpy") as f:
        meta = json.loads(f.metadata()["starlight.quantization"])
        assert meta == {"version": 1, "tensors": {"proj": {"format": "int4" if fmt == QuantFormat.INT4 else "int8",
                                                           "group_size": group, "shape": [n, k],
                                                           "scale": "proj.__scales"}}}
        assert f.get_tensor("proj").dtype == (np.uint8 if fmt == QuantFormat.INT4 else np.int8)


def test_int4_payload_bytes_hold_two_complement_nibbles_even_k_low():
    r = rng(5)
    w = (r.standard_normal((5, 10)) * 0.1).astype(np.float32)
    q = formats.quantize_tensor(w, QuantFormat.INT4, 2)
    codes, _ = quant.quantize_codes(w, 2, QuantFormat.INT4)
    b = q.payload.astype(np.int32)
    lo = np.where((b & 0xF) >= 8, (b & 0xF) - 16, b & 0xF)
    hi = np.where((b >> 4) >= 8, (b >> 4) - 16, b >> 4)
    decoded = np.empty((5, 10), np.int32)
    decoded[:, 0::2], decoded[:, 1::2] = lo, hi
    np.testing.assert_array_equal(decoded, codes)
    assert q.payload.shape == (5, 5)


def write_raw(path, tensors, meta):
    from safetensors.numpy import save_file
    save_file(tensors, path, metadata=None if meta is None else {"starlight.quantization": json.dumps(meta)})


@pytest.mark.parametrize("case,message", [
    ("no_scale", "missing"), ("payload_dtype", "payload"), ("scale_shape", "scales"), ("format", "unknown format"),
    ("version", "version"), ("stray_u8", "without a"), ("group", "multiple of group_size")])
def test_malformed_checkpoints_are_rejected(tmp_path, case, message):
    n, k, g = 4, 8, 4
    payload = np.zeros((n, k // 2), np.uint8)
    scales = np.ones((n, k // g), np.float32)
    entry = {"format": "int4", "group_size": g, "shape": [n, k], "scale": "w.__scales"}
    tensors = {"w": payload, "w.__scales": scales}
    meta = {"version": 1, "tensors": {"w": entry}}
    if case == "no_scale":
        del tensors["w.__scales"]
    elif case == "payload_dtype":
        tensors["w"] = payload.view(np.int8)
    elif case == "scale_shape":
        tensors["w.__scales"] = np.ones((n, 1), np.float32)
    elif case == "format":
        entry["format"] = "int3"
    elif case == "version":
        meta["version"] = 2
    elif case == "stray_u8":
        tensors["extra"] = np.zeros(3, np.uint8)
    elif case == "group":
        entry["group_size"] = 3
    path = str(tmp_path / "bad.safetensors")
    write_raw(path, tensors, meta)
    with pytest.raises(ValueError, match=message):
        formats.load(path)


CFG = LlamaConfig(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=512, theta=500_000.0,
                  quant=QuantFormat.INT4)


def test_model_from_a_saved_checkpoint_generates_what_its_weights_do(tmp_path):
    """The same model uploaded from f32 weights (quantized on upload) and from
    a saved quantized checkpoint: identical greedy ids and logits on the
    oracle device."""
    weights = synth.llama_weights(CFG, 4)
    prompt = synth.prompt(CFG.vocab, 5, 4)
    path = str(tmp_path / "model.safetensors")
    formats.save(path, *formats.quantize_model(CFG, weights))

    def run(upload):
        dev = OracleDevice()
        bufs = upload(dev)
        eng = engine.Engine(dev, engine.compile_program(graph.lower_llama(CFG, 1, 5, 16), bufs),
                            engine.compile_program(graph.lower_llama(CFG, 1, 1, 16), bufs), 1, 16)
        return eng.generate(prompt, 3, CFG.vocab)

    t_ref, l_ref = run(lambda dev: engine.upload_weights(dev, CFG, weights))
    t_ck, l_ck = run(lambda dev: formats.upload(dev, CFG, *formats.load(path)))
    np.testing.assert_array_equal(np.asarray(t_ck), np.asarray(t_ref))
    np.testing.assert_array_equal(np.asarray(l_ck), np.asarray(l_ref))


def test_upload_rejects_a_checkpoint_for_another_model(tmp_path):
    weights = synth.llama_weights(CFG, 4)
    dense, quantized = formats.quantize_model(CFG, weights)
    other = LlamaConfig(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=512,
                        theta=500_000.0, quant=QuantFormat.INT8)
    with pytest.raises(ValueError, match="does not match"):
        formats.upload(OracleDevice(), other, dense, quantized)
    del quantized["layers.0.mlp.down"]
    with pytest.raises(ValueError, match="missing"):
        formats.upload(OracleDevice(), CFG, dense, quantized)
