"""Shared synthetic models for the engine parity tests, built once per
session: f32 weights from starlight_amd.synth, their group-quantized form,
and a GPU-vs-oracle step runner that feeds both engines the same tokens.

Quantization here goes through the oracle's C routine (threaded); it gives
quant.quantize's payload and scales bit for bit
(tests/test_quant.py::test_numpy_and_c_oracle_agree_bit_exactly), only
faster at the 8B shapes.
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

import oracle
from conftest import assert_normwise
from oracle.cpu_device import OracleDevice
from starlight_amd import device as hipdevice
from starlight_amd import engine, formats, graph, synth
from starlight_amd.graph import LlamaConfig, weight_specs
from starlight_amd.ir import QuantFormat, ValueRole

_F32: Dict[Tuple, Dict[str, np.ndarray]] = {}
_QUANT: Dict[Tuple, Tuple[Dict[str, np.ndarray], Dict[str, formats.QuantTensor]]] = {}


def _shape_key(cfg: LlamaConfig, seed: int):
    return (cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab, seed)


def f32_weights(cfg: LlamaConfig, seed: int) -> Dict[str, np.ndarray]:
    key = _shape_key(cfg, seed)
    if key not in _F32:
        _F32.clear()  # keep one model's f32 weights alive at a time
        _F32[key] = synth.llama_weights(cfg, seed)
    return _F32[key]


def quantized_model(cfg: LlamaConfig, seed: int):
    """(dense f32 tensors, quantized tensors) of cfg's synthetic weights."""
    key = _shape_key(cfg, seed) + (cfg.quant, cfg.group, cfg.quant_lm_head)
    if key not in _QUANT:
        w = f32_weights(cfg, seed)
        dense, quantized = {}, {}
        bits = 4 if cfg.quant == QuantFormat.INT4 else 8
        for spec in weight_specs(cfg):
            a = w[spec.name]
            if spec.quantized:
                n, k = spec.shape
                payload, scales = oracle.quantize_groupwise(a, n, k, cfg.group, bits)
                if bits == 8:
                    payload = payload.view(np.int8)
                quantized[spec.name] = formats.QuantTensor(QuantFormat(cfg.quant), cfg.group, n, k, payload, scales)
            else:
                dense[spec.name] = a
        if len(_QUANT) >= 2:
            _QUANT.pop(next(iter(_QUANT)))
        _QUANT[key] = (dense, quantized)
    return _QUANT[key]


def upload(device, cfg: LlamaConfig, seed: int) -> Dict[str, int]:
    if cfg.quant is None:
        return engine.upload_weights(device, cfg, f32_weights(cfg, seed))
    return formats.upload(device, cfg, *quantized_model(cfg, seed))


def near_tie(logits: np.ndarray) -> bool:
    """The oracle's top-2 logit gap is below 1e-4 * ||logits||_2: either id
    is an acceptable greedy choice."""
    top2 = np.sort(logits.astype(np.float64))[-2:]
    return (top2[1] - top2[0]) < 1e-4 * np.linalg.norm(logits.astype(np.float64))


class Pair:
    """The same compiled programs on the HIP engine and on the oracle engine."""

    def __init__(self, hip, cfg: LlamaConfig, batch: int, prompt_len: int, max_seq: int, seed: int):
        self.cfg, self.batch, self.prompt_len, self.max_seq = cfg, batch, prompt_len, max_seq
        self.hip = hip
        self.past0 = 0  # positions already in the cache when the prompt starts
        caps = graph.DeviceCapabilities.from_c(hipdevice.capabilities())
        pre_l = graph.compile_for(graph.lower_llama(cfg, batch, prompt_len, max_seq), caps)
        self.kv_value = next(i for i, v in enumerate(pre_l.ir.values) if v.role == ValueRole.STATE)
        self.kv_shape = pre_l.ir.values[self.kv_value].shape
        dec_l = graph.compile_for(graph.lower_llama(cfg, batch, 1, max_seq), caps)
        gb = upload(hip, cfg, seed)
        self.gpu = engine.NativeEngine(hip, engine.compile_program(pre_l, gb), engine.compile_program(dec_l, gb),
                                       batch, max_seq)
        self.cdev = OracleDevice()
        cb = upload(self.cdev, cfg, seed)
        self.cpu = engine.Engine(self.cdev, engine.compile_program(pre_l, cb), engine.compile_program(dec_l, cb),
                                 batch, max_seq)
        self.prompts = np.concatenate([synth.prompt(cfg.vocab, prompt_len, seed + b) for b in range(batch)])
        self.mismatched_ids = 0

    def _compare(self, g: np.ndarray, c: np.ndarray) -> np.ndarray:
        g = g.reshape(self.batch, -1)
        c = c.reshape(self.batch, -1)
        for b in range(self.batch):
            assert_normwise(g[b], c[b])
            if int(np.argmax(g[b])) != int(np.argmax(c[b])):
                assert near_tie(c[b]), f"row {b}: greedy id differs without a near-tie"
                self.mismatched_ids += 1
        return c.argmax(axis=1).astype(np.uint32)

    def seed_cache(self, past: int, seed: int) -> None:
        """Writes the same keys and values ~N(0, 1) at positions [0, past)
        of every layer into both engines' KV caches (uploaded through the
        Device contract), so the prompt starts at past_len = past and
        attends over past + prompt_len positions."""
        cache = np.zeros(self.kv_shape, np.float32)  # [B, layers, 2, max_seq, Hkv, D]
        prefix = cache[:, :, :, :past]
        prefix[...] = np.random.default_rng(seed).standard_normal(prefix.shape, dtype=np.float32)
        self.hip.upload_f32(self.gpu.state_buffer(self.kv_value), cache.ravel())
        self.cdev.upload_f32(self.cpu.states[self.kv_value], cache.ravel())
        self.past0 = past

    def prefill(self, repeats: int = 1) -> np.ndarray:
        B, S, V, P = self.batch, self.prompt_len, self.cfg.vocab, self.past0
        pos = np.tile(np.arange(P, P + S, dtype=np.uint32), B)
        c = np.zeros(B * V, np.float32)
        self.cpu.step(self.cpu.PREFILL, self.prompts, pos, S, P, c)
        ids = None
        for _ in range(repeats):
            g = np.zeros(B * V, np.float32)
            self.gpu.step(self.gpu.PREFILL, self.prompts, pos, S, P, g)
            ids = self._compare(g, c)
        return ids

    def decode(self, ids: np.ndarray, steps: int) -> List[np.ndarray]:
        """Teacher-forced decode: both engines take the oracle's greedy ids,
        so every step's logits are compared on identical inputs."""
        B, V = self.batch, self.cfg.vocab
        out = []
        for s in range(steps):
            past = self.past0 + self.prompt_len + s
            pos = np.full(B, past, np.uint32)
            g = np.zeros(B * V, np.float32)
            c = np.zeros(B * V, np.float32)
            self.gpu.step(self.gpu.DECODE, ids, pos, 1, past, g)
            self.cpu.step(self.cpu.DECODE, ids, pos, 1, past, c)
            ids = self._compare(g, c)
            out.append(ids)
        return out

    def close(self):
        self.gpu.close()
