"""Synthetic model weights and prompts (no checkpoints are available).

One numpy PCG64 generator seeded with `seed` draws every tensor in the
canonical weight order of graph.weight_specs: linear and embedding weights
~N(0, 0.02) in float32, RMSNorm weights 1.0. Prompts are uniform ids below
the vocabulary from a second generator seeded with seed + 1.
"""
from __future__ import annotations

from typing import Dict

import numpy as np

from .graph import LlamaConfig, weight_specs


def llama_weights(cfg: LlamaConfig, seed: int = 0, std: float = 0.02) -> Dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    out = {}
    for spec in weight_specs(cfg):
        if spec.kind == "norm":
            out[spec.name] = np.ones(spec.shape, np.float32)
        else:
            out[spec.name] = (rng.standard_normal(spec.shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
    return out


def prompt(vocab: int, length: int, seed: int = 0) -> np.ndarray:
    return np.random.default_rng(seed + 1).integers(0, vocab, length).astype(np.uint32)
