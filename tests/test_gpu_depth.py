"""The benchmark models at depth, against the oracle engine.

The other engine tests run two layers. These run the 1B-class model at all
16 layers and the 8B shape at eight layers with its full 128,256-token
vocabulary, so that KV-cache layers past the first two, the deeper
scratchpad plans and the fused decode units of later layers (the last
layer's rotated-q staging among them) meet the oracle. The 8B prompt starts
at past_len 1024 after a seeded KV prefix, so its prefill attends over
1,064 positions and every decode step over more than 1,024 keys.

Engine steps are teacher-forced: both engines take the oracle's greedy ids,
every step's logits are compared at 1e-4 normwise, and the GPU's greedy id
must equal the oracle's unless the oracle's top-2 gap is below
1e-4 * ||logits||_2 (tests/models.py).
"""
import dataclasses

import pytest

from models import Pair
from starlight_amd.graph import LLAMA_1B_INT4, LLAMA_8B_INT4

pytestmark = pytest.mark.gpu


def test_1b_class_all_16_layers(hip):
    """16 layers, hidden 2048, 32/8 heads x 64, ffn 8192, vocab 32000,
    INT4 g128: a 64-token prompt (graph-replayed on its second run), then
    8 decode steps, KV cache for 2048 positions."""
    pair = Pair(hip, LLAMA_1B_INT4, batch=1, prompt_len=64, max_seq=2048, seed=30)
    try:
        ids = pair.prefill(repeats=2)
        steps = pair.decode(ids, 8)
        assert len(steps) == 8
        assert pair.mismatched_ids <= 1
    finally:
        pair.close()


def test_8b_shape_8_layers_full_vocab_past_1024(hip):
    """8 layers of the 8B shape (hidden 4096, 32/8 heads x 128, ffn 14336,
    INT4 g128 with an INT4 lm_head of [128256 x 4096]), KV cache for 4096
    positions with 1024 seeded ones: a 40-token prompt at positions
    1024-1063, then 4 decode steps."""
    cfg = dataclasses.replace(LLAMA_8B_INT4, layers=8)
    pair = Pair(hip, cfg, batch=1, prompt_len=40, max_seq=4096, seed=31)
    try:
        pair.seed_cache(1024, seed=32)
        ids = pair.prefill(repeats=2)
        steps = pair.decode(ids, 4)
        assert len(steps) == 4
        assert pair.mismatched_ids <= 1
    finally:
        pair.close()
