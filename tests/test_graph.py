"""Lowering and static memory planning (restated sl-graph / sl-model-adapters
slices): op counts, plan invariants of ARCH-0004 §7, determinism."""
import random

import numpy as np
import pytest

from starlight_amd import graph
from starlight_amd.ir import Command, Op, OpCode, Value, ValueRole


@pytest.mark.parametrize("cfg,layers", [(graph.TINY, 2), (graph.LLAMA_1B_INT4, 16), (graph.LLAMA_8B_INT4, 32)])
@pytest.mark.parametrize("seq", [1, 7])
def test_llama_lowering_shape_and_plan(cfg, layers, seq):
    lw = graph.lower_llama(cfg, 1, seq, 64)
    cmds = lw.ir.commands
    assert len(cmds) == 16 * layers + 4
    assert [c.op.code for c in cmds[:2]] == [OpCode.GATHER, OpCode.RMS_NORM]
    assert [c.op.code for c in cmds[-3:]] == [OpCode.LAST_TOKEN, OpCode.RMS_NORM, OpCode.MATMUL_NT]
    assert sum(c.op.code == OpCode.CAUSAL_ATTENTION for c in cmds) == layers
    assert sum(c.op.code == OpCode.SWIGLU for c in cmds) == layers
    graph.validate_plan(lw.ir.values, cmds, lw.ir.plan)
    assert lw.ir.values[lw.logits].shape == (1, cfg.vocab)


def test_lowering_is_deterministic():
    a = graph.lower_llama(graph.TINY, 1, 5, 32)
    b = graph.lower_llama(graph.TINY, 1, 5, 32)
    assert repr(a.ir) == repr(b.ir)


def test_fixture_program_command_order():
    """rt/tests/fixture_compile.rs:35-48."""
    lw = graph.lower_fixture(2)
    assert [c.op.code for c in lw.ir.commands] == [OpCode.GATHER, OpCode.RMS_NORM, OpCode.MATMUL_NT,
                                                   OpCode.LAST_TOKEN]
    graph.validate_plan(lw.ir.values, lw.ir.commands, lw.ir.plan)


def test_plan_of_a_random_100_node_graph_has_no_conflicts():
    """ARCH-0004 §7 acceptance: 100 nodes with overlapping lifetimes; any two
    values sharing bytes have disjoint lifetimes (validate_plan checks it)."""
    rnd = random.Random(5)
    values = [Value.f32([rnd.randint(1, 300)], ValueRole.TEMP) for _ in range(120)]
    commands = []
    for i in range(100):
        ins = rnd.sample(range(i + 1), min(2, i + 1)) if i else []
        commands.append(Command(Op.add(), ins, [i + 1]))
    plan = graph.plan_memory(values, commands)
    graph.validate_plan(values, commands, plan)
    total = sum(v.byte_size() for i, v in enumerate(values) if i <= 100)
    assert plan.scratchpad_bytes < total  # reuse happened


def test_plan_rejects_a_planted_conflict():
    """The invariant check itself catches two live values sharing bytes."""
    values = [Value.f32([64], ValueRole.TEMP) for _ in range(3)]
    commands = [Command(Op.add(), [], [0]), Command(Op.add(), [0], [1]), Command(Op.add(), [0, 1], [2])]
    plan = graph.plan_memory(values, commands)
    graph.validate_plan(values, commands, plan)
    plan.slots[1].offset = plan.slots[0].offset
    with pytest.raises(AssertionError):
        graph.validate_plan(values, commands, plan)
