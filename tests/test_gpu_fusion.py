"""Fused submission units on the GPU, against the oracle run op by op.

The device fuses SplitHeads x3 + Rope x2 + CausalAttention + MergeHeads into
the decode attention kernels, and for prefill chunks into one pass that
splits, rotates and appends followed by the prefill attention. The split and rotated heads are written only
when a later command of the same submission reads them (dead ones, every
element overwritten before any read, are skipped). These tests lay the values
out in one scratch buffer, make the intermediates dead with a later Scale over
their region, and check the attention output, the merged heads and the KV
cache; variants where a later command reads an intermediate, or where nothing
overwrites them, must fuse as well and leave every intermediate as the op
sequence would.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import assert_elementwise, assert_normwise, rel_l2
from starlight_amd.device import DeviceError
from starlight_amd.ir import BufferRef, Op, RopeVariant, Value, ValueRole

pytestmark = pytest.mark.gpu

CASES = [
    # batch, heads, kv_heads, seq, past_len, head_dim, max_seq, variant
    (1, 32, 8, 1, 1000, 128, 1100, RopeVariant.NEOX),   # 8B-shaped decode step
    (1, 8, 2, 1, 77, 256, 128, RopeVariant.NEOX),
    (2, 16, 4, 1, 300, 128, 512, RopeVariant.GPTJ),
    (1, 8, 2, 2, 40, 64, 64, RopeVariant.GPTJ),         # two-token chunk, head_dim 64
    (1, 4, 4, 1, 0, 128, 16, RopeVariant.NEOX),         # first token
    (1, 32, 8, 1, 300, 64, 512, RopeVariant.NEOX),      # 1B-shaped decode step: head_dim 64, NeoX pairs across lanes
    (2, 8, 2, 3, 20, 64, 64, RopeVariant.NEOX),         # head_dim 64 NeoX, three-token chunk, batch 2
    (1, 32, 8, 64, 0, 128, 128, RopeVariant.NEOX),      # 8B-shaped prefill of 64 tokens
    (2, 8, 2, 40, 17, 64, 128, RopeVariant.GPTJ),       # prefill chunk after a prefix, batch 2, head_dim 64
    (1, 4, 4, 20, 5, 128, 64, RopeVariant.NEOX),        # MHA prefill chunk of 20 after 5
]


def run_group(hip, case, consume_intermediate, keep_all=False):
    B, H, Hkv, S, past, D, max_seq, variant = case
    r = np.random.default_rng(sum(case[:-1]))
    nq, nk = B * S * H * D, B * S * Hkv * D
    q = r.uniform(-1, 1, nq).astype(np.float32)
    k = r.uniform(-1, 1, nk).astype(np.float32)
    v = r.uniform(-1, 1, nk).astype(np.float32)
    cache = r.uniform(-1, 1, B * 1 * 2 * max_seq * Hkv * D).astype(np.float32)
    pos = (past + np.arange(S, dtype=np.uint32))[None, :].repeat(B, 0).ravel()
    theta = 500000.0
    scale = float(np.float32(1.0 / math.sqrt(D)))

    # scratch layout: q k v | qh kh vh qr kr | att merged
    offs = {}
    cur = 0
    for name, size in [("q", nq), ("k", nk), ("v", nk), ("qh", nq), ("kh", nk), ("vh", nk), ("qr", nq),
                       ("kr", nk), ("att", nq), ("merged", nq)]:
        offs[name] = (cur, size)
        cur += (size + 63) // 64 * 64
    scratch = hip.allocate_f32(cur, 256)
    init = np.zeros(cur, np.float32)
    for name, arr in (("q", q), ("k", k), ("v", v)):
        o, n = offs[name]
        init[o:o + n] = arr
    hip.upload_f32(scratch, init)
    ref = {name: BufferRef(scratch, o, n) for name, (o, n) in offs.items()}
    cb = hip.upload_new_f32(cache)
    pb = hip.upload_new_u32(pos)
    posr = BufferRef(pb, 0, B * S)

    inter_lo = offs["qh"][0]
    inter_hi = offs["kr"][0] + offs["kr"][1]
    # (uploads submit the log, so everything is uploaded before the group)
    src = hip.upload_new_f32(np.ones(inter_hi - inter_lo, np.float32))
    extra = hip.allocate_f32(nq, 256) if consume_intermediate else None

    qf, kf = Value.f32([B, S, H * D]), Value.f32([B, S, Hkv * D])
    q4, k4 = Value.f32([B, H, S, D]), Value.f32([B, Hkv, S, D])
    pv = Value.u32([B, S])
    before = hip.stats()
    hip.dispatch(Op.split_heads(H, D), [ref["q"]], [qf], [ref["qh"]], [q4])
    hip.dispatch(Op.split_heads(Hkv, D), [ref["k"]], [kf], [ref["kh"]], [k4])
    hip.dispatch(Op.split_heads(Hkv, D), [ref["v"]], [kf], [ref["vh"]], [k4])
    hip.dispatch(Op.rope(variant, theta), [ref["qh"], posr], [q4, pv], [ref["qr"]], [q4])
    hip.dispatch(Op.rope(variant, theta), [ref["kh"], posr], [k4, pv], [ref["kr"]], [k4])
    hip.dispatch(Op.causal_attention(0, H, Hkv, D, scale),
                 [ref["qr"], ref["kr"], ref["vh"], BufferRef(cb, 0, cache.size)],
                 [q4, k4, k4, Value.f32([B, 1, 2, max_seq, Hkv, D], ValueRole.STATE)],
                 [ref["att"]], [q4], [past])
    hip.dispatch(Op.merge_heads(H, D), [ref["att"]], [q4], [ref["merged"]], [qf])
    span = BufferRef(scratch, inter_lo, inter_hi - inter_lo)
    sv = Value.f32([inter_hi - inter_lo])
    if consume_intermediate:
        # a later read of qr keeps it alive: the group must run unfused
        hip.dispatch(Op.scale_by(2.0), [ref["qr"]], [q4], [BufferRef(extra, 0, nq)], [q4])
    if not keep_all:
        # overwrite the split / rotated heads: they are dead after the group
        hip.dispatch(Op.scale_by(3.0), [BufferRef(src, 0, inter_hi - inter_lo)], [sv], [span], [sv])
    hip.synchronize()
    after = hip.stats()

    qh = oracle.split_heads(q, B, S, H, D)
    kh = oracle.split_heads(k, B, S, Hkv, D)
    vh = oracle.split_heads(v, B, S, Hkv, D)
    vname = "neox" if variant == RopeVariant.NEOX else "gptj"
    qr = oracle.rope(qh, pos, B, H, S, D, theta, vname)
    kr = oracle.rope(kh, pos, B, Hkv, S, D, theta, vname)
    want_att, want_cache = oracle.causal_attention(qr, kr, vh, cache, B, 1, 0, H, Hkv, S, past, D, max_seq, scale)
    want_merged = oracle.merge_heads(want_att, B, S, H, D)
    got = hip.read_f32(scratch, cur)
    got_cache = hip.read_f32(cb, cache.size)
    o, n = offs["att"]
    assert_normwise(got[o:o + n], want_att)
    o, n = offs["merged"]
    assert_normwise(got[o:o + n], want_merged)
    if keep_all:
        # nothing overwrites them: every intermediate holds the op's result
        for name, want in (("qh", qh), ("kh", kh), ("vh", vh)):
            o, n = offs[name]
            np.testing.assert_array_equal(got[o:o + n], want)
        for name, want in (("qr", qr), ("kr", kr)):
            o, n = offs[name]
            assert_elementwise(got[o:o + n], want)  # RoPE: elementwise, 1e-6 relative per element
    else:
        assert np.all(got[inter_lo:inter_hi] == 3.0)
    # the appended K rows are rotated (1e-6 per element), V rows copied;
    # every other cache position is untouched
    assert_elementwise(got_cache, want_cache)
    gc = got_cache.reshape(B, 2, max_seq, Hkv * D)
    wc = want_cache.reshape(B, 2, max_seq, Hkv * D)
    untouched = np.ones(max_seq, bool)
    untouched[past:past + S] = False
    np.testing.assert_array_equal(gc[:, :, untouched], wc[:, :, untouched])
    np.testing.assert_array_equal(gc[:, 1, past:past + S], wc[:, 1, past:past + S])
    if extra is not None:
        np.testing.assert_array_equal(hip.read_f32(extra, nq), (qr * np.float32(2.0)).astype(np.float32))
    return after["fused_commands"] - before["fused_commands"]


@pytest.mark.parametrize("case", CASES)
def test_attention_group_fuses_and_matches(hip, case):
    fused = run_group(hip, case, consume_intermediate=False)
    B, H, Hkv, S, past, D, max_seq, variant = case
    if not fusable(case):
        assert fused == 0  # NEOX pairs of head_dim 192 span lanes and float4 slots: not fused
    else:
        assert fused >= 7


def fusable(case, live=False):
    """Decode-sized units (at most 16 query rows per KV head) fuse into the
    decode kernels, except NeoX at head_dim 192; prefill units (16 or more
    tokens, head_dim 64 or 128) into the prefill pass, when every
    intermediate is dead."""
    B, H, Hkv, S, past, D, max_seq, variant = case
    if (H // Hkv) * S <= 16:
        return not (variant == RopeVariant.NEOX and D // 64 == 3)
    return not live and S >= 16 and D in (64, 128)


@pytest.mark.parametrize("case", CASES[:2])
def test_attention_group_with_live_intermediate_fuses_and_writes_it(hip, case):
    fused = run_group(hip, case, consume_intermediate=True)
    assert fused >= 7 if fusable(case, live=True) else fused == 0


@pytest.mark.parametrize("case", CASES)
def test_attention_group_keeps_every_live_intermediate(hip, case):
    fused = run_group(hip, case, consume_intermediate=False, keep_all=True)
    assert fused >= 7 if fusable(case, live=True) else fused == 0


# The scratch layout of the last layer of an 8B-shaped step as the memory
# plan lays it out (floats per token): q/k/v projections, then the split and
# rotated heads reusing their space. The rotated q overlaps the q tail, k and
# v, which the fused kernels still read, and MergeHeads leaves its last 1024
# floats per token holding it when nothing after the group overwrites them.
LAST_LAYER = {"q": (8192, 4096), "k": (12288, 1024), "v": (13312, 1024), "qh": (4096, 4096),
              "kh": (8192, 1024), "vh": (9216, 1024), "qr": (10240, 4096), "kr": (4096, 1024),
              "att": (5120, 4096), "merged": (9216, 4096)}


@pytest.mark.parametrize("projection_after", [True, False])
@pytest.mark.parametrize("S,past,max_seq", [(1, 1000, 1100), (64, 100, 256)])
def test_attention_group_stages_rotated_q_that_overlaps_its_inputs(hip, projection_after, S, past, max_seq):
    """A decode step (one token) and a 64-token prefill chunk laid out as
    the last layer's plan: the rotated q is live (its tail survives) and is
    staged and copied into place. The prefill form takes no other live
    intermediate, so without the projection (which overwrites the rotated
    k) its unit runs unfused."""
    B, H, Hkv, D = 1, 32, 8, 128
    theta, scale = 500000.0, float(np.float32(1.0 / math.sqrt(D)))
    r = np.random.default_rng(31 + S)
    nq, nk, total = B * S * H * D, B * S * Hkv * D, 14336 * S
    layout = {name: (o * S, n * S) for name, (o, n) in LAST_LAYER.items()}
    q = r.uniform(-1, 1, nq).astype(np.float32)
    k = r.uniform(-1, 1, nk).astype(np.float32)
    v = r.uniform(-1, 1, nk).astype(np.float32)
    cache = r.uniform(-1, 1, B * 2 * max_seq * Hkv * D).astype(np.float32)
    pos = (past + np.arange(B * S)).astype(np.uint32)
    init = np.zeros(total, np.float32)
    for name, arr in (("q", q), ("k", k), ("v", v)):
        o, n = layout[name]
        init[o:o + n] = arr
    scratch = hip.upload_new_f32(init)
    cb = hip.upload_new_f32(cache)
    pb = hip.upload_new_u32(pos)
    proj = r.uniform(-1, 1, 4096 * S).astype(np.float32)
    pr = hip.upload_new_f32(proj)
    ref = {name: BufferRef(scratch, o, n) for name, (o, n) in layout.items()}
    posr = BufferRef(pb, 0, B * S)
    qf, kf = Value.f32([B, S, H * D]), Value.f32([B, S, Hkv * D])
    q4, k4 = Value.f32([B, H, S, D]), Value.f32([B, Hkv, S, D])
    pv = Value.u32([B, S])
    before = hip.stats()
    hip.dispatch(Op.split_heads(H, D), [ref["q"]], [qf], [ref["qh"]], [q4])
    hip.dispatch(Op.split_heads(Hkv, D), [ref["k"]], [kf], [ref["kh"]], [k4])
    hip.dispatch(Op.split_heads(Hkv, D), [ref["v"]], [kf], [ref["vh"]], [k4])
    hip.dispatch(Op.rope(RopeVariant.NEOX, theta), [ref["qh"], posr], [q4, pv], [ref["qr"]], [q4])
    hip.dispatch(Op.rope(RopeVariant.NEOX, theta), [ref["kh"], posr], [k4, pv], [ref["kr"]], [k4])
    hip.dispatch(Op.causal_attention(0, H, Hkv, D, scale),
                 [ref["qr"], ref["kr"], ref["vh"], BufferRef(cb, 0, cache.size)],
                 [q4, k4, k4, Value.f32([B, 1, 2, max_seq, Hkv, D], ValueRole.STATE)],
                 [ref["att"]], [q4], [past])
    hip.dispatch(Op.merge_heads(H, D), [ref["att"]], [q4], [ref["merged"]], [qf])
    if projection_after:
        # in place of the output projection, which writes [4096, 8192) per token
        pvv = Value.f32([4096 * S])
        hip.dispatch(Op.scale_by(2.0), [BufferRef(pr, 0, 4096 * S)], [pvv], [BufferRef(scratch, 4096 * S, 4096 * S)],
                     [pvv])
    hip.synchronize()
    after = hip.stats()
    fused = after["fused_commands"] - before["fused_commands"]
    if S == 1 or projection_after:
        assert fused >= 7
    else:
        assert fused == 0

    # the op sequence on the oracle, writing the same layout in order
    qh = oracle.split_heads(q, B, S, H, D)
    kh = oracle.split_heads(k, B, S, Hkv, D)
    vh = oracle.split_heads(v, B, S, Hkv, D)
    qr = oracle.rope(qh, pos, B, H, S, D, theta, "neox")
    kr = oracle.rope(kh, pos, B, Hkv, S, D, theta, "neox")
    att, want_cache = oracle.causal_attention(qr, kr, vh, cache, B, 1, 0, H, Hkv, S, past, D, max_seq, scale)
    merged = oracle.merge_heads(att, B, S, H, D)
    want = init.copy()
    kind = np.zeros(total, np.int8)  # 0 exact, 1 Rope, 2 attention
    steps = [("qh", qh, 0), ("kh", kh, 0), ("vh", vh, 0), ("qr", qr, 1), ("kr", kr, 1), ("att", att, 2),
             ("merged", merged, 2)]
    for name, val, kd in steps:
        o, n = layout[name]
        want[o:o + n] = val
        kind[o:o + n] = kd
    if projection_after:
        want[4096 * S:8192 * S] = proj * np.float32(2.0)
        kind[4096 * S:8192 * S] = 0
    got = hip.read_f32(scratch, total)
    np.testing.assert_array_equal(got[kind == 0], want[kind == 0])
    assert_elementwise(got[kind == 1], want[kind == 1])
    assert_normwise(got[kind == 2], want[kind == 2])
    # the rotated q tail is what the staged copy wrote
    assert np.count_nonzero(kind == 1) >= 1024 * S
    assert_elementwise(hip.read_f32(cb, cache.size), want_cache)


@pytest.mark.parametrize("silu_first", [True, False])
@pytest.mark.parametrize("dead", [True, False])
def test_silu_then_mul_fuses_only_when_the_silu_result_is_dead(hip, silu_first, dead):
    n = 10007  # ragged: vector body plus a scalar tail
    r = np.random.default_rng(41 + silu_first + 2 * dead)
    x = (r.standard_normal(n) * 4).astype(np.float32)
    u = r.standard_normal(n).astype(np.float32)
    src = r.standard_normal(n).astype(np.float32)
    # scratch layout: x | u | t | out | src
    stride = (n + 63) // 64 * 64
    init = np.zeros(5 * stride, np.float32)
    init[0:n], init[stride:stride + n], init[4 * stride:4 * stride + n] = x, u, src
    v = Value.f32([n])

    def run(fusion):
        buf = hip.upload_new_f32(init)
        xr, ur, tr, outr, srcr = [BufferRef(buf, i * stride, n) for i in range(5)]
        hip.set_options(fusion=fusion)
        before = hip.stats()
        hip.dispatch(Op.silu(), [xr], [v], [tr], [v])
        hip.dispatch(Op.mul(), [tr, ur] if silu_first else [ur, tr], [v, v], [outr], [v])
        if dead:
            hip.dispatch(Op.scale_by(0.5), [srcr], [v], [tr], [v])  # overwrites every element of t
        hip.synchronize()
        fused = hip.stats()["fused_commands"] - before["fused_commands"]
        hip.set_options()
        got = hip.read_f32(buf, 5 * stride)
        return fused, got[3 * stride:3 * stride + n], got[2 * stride:2 * stride + n]

    fused, out, t = run(True)
    assert fused == (2 if dead else 0)
    unfused, out_ref, t_ref = run(False)
    assert unfused == 0
    # the same IEEE operations as the op pair: bit-identical to it
    np.testing.assert_array_equal(out, out_ref)
    np.testing.assert_array_equal(t, t_ref)
    t_want = oracle.silu(x)
    want = oracle.mul(t_want, u, n) if silu_first else oracle.mul(u, t_want, n)
    assert_elementwise(out, want)
    if dead:
        np.testing.assert_array_equal(t, oracle.scale(src, 0.5))
    else:
        assert_elementwise(t, t_want)


def test_projection_after_attention_when_the_mirror_does_not_fit(hip, monkeypatch):
    """A device whose workspace holds the decode partials but not the copy of
    the merged heads the chained output projection would read: the
    projection runs on its own from MergeHeads' output, which must then be
    written (8B decode shapes at 1000 cached positions, INT4 o-proj, and the
    residual Add)."""
    from starlight_amd import quant
    from starlight_amd.device import HipDevice
    from starlight_amd.ir import QuantFormat

    B, H, Hkv, S, past, D, max_seq = 1, 32, 8, 1, 1000, 128, 1100
    parts = (max_seq + 127) // 128
    partials = B * Hkv * parts * (H // Hkv) * S * (4 + D)  # floats of the decode partials
    monkeypatch.setenv("SL_HIP_WORKSPACE_BYTES", str((partials + 2048) * 4))
    small = HipDevice(0)
    try:
        theta, scale = 500000.0, float(np.float32(1.0 / math.sqrt(D)))
        r = np.random.default_rng(77)
        nq, nk = B * S * H * D, B * S * Hkv * D
        q, k, v = (r.uniform(-1, 1, n).astype(np.float32) for n in (nq, nk, nk))
        cache = r.uniform(-1, 1, B * 2 * max_seq * Hkv * D).astype(np.float32)
        resid = r.standard_normal(4096).astype(np.float32)
        w = (r.standard_normal((4096, H * D)) * 0.02).astype(np.float32)
        words, scales = quant.quantize(w, 128, QuantFormat.INT4)
        wb, sb = small.upload_new_u32(words), small.upload_new_f32(scales)
        small.bind_quantized(wb, sb, QuantFormat.INT4, 128, 4096, H * D)
        pos = np.full(B * S, past, np.uint32)
        names = [("q", nq), ("k", nk), ("v", nk), ("qh", nq), ("kh", nk), ("vh", nk), ("qr", nq), ("kr", nk),
                 ("att", nq), ("merged", nq), ("o", 4096), ("h2", 4096)]
        offs, cur = {}, 0
        for name, n in names:
            offs[name] = (cur, n)
            cur += (n + 63) // 64 * 64
        init = np.zeros(cur, np.float32)
        for name, arr in (("q", q), ("k", k), ("v", v)):
            o, n = offs[name]
            init[o:o + n] = arr
        scratch = small.upload_new_f32(init)
        cb, pb, rb = small.upload_new_f32(cache), small.upload_new_u32(pos), small.upload_new_f32(resid)
        ref = {name: BufferRef(scratch, o, n) for name, (o, n) in offs.items()}
        posr = BufferRef(pb, 0, B * S)
        qf, kf = Value.f32([B, S, H * D]), Value.f32([B, S, Hkv * D])
        q4, k4 = Value.f32([B, H, S, D]), Value.f32([B, Hkv, S, D])
        hv = Value.f32([B, S, 4096])
        before = small.stats()
        small.dispatch(Op.split_heads(H, D), [ref["q"]], [qf], [ref["qh"]], [q4])
        small.dispatch(Op.split_heads(Hkv, D), [ref["k"]], [kf], [ref["kh"]], [k4])
        small.dispatch(Op.split_heads(Hkv, D), [ref["v"]], [kf], [ref["vh"]], [k4])
        small.dispatch(Op.rope(RopeVariant.NEOX, theta), [ref["qh"], posr], [q4, Value.u32([B, S])], [ref["qr"]],
                       [q4])
        small.dispatch(Op.rope(RopeVariant.NEOX, theta), [ref["kh"], posr], [k4, Value.u32([B, S])], [ref["kr"]],
                       [k4])
        small.dispatch(Op.causal_attention(0, H, Hkv, D, scale),
                       [ref["qr"], ref["kr"], ref["vh"], BufferRef(cb, 0, cache.size)],
                       [q4, k4, k4, Value.f32([B, 1, 2, max_seq, Hkv, D], ValueRole.STATE)], [ref["att"]], [q4],
                       [past])
        small.dispatch(Op.merge_heads(H, D), [ref["att"]], [q4], [ref["merged"]], [qf])
        small.dispatch(Op.matmul_nt(), [ref["merged"], BufferRef(wb, 0, words.size)],
                       [qf, Value.quantized([4096, H * D], QuantFormat.INT4, 128)], [ref["o"]], [hv])
        small.dispatch(Op.add(), [BufferRef(rb, 0, 4096), ref["o"]], [hv, hv], [ref["h2"]], [hv])
        small.synchronize()
        assert small.stats()["fused_commands"] - before["fused_commands"] >= 7
        got = small.read_f32(scratch, cur)
    finally:
        small.close()
    qh, kh, vh = (oracle.split_heads(x, B, S, h, D) for x, h in ((q, H), (k, Hkv), (v, Hkv)))
    qr = oracle.rope(qh, pos, B, H, S, D, theta, "neox")
    kr = oracle.rope(kh, pos, B, Hkv, S, D, theta, "neox")
    att, _ = oracle.causal_attention(qr, kr, vh, cache, B, 1, 0, H, Hkv, S, past, D, max_seq, scale)
    merged = oracle.merge_heads(att, B, S, H, D)
    o_want = oracle.matmul_nt(merged, quant.dequantize(words, scales, 4096, H * D, 128, QuantFormat.INT4), 1, 1,
                              H * D, 4096)
    for name, want in (("merged", merged), ("o", o_want)):
        o, n = offs[name]
        assert_normwise(got[o:o + n], want)
    o, n = offs["h2"]
    og, _ = offs["o"]
    np.testing.assert_array_equal(got[o:o + n], oracle.add(resid, got[og:og + 4096], 4096))


@pytest.mark.parametrize("variant", ["separate", "out_is_gemv_out", "out_is_residual", "swiglu", "norm_reads"])
def test_gemv_residual_add_fusions(hip, variant):
    """A quantized MatMulNT (or the SwiGlu down projection) followed by the
    residual Add runs as one launch with the Add in its epilogue. An Add
    writing over the GEMV's output or over its residual input never reaches
    the fusion: dispatch rejects an output overlapping an input
    (device.rs:338-377). When the residual operand is the output of the
    RmsNorm fused into the same launch, the Add stays separate: block 0
    writes that output while other blocks read it."""
    from starlight_amd import quant
    from starlight_amd.ir import QuantFormat

    r = np.random.default_rng(90 + len(variant))
    k, n, inter = 512, 512, 1024
    x = r.standard_normal(k).astype(np.float32)
    resid = r.standard_normal(n).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)

    def qw(rows, cols):
        w = (r.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        words, scales = quant.quantize(w, 128, QuantFormat.INT4)
        wb, sb = hip.upload_new_u32(words), hip.upload_new_f32(scales)
        hip.bind_quantized(wb, sb, QuantFormat.INT4, 128, rows, cols)
        return (BufferRef(wb, 0, words.size), Value.quantized([rows, cols], QuantFormat.INT4, 128),
                quant.dequantize(words, scales, rows, cols, 128, QuantFormat.INT4))

    # scratch: x | normed | y | resid | out
    stride = 1024
    init = np.zeros(5 * stride, np.float32)
    init[0:k], init[3 * stride:3 * stride + n] = x, resid
    buf = hip.upload_new_f32(init)
    X, NORMED, Y, RES, OUT = (BufferRef(buf, i * stride, n) for i in range(5))
    gb = hip.upload_new_f32(gamma)
    xv, yv = Value.f32([1, 1, k]), Value.f32([1, 1, n])
    before = hip.stats()
    if variant == "swiglu":
        g, u, d = qw(inter, k), qw(inter, k), qw(n, inter)
        hip.dispatch(Op.swiglu(), [X, g[0], u[0], d[0]], [xv, g[1], u[1], d[1]], [Y], [yv])
        y_want = oracle.swiglu(x, g[2], u[2], d[2], 1, k, inter)
        add_in, add_out = [RES, Y], OUT
        resid_want = resid
    elif variant == "norm_reads":
        w = qw(n, k)
        hip.dispatch(Op.rms_norm(1e-5), [X, BufferRef(gb, 0, k)], [xv, Value.f32([k], ValueRole.PARAM)], [NORMED],
                     [xv])
        hip.dispatch(Op.matmul_nt(), [NORMED, w[0]], [xv, w[1]], [Y], [yv])
        normed = oracle.rms_norm(x, gamma, 1, k, 1e-5)
        y_want = oracle.matmul_nt(normed, w[2], 1, 1, k, n)
        add_in, add_out = [NORMED, Y], OUT  # the residual operand is the norm's output
        resid_want = normed
    else:
        w = qw(n, k)
        hip.dispatch(Op.matmul_nt(), [X, w[0]], [xv, w[1]], [Y], [yv])
        y_want = oracle.matmul_nt(x, w[2], 1, 1, k, n)
        add_out = {"separate": OUT, "out_is_gemv_out": Y, "out_is_residual": RES}[variant]
        add_in = [RES, Y]
        resid_want = resid
    if add_out is not OUT:
        with pytest.raises(DeviceError) as e:
            hip.dispatch(Op.add(), add_in, [yv, yv], [add_out], [yv])
        assert e.value == DeviceError.execution("a command output aliases an overlapping input range")
        hip.synchronize()
        assert_normwise(hip.read_f32(buf, 5 * stride)[Y.offset:Y.offset + n], y_want)
        return
    hip.dispatch(Op.add(), add_in, [yv, yv], [add_out], [yv])
    hip.synchronize()
    fused = hip.stats()["fused_commands"] - before["fused_commands"]
    got = hip.read_f32(buf, 5 * stride)
    y_got = got[Y.offset:Y.offset + n]
    out_got = got[add_out.offset:add_out.offset + n]
    assert_normwise(y_got, y_want)
    np.testing.assert_array_equal(out_got, oracle.add(resid_want, y_got, n))
    if variant == "norm_reads":
        assert fused == 2  # RmsNorm + MatMulNT; the Add runs on its own
        assert_normwise(got[NORMED.offset:NORMED.offset + k], resid_want)
    else:
        assert fused == 2  # MatMulNT (or SwiGlu) + Add


@pytest.mark.parametrize("fmt_name", ["INT4", "INT8"])
def test_prefill_norm_and_projections_run_as_one_gemm(hip, fmt_name):
    """RmsNorm and three quantized MatMulNT reading its output, at 64 rows
    (prefill): the norm runs on its own, then q/k/v as one q-GEMM launch over
    one activation split. Every output — the norm's and each projection's —
    matches the oracle (norm per element at 1e-6, projections normwise per
    row at 1e-4), and the unit counts as fused; a SwiGlu at 64 rows (gate
    and up in one launch) matches too."""
    from starlight_amd import quant
    from starlight_amd.ir import QuantFormat

    fmt = QuantFormat[fmt_name]
    r = np.random.default_rng(120 + len(fmt_name))
    rows, k, nq, nkv, inter = 64, 512, 512, 128, 384
    x = r.standard_normal((rows, k)).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)

    def qw(n, cols):
        w = (r.standard_normal((n, cols)) * 0.05).astype(np.float32)
        words, scales = quant.quantize(w, 128, fmt)
        wb, sb = hip.upload_new_u32(words), hip.upload_new_f32(scales)
        hip.bind_quantized(wb, sb, fmt, 128, n, cols)
        return (BufferRef(wb, 0, words.size), Value.quantized([n, cols], fmt, 128),
                quant.dequantize(words, scales, n, cols, 128, fmt))

    wq, wk, wv = qw(nq, k), qw(nkv, k), qw(nkv, k)
    X = BufferRef(hip.upload_new_f32(x.ravel()), 0, rows * k)
    G = BufferRef(hip.upload_new_f32(gamma), 0, k)
    N = BufferRef(hip.allocate_f32(rows * k, 256), 0, rows * k)
    outs = {name: BufferRef(hip.allocate_f32(rows * n, 256), 0, rows * n) for name, n in
            (("q", nq), ("k", nkv), ("v", nkv))}
    xv = Value.f32([1, rows, k])
    before = hip.stats()
    hip.dispatch(Op.rms_norm(1e-5), [X, G], [xv, Value.f32([k], ValueRole.PARAM)], [N], [xv])
    for name, w, n in (("q", wq, nq), ("k", wk, nkv), ("v", wv, nkv)):
        hip.dispatch(Op.matmul_nt(), [N, w[0]], [xv, w[1]], [outs[name]], [Value.f32([1, rows, n])])
    hip.synchronize()
    assert hip.stats()["fused_commands"] - before["fused_commands"] == 4
    normed = oracle.rms_norm(x.ravel(), gamma, rows, k, 1e-5)
    assert_elementwise(hip.read_f32(N.buffer, rows * k), normed)
    for name, w, n in (("q", wq, nq), ("k", wk, nkv), ("v", wv, nkv)):
        got = hip.read_f32(outs[name].buffer, rows * n).reshape(rows, n)
        want = oracle.matmul_nt(normed, w[2], 1, rows, k, n).reshape(rows, n)
        for i in range(rows):
            assert_normwise(got[i], want[i])

    g, u, d = qw(inter, k), qw(inter, k), qw(k, inter)
    Y = BufferRef(hip.allocate_f32(rows * k, 256), 0, rows * k)
    hip.dispatch(Op.swiglu(), [X, g[0], u[0], d[0]], [xv, g[1], u[1], d[1]], [Y], [xv])
    got = hip.read_f32(Y.buffer, rows * k).reshape(rows, k)
    want = oracle.swiglu(x.ravel(), g[2], u[2], d[2], rows, k, inter).reshape(rows, k)
    for i in range(rows):
        assert_normwise(got[i], want[i])


@pytest.mark.parametrize("fmt_name,k", [("INT4", 512), ("INT4", 4096), ("INT8", 2048)])
def test_prefill_norm_inside_the_activation_split(hip, fmt_name, k):
    """RmsNorm at 64 rows whose output nothing reads after its projections
    (a later command overwrites it): the norm runs inside the q-GEMM's
    activation split and its output is never written. Two units: q/k/v
    (three MatMulNT as one launch), and a SwiGlu with the residual Add of
    the norm's input after it (h2 = h + ffn(norm(h))), once also with h2
    written over the norm output by the unit's own Add. Each result
    is bit-identical to the same commands with the norm output left live
    (the norm then runs as its own launch first), and matches the oracle
    normwise per row (1e-4)."""
    from starlight_amd import quant
    from starlight_amd.ir import QuantFormat

    fmt = QuantFormat[fmt_name]
    r = np.random.default_rng(k + len(fmt_name))
    rows, nq, nkv, inter = 64, 256, 128, 384
    x = r.standard_normal((rows, k)).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)

    def qw(n, cols):
        w = (r.standard_normal((n, cols)) * 0.05).astype(np.float32)
        words, scales = quant.quantize(w, 128, fmt)
        wb, sb = hip.upload_new_u32(words), hip.upload_new_f32(scales)
        hip.bind_quantized(wb, sb, fmt, 128, n, cols)
        return (BufferRef(wb, 0, words.size), Value.quantized([n, cols], fmt, 128),
                quant.dequantize(words, scales, n, cols, 128, fmt))

    wq, wk, wv = qw(nq, k), qw(nkv, k), qw(nkv, k)
    g, u, d = qw(inter, k), qw(inter, k), qw(k, inter)
    G = BufferRef(hip.upload_new_f32(gamma), 0, k)
    xv, gv = Value.f32([1, rows, k]), Value.f32([k], ValueRole.PARAM)
    normed = oracle.rms_norm(x.ravel(), gamma, rows, k, 1e-5)

    def run(dead, add_into_norm=False):
        X = BufferRef(hip.upload_new_f32(x.ravel()), 0, rows * k)
        N = BufferRef(hip.allocate_f32(rows * k, 256), 0, rows * k)
        W = BufferRef(hip.upload_new_f32(np.ones(rows * k, np.float32)), 0, rows * k)
        outs = {name: BufferRef(hip.allocate_f32(rows * n, 256), 0, rows * n) for name, n in
                (("q", nq), ("k", nkv), ("v", nkv))}
        before = hip.stats()
        hip.dispatch(Op.rms_norm(1e-5), [X, G], [xv, gv], [N], [xv])
        for name, w, n in (("q", wq, nq), ("k", wk, nkv), ("v", wv, nkv)):
            hip.dispatch(Op.matmul_nt(), [N, w[0]], [xv, w[1]], [outs[name]], [Value.f32([1, rows, n])])
        if dead:
            hip.dispatch(Op.scale_by(2.0), [W], [xv], [N], [xv])
        hip.synchronize()
        assert hip.stats()["fused_commands"] - before["fused_commands"] == 4
        got = {name: hip.read_f32(o.buffer, o.len) for name, o in outs.items()}
        if dead:
            np.testing.assert_array_equal(hip.read_f32(N.buffer, rows * k), np.full(rows * k, 2, np.float32))
        # the feed-forward half of a layer: h2 = h + SwiGlu(norm(h))
        # (add_into_norm: the Add's output takes the norm output's place, as
        # a memory plan reuses it once the SwiGlu has read it)
        Y = BufferRef(hip.allocate_f32(rows * k, 256), 0, rows * k)
        H2 = N if add_into_norm else BufferRef(hip.allocate_f32(rows * k, 256), 0, rows * k)
        before = hip.stats()
        hip.dispatch(Op.rms_norm(1e-5), [X, G], [xv, gv], [N], [xv])
        hip.dispatch(Op.swiglu(), [N, g[0], u[0], d[0]], [xv, g[1], u[1], d[1]], [Y], [xv])
        hip.dispatch(Op.add(), [Y, X], [xv, xv], [H2], [xv])
        if dead and not add_into_norm:
            hip.dispatch(Op.scale_by(2.0), [W], [xv], [N], [xv])
        hip.synchronize()
        assert hip.stats()["fused_commands"] - before["fused_commands"] == 3
        got["h"] = hip.read_f32(H2.buffer, rows * k)
        return got

    folded, separate, overwritten = run(True), run(False), run(True, add_into_norm=True)
    for name in ("q", "k", "v", "h"):
        np.testing.assert_array_equal(folded[name], separate[name])
    np.testing.assert_array_equal(overwritten["h"], separate["h"])
    for name, w, n in (("q", wq, nq), ("k", wk, nkv), ("v", wv, nkv)):
        want = oracle.matmul_nt(normed, w[2], 1, rows, k, n).reshape(rows, n)
        for i in range(rows):
            assert_normwise(folded[name].reshape(rows, n)[i], want[i])
    ffn = oracle.swiglu(normed, g[2], u[2], d[2], rows, k, inter).reshape(rows, k)
    h = folded["h"].reshape(rows, k)
    for i in range(rows):
        assert_normwise(h[i] - x[i], ffn[i])


@pytest.mark.parametrize("fmt_name,residual", [("INT4", True), ("INT4", False), ("INT8", True)])
def test_long_k_gemv_with_many_rows(hip, fmt_name, residual):
    """A quantized MatMulNT with 8 rows of k = 14336 (the down projection at
    batch 8) has more activations than the fused GEMV's LDS holds: its grid
    cuts k into slices whose partial sums a second launch adds up, together
    with the residual Add when one follows (fused into the unit). The
    product matches the oracle per row (normwise 1e-4); the Add's output is
    exactly residual + the product."""
    from starlight_amd import quant
    from starlight_amd.ir import QuantFormat

    fmt = QuantFormat[fmt_name]
    r = np.random.default_rng(140 + residual + len(fmt_name))
    m, k, n = 8, 14336, 512
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    words, scales = quant.quantize(w, 128, fmt)
    wb, sb = hip.upload_new_u32(words), hip.upload_new_f32(scales)
    hip.bind_quantized(wb, sb, fmt, 128, n, k)
    deq = quant.dequantize(words, scales, n, k, 128, fmt)
    resid = r.standard_normal(m * n).astype(np.float32)
    X = BufferRef(hip.upload_new_f32(x.ravel()), 0, m * k)
    Y = BufferRef(hip.allocate_f32(m * n, 256), 0, m * n)
    R = BufferRef(hip.upload_new_f32(resid), 0, m * n)
    Z = BufferRef(hip.allocate_f32(m * n, 256), 0, m * n)
    yv = Value.f32([1, m, n])
    before = hip.stats()
    hip.dispatch(Op.matmul_nt(), [X, BufferRef(wb, 0, words.size)], [Value.f32([1, m, k]),
                 Value.quantized([n, k], fmt, 128)], [Y], [yv])
    if residual:
        hip.dispatch(Op.add(), [R, Y], [yv, yv], [Z], [yv])
    hip.synchronize()
    if residual:
        assert hip.stats()["fused_commands"] - before["fused_commands"] == 2
    got = hip.read_f32(Y.buffer, m * n).reshape(m, n)
    want = oracle.matmul_nt(x.ravel(), deq, 1, m, k, n).reshape(m, n)
    for i in range(m):
        assert_normwise(got[i], want[i])
    if residual:
        np.testing.assert_array_equal(hip.read_f32(Z.buffer, m * n), resid + got.ravel())


@pytest.mark.parametrize("alias", [False, True])
@pytest.mark.parametrize("variant", ["matmul", "swiglu", "norm_swiglu"])
def test_prefill_residual_add_in_the_gemm_epilogue(hip, variant, alias):
    """At 64 rows (prefill) a quantized MatMulNT, or a SwiGlu (after an
    RmsNorm), followed by the residual Add runs with the Add in the q-GEMM's
    epilogue (the SwiGlu's silu(g) * u formed by the down projection's
    activation split). Products match the oracle per row (normwise 1e-4);
    the Add's output is exactly residual + the product written. With alias,
    the Add writes over the product's input (the MatMulNT's or SwiGlu's
    activations), as a memory plan reusing their space after their last read
    does."""
    from starlight_amd import quant
    from starlight_amd.ir import QuantFormat

    r = np.random.default_rng(160 + len(variant))
    rows, k, n, inter = 64, 512, 512, 1024
    x = r.standard_normal((rows, k)).astype(np.float32)
    resid = r.standard_normal(rows * n).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(k)).astype(np.float32)

    def qw(nr, cols):
        w = (r.standard_normal((nr, cols)) * 0.05).astype(np.float32)
        words, scales = quant.quantize(w, 128, QuantFormat.INT4)
        wb, sb = hip.upload_new_u32(words), hip.upload_new_f32(scales)
        hip.bind_quantized(wb, sb, QuantFormat.INT4, 128, nr, cols)
        return (BufferRef(wb, 0, words.size), Value.quantized([nr, cols], QuantFormat.INT4, 128),
                quant.dequantize(words, scales, nr, cols, 128, QuantFormat.INT4))

    X = BufferRef(hip.upload_new_f32(x.ravel()), 0, rows * k)
    N = BufferRef(hip.allocate_f32(rows * k, 256), 0, rows * k)
    Y = BufferRef(hip.allocate_f32(rows * n, 256), 0, rows * n)
    R = BufferRef(hip.upload_new_f32(resid), 0, rows * n)
    Z = BufferRef(hip.allocate_f32(rows * n, 256), 0, rows * n)
    if alias:
        Z = N if variant == "norm_swiglu" else X
    xv, yv = Value.f32([1, rows, k]), Value.f32([1, rows, n])
    before = hip.stats()
    if variant == "matmul":
        w = qw(n, k)
        hip.dispatch(Op.matmul_nt(), [X, w[0]], [xv, w[1]], [Y], [yv])
        want = oracle.matmul_nt(x.ravel(), w[2], 1, rows, k, n)
        expect_fused = 2
    else:
        # weights first: an upload runs what the log holds so far
        g, u, dn = qw(inter, k), qw(inter, k), qw(n, inter)
        G = BufferRef(hip.upload_new_f32(gamma), 0, k)
        src = x.ravel()
        inp = X
        if variant == "norm_swiglu":
            hip.dispatch(Op.rms_norm(1e-5), [X, G],
                         [xv, Value.f32([k], ValueRole.PARAM)], [N], [xv])
            src = oracle.rms_norm(x.ravel(), gamma, rows, k, 1e-5)
            inp = N
        hip.dispatch(Op.swiglu(), [inp, g[0], u[0], dn[0]], [xv, g[1], u[1], dn[1]], [Y], [yv])
        want = oracle.swiglu(src, g[2], u[2], dn[2], rows, k, inter)
        expect_fused = 3 if variant == "norm_swiglu" else 2
    hip.dispatch(Op.add(), [R, Y], [yv, yv], [Z], [yv])
    hip.synchronize()
    assert hip.stats()["fused_commands"] - before["fused_commands"] == expect_fused
    got = hip.read_f32(Y.buffer, rows * n).reshape(rows, n)
    for i in range(rows):
        assert_normwise(got[i], want.reshape(rows, n)[i])
    np.testing.assert_array_equal(hip.read_f32(Z.buffer, rows * n), resid + got.ravel())
