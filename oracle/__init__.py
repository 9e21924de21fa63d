"""ORACLE — test infrastructure only.

ctypes front end over ``liboracle.so``, the scalar C restatement of StarLight's
``backend-cpu`` reference kernels (crates/backends/backend-cpu/src/reference/).
Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` import this package, and only to check or time against it; the
product package ``starlight_amd`` never imports it.

Functions take and return numpy arrays. Kernel errors raise ``OracleError``
carrying the reference's ``KernelError`` kind and static reason
(reference/mod.rs:44-61).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

KINDS = {1: "LengthMismatch", 2: "ShapeOverflow", 3: "InvalidShape", 4: "Unsupported"}


class OracleError(Exception):
    """A reference kernel rejected its arguments."""

    def __init__(self, kind: str, reason: str):
        super().__init__(f"{kind}: {reason}")
        self.kind = kind
        self.reason = reason


def build() -> str:
    """Compiles liboracle.so from sl_reference.c with the oracle Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_F = ctypes.POINTER(ctypes.c_float)
_U32 = ctypes.POINTER(ctypes.c_uint32)
_U8 = ctypes.POINTER(ctypes.c_uint8)
_I8 = ctypes.POINTER(ctypes.c_int8)
_SZ = ctypes.c_size_t
_WHY = ctypes.POINTER(ctypes.c_char_p)


def _declare(l: ctypes.CDLL) -> None:
    sigs = {
        "slr_matmul_nt": [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _WHY],
        "slr_matmul_nn": [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _WHY],
        "slr_softmax": [_F, _SZ, _SZ, _SZ, _WHY],
        "slr_softmax_causal": [_F, _SZ, _SZ, _SZ, _SZ, _SZ, _WHY],
        "slr_rms_norm": [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, ctypes.c_float, _WHY],
        "slr_rope_neox": [_F, _SZ, _U32, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _WHY],
        "slr_rope_gptj": [_F, _SZ, _U32, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _WHY],
        "slr_silu": [_F, _SZ, _WHY],
        "slr_mul": [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _WHY],
        "slr_add": [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _WHY],
        "slr_scale": [_F, _SZ, ctypes.c_float, _WHY],
        "slr_gather": [_F, _SZ, _U32, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _WHY],
        "slr_last_token": [_F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _WHY],
        "slr_split_heads": [_F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _WHY],
        "slr_merge_heads": [_F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _WHY],
        "slr_kv_append": [_F, _SZ, _F, _SZ, _F, _SZ] + [_SZ] * 8 + [_WHY],
        "slr_causal_attention": [_F, _SZ, _F, _SZ, _F, _SZ, _F, _SZ, _F, _SZ]
        + [_SZ] * 9
        + [ctypes.c_float, _WHY],
        "slr_swiglu": [_F, _SZ] * 5 + [_SZ, _SZ, _SZ, _WHY],
        "slr_rms_norm_matmul": [_F, _SZ] * 4 + [_SZ, _SZ, _SZ, ctypes.c_float, _WHY],
        "slr_paged_attention_decode": [_F, _F, _F, _F, _SZ, _U32, _U32, _F] + [_SZ] * 9 + [ctypes.c_float, _WHY],
        "slr_quantize_groupwise": [_F, _SZ, _SZ, _SZ, ctypes.c_int, _U8, _F, _WHY],
        "slr_unpack_codes": [_U8, _SZ, _SZ, ctypes.c_int, _I8, _WHY],
        "slr_dequantize_groupwise": [_U8, _F, _SZ, _SZ, _SZ, ctypes.c_int, _F, _WHY],
        "slr_lcg_next_u32": [ctypes.POINTER(ctypes.c_uint64)],
        "slr_lcg_fill": [ctypes.POINTER(ctypes.c_uint64), _F, _SZ, ctypes.c_float, ctypes.c_float],
        "slr_lcg_below": [ctypes.POINTER(ctypes.c_uint64), _SZ],
    }
    for name, args in sigs.items():
        fn = getattr(l, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    l.slr_set_threads.argtypes = [ctypes.c_int]
    l.slr_set_threads.restype = None
    l.slr_get_threads.argtypes = []
    l.slr_get_threads.restype = ctypes.c_int
    l.slr_lcg_next_u32.restype = ctypes.c_uint32
    l.slr_lcg_fill.restype = None
    l.slr_lcg_below.restype = ctypes.c_size_t


def set_threads(n: int) -> None:
    """Threads for the oracle's independent outputs (1 = the reference's
    sequential execution; results are bit-identical for any count)."""
    lib().slr_set_threads(int(n))


def get_threads() -> int:
    return int(lib().slr_get_threads())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray, ctype=_F):
    return a.ctypes.data_as(ctype)


def _check(rc: int, why: ctypes.c_char_p) -> None:
    if rc != 0:
        reason = why.value.decode() if why.value else ""
        raise OracleError(KINDS.get(rc, f"code {rc}"), reason)


def _call(name: str, *args) -> None:
    why = ctypes.c_char_p()
    rc = getattr(lib(), name)(*args, ctypes.byref(why))
    _check(rc, why)


# --------------------------------------------------------------------------
# Kernels. Arguments mirror the reference signatures; the slice lengths are
# taken from the arrays, so a short array reproduces LengthMismatch.
# --------------------------------------------------------------------------


def matmul_nt(a, b, batch, m, k, n, out_len=None):
    a, b = _f32(a), _f32(b)
    out = np.zeros(batch * m * n if out_len is None else out_len, np.float32)
    _call("slr_matmul_nt", _ptr(a), a.size, _ptr(b), b.size, _ptr(out), out.size, batch, m, k, n)
    return out


def matmul_nn(a, b, batch, m, k, n, out_len=None):
    a, b = _f32(a), _f32(b)
    out = np.zeros(batch * m * n if out_len is None else out_len, np.float32)
    _call("slr_matmul_nn", _ptr(a), a.size, _ptr(b), b.size, _ptr(out), out.size, batch, m, k, n)
    return out


def softmax(x, rows, cols):
    x = _f32(x).copy()
    _call("slr_softmax", _ptr(x), x.size, rows, cols)
    return x


def softmax_causal(x, rows, cols, seq, past_len):
    x = _f32(x).copy()
    _call("slr_softmax_causal", _ptr(x), x.size, rows, cols, seq, past_len)
    return x


def rms_norm(x, weight, rows, hidden, eps, out_len=None):
    x, weight = _f32(x), _f32(weight)
    out = np.zeros(rows * hidden if out_len is None else out_len, np.float32)
    _call("slr_rms_norm", _ptr(x), x.size, _ptr(weight), weight.size, _ptr(out), out.size, rows,
          hidden, eps)
    return out


def rope(x, positions, batch, heads, seq, head_dim, theta, variant="neox"):
    x = _f32(x).copy()
    positions = np.ascontiguousarray(positions, dtype=np.uint32)
    name = "slr_rope_neox" if variant == "neox" else "slr_rope_gptj"
    _call(name, _ptr(x), x.size, _ptr(positions, _U32), positions.size, batch, heads, seq,
          head_dim, theta)
    return x


def silu(x):
    x = _f32(x).copy()
    _call("slr_silu", _ptr(x), x.size)
    return x


def mul(a, b, length, out_len=None):
    a, b = _f32(a), _f32(b)
    out = np.zeros(length if out_len is None else out_len, np.float32)
    _call("slr_mul", _ptr(a), a.size, _ptr(b), b.size, _ptr(out), out.size, length)
    return out


def add(a, b, length, out_len=None):
    a, b = _f32(a), _f32(b)
    out = np.zeros(length if out_len is None else out_len, np.float32)
    _call("slr_add", _ptr(a), a.size, _ptr(b), b.size, _ptr(out), out.size, length)
    return out


def scale(x, factor):
    x = _f32(x).copy()
    _call("slr_scale", _ptr(x), x.size, factor)
    return x


def gather(table, ids, vocab, hidden, rows, out=None):
    table = _f32(table)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    if out is None:
        out = np.zeros(rows * hidden, np.float32)
    _call("slr_gather", _ptr(table), table.size, _ptr(ids, _U32), ids.size, _ptr(out), out.size,
          vocab, hidden, rows)
    return out


def last_token(inp, batch, seq, hidden, seq_len, out_len=None):
    inp = _f32(inp)
    out = np.zeros(batch * hidden if out_len is None else out_len, np.float32)
    _call("slr_last_token", _ptr(inp), inp.size, _ptr(out), out.size, batch, seq, hidden, seq_len)
    return out


def split_heads(inp, batch, seq, heads, head_dim, out_len=None):
    inp = _f32(inp)
    out = np.zeros(inp.size if out_len is None else out_len, np.float32)
    _call("slr_split_heads", _ptr(inp), inp.size, _ptr(out), out.size, batch, seq, heads, head_dim)
    return out


def merge_heads(inp, batch, seq, heads, head_dim, out_len=None):
    inp = _f32(inp)
    out = np.zeros(inp.size if out_len is None else out_len, np.float32)
    _call("slr_merge_heads", _ptr(inp), inp.size, _ptr(out), out.size, batch, seq, heads, head_dim)
    return out


def kv_append(k, v, cache, batch, layers, layer, kv_heads, head_dim, max_seq, past_len, seq):
    """Returns the updated cache (the input cache array is not modified)."""
    k, v = _f32(k), _f32(v)
    cache = _f32(cache).copy()
    _call("slr_kv_append", _ptr(k), k.size, _ptr(v), v.size, _ptr(cache), cache.size, batch, layers,
          layer, kv_heads, head_dim, max_seq, past_len, seq)
    return cache


def causal_attention(q, k, v, cache, batch, layers, layer, heads, kv_heads, seq, past_len, head_dim,
                     max_seq, scale_, out_len=None):
    """Returns (out, updated cache)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    cache = _f32(cache).copy()
    out = np.zeros(batch * heads * seq * head_dim if out_len is None else out_len, np.float32)
    _call("slr_causal_attention", _ptr(q), q.size, _ptr(k), k.size, _ptr(v), v.size, _ptr(cache),
          cache.size, _ptr(out), out.size, batch, layers, layer, heads, kv_heads, seq, past_len,
          head_dim, max_seq, scale_)
    return out, cache


def swiglu(x, w_gate, w_up, w_down, rows, hidden, inter, out_len=None):
    x, g, u, d = _f32(x), _f32(w_gate), _f32(w_up), _f32(w_down)
    out = np.zeros(rows * hidden if out_len is None else out_len, np.float32)
    _call("slr_swiglu", _ptr(x), x.size, _ptr(g), g.size, _ptr(u), u.size, _ptr(d), d.size,
          _ptr(out), out.size, rows, hidden, inter)
    return out


def rms_norm_matmul(x, weight, w, rows, hidden, out_features, eps, out_len=None):
    x, weight, w = _f32(x), _f32(weight), _f32(w)
    out = np.zeros(rows * out_features if out_len is None else out_len, np.float32)
    _call("slr_rms_norm_matmul", _ptr(x), x.size, _ptr(weight), weight.size, _ptr(w), w.size,
          _ptr(out), out.size, rows, hidden, out_features, eps)
    return out


# --------------------------------------------------------------------------
# Quantization convention (no reference code; parity unpinned vs sl-precision)
# --------------------------------------------------------------------------


def paged_attention_decode(q, k_new, v_new, pool, block_table, seq_lens, batch, layers, layer, num_pages,
                           page_size, pages_per_seq, heads, kv_heads, head_dim, scale):
    """Returns (out [batch, heads, head_dim] flat, the pool after the append)."""
    q, k_new, v_new = _f32(q), _f32(k_new), _f32(v_new)
    pool = np.array(pool, dtype=np.float32, copy=True)
    table = np.ascontiguousarray(block_table, dtype=np.uint32)
    lens = np.ascontiguousarray(seq_lens, dtype=np.uint32)
    out = np.zeros(batch * heads * head_dim, np.float32)
    _call("slr_paged_attention_decode", _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(pool), pool.size, _ptr(table, _U32),
          _ptr(lens, _U32), _ptr(out), batch, layers, layer, num_pages, page_size, pages_per_seq, heads, kv_heads,
          head_dim, ctypes.c_float(scale))
    return out, pool


def quantize_groupwise(w, n, k, group, bits):
    """Returns (payload uint8 [n, row_bytes], scales float32 [n, k/group])."""
    w = _f32(w)
    row_bytes = (k + 1) // 2 if bits == 4 else k
    payload = np.zeros(n * row_bytes, np.uint8)
    scales = np.zeros(n * (k // group if group else 0), np.float32)
    _call("slr_quantize_groupwise", _ptr(w), n, k, group, bits, _ptr(payload, _U8), _ptr(scales))
    return payload.reshape(n, row_bytes), scales.reshape(n, -1)


def unpack_codes(payload, n, k, bits):
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    codes = np.zeros(n * k, np.int8)
    _call("slr_unpack_codes", _ptr(payload, _U8), n, k, bits, _ptr(codes, _I8))
    return codes.reshape(n, k)


def dequantize_groupwise(payload, scales, n, k, group, bits):
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    scales = _f32(scales)
    out = np.zeros(n * k, np.float32)
    _call("slr_dequantize_groupwise", _ptr(payload, _U8), _ptr(scales), n, k, group, bits, _ptr(out))
    return out.reshape(n, k)


# --------------------------------------------------------------------------
# Test-support LCG (reference/mod.rs:118-148)
# --------------------------------------------------------------------------


class Lcg:
    """The reference's deterministic test generator, run through the C restatement."""

    def __init__(self, seed: int):
        self.state = ctypes.c_uint64(seed)

    def next_u32(self) -> int:
        return int(lib().slr_lcg_next_u32(ctypes.byref(self.state)))

    def fill(self, n: int, low: float, high: float) -> np.ndarray:
        out = np.zeros(n, np.float32)
        lib().slr_lcg_fill(ctypes.byref(self.state), _ptr(out), n, low, high)
        return out

    def below(self, upper: int) -> int:
        assert upper > 0, "upper bound must be nonzero"
        return int(lib().slr_lcg_below(ctypes.byref(self.state), upper))
