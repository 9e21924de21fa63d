"""The backend-hip crate's FFI (starlight_amd/backend-hip/src/ffi.rs) against
include/starlight_hip.h, without a Rust toolchain:

 * every #[repr(C)] struct has the header struct's fields in the same order,
   and C layout rules applied to the Rust field types give the offsets and
   size gcc computes for the header struct (offsetof / sizeof);
 * every function the header declares has an extern "C" declaration with the
   same parameter count, and nothing else is declared;
 * every enum value and #define the Rust side restates has the header's value.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FFI = os.path.join(ROOT, "starlight_amd", "backend-hip", "src", "ffi.rs")
HEADER = os.path.join(ROOT, "include", "starlight_hip.h")

SCALARS = {"u32": 4, "i32": 4, "f32": 4, "c_int": 4, "u64": 8, "usize": 8, "u8": 1}


def rust_source():
    return open(FFI).read()


def rust_consts(src):
    consts = {}
    for name, expr in re.findall(r"pub const (\w+): [\w:]+ = ([^;]+);", src):
        consts[name] = int(eval(expr, {}, consts))  # literals, shifts and earlier constants only
    return consts


def rust_structs(src):
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct (\w+) \{(.*?)\n\}", src,
                                 re.S):
        fields = re.findall(r"(?:pub )?(\w+): ([^,]+),", body)
        out[name] = [(f, t.strip()) for f, t in fields]
    return out


def size_align(ty, consts):
    if ty.startswith("*"):
        return 8, 8
    m = re.fullmatch(r"\[(\w+); (\w+)\]", ty)
    if m:
        s, a = size_align(m.group(1), consts)
        n = int(m.group(2)) if m.group(2).isdigit() else consts[m.group(2)]
        return s * n, a
    return SCALARS[ty], SCALARS[ty]


def c_layout(fields, consts):
    off, align, offsets = 0, 1, []
    for _, ty in fields:
        s, a = size_align(ty, consts)
        off = (off + a - 1) // a * a
        offsets.append(off)
        off += s
        align = max(align, a)
    return offsets, (off + align - 1) // align * align


@pytest.fixture(scope="module")
def header_layouts(tmp_path_factory):
    """offsetof / sizeof of every header struct the FFI restates, from gcc."""
    structs = {k: v for k, v in rust_structs(rust_source()).items() if k != "sl_hip_device"}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "starlight_hip.h"', "int main(void) {"]
    for name, fields in structs.items():
        lines.append(f'printf("{name} size %zu\\n", sizeof({name}));')
        for f, _ in fields:
            lines.append(f'printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines.append("return 0; }")
    d = tmp_path_factory.mktemp("layout")
    c = d / "layout.c"
    c.write_text("\n".join(lines))
    exe = d / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(c), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        name, field, value = line.split()
        got[(name, field)] = int(value)
    return structs, got


def test_repr_c_structs_match_the_header_layout(header_layouts):
    structs, got = header_layouts
    consts = rust_consts(rust_source())
    assert {"sl_error", "sl_value", "sl_op", "sl_buffer_ref", "sl_buffer_desc", "sl_capabilities",
            "sl_hip_stats"} <= set(structs)
    for name, fields in structs.items():
        offsets, size = c_layout(fields, consts)
        assert size == got[(name, "size")], name
        for (field, _), off in zip(fields, offsets):
            assert off == got[(name, field)], (name, field)


def test_header_structs_have_no_fields_the_ffi_misses():
    """The Rust structs list every field of the header structs, in order."""
    text = open(HEADER).read()
    structs = rust_structs(rust_source())
    for name, fields in structs.items():
        if name == "sl_hip_device":
            continue
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        c_fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            names = decl.split(None, 1)[1] if not decl.startswith("const") else decl.split(None, 2)[2]
            for part in names.split(","):
                c_fields.append(re.sub(r"[\s*]|\[.*\]", "", part))
        assert [f for f, _ in fields] == c_fields, name


def declared_functions(text, pattern):
    out = {}
    for name, params in re.findall(pattern, text, re.S):
        params = params.strip().rstrip(",").strip()  # a trailing comma (rustfmt) is no parameter
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_every_header_function_is_declared_with_its_arity():
    header = declared_functions(re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S),
                                r"\b(sl_hip_\w+)\s*\(([^;{]*?)\)\s*;")
    rust = declared_functions(rust_source(), r"pub fn (sl_hip_\w+)\(([^)]*)\)")
    assert header == rust


def test_restated_constants_match_the_header():
    text = open(HEADER).read()
    header = {k: int(v) for k, v in re.findall(r"\b(SL_[A-Z0-9_]+) = (\d+)", text)}
    defines = {}
    for k, a, b in re.findall(r"#define (SL_[A-Z0-9_]+) \(?(\d+)u?(?: << (\d+)\))?", text):
        defines[k] = int(a) << (int(b) if b else 0)
    consts = rust_consts(rust_source())
    checked = 0
    for k, v in consts.items():
        if k in header:
            assert v == header[k], k
            checked += 1
        elif k in defines:
            assert v == defines[k], k
            checked += 1
    assert checked >= 50
