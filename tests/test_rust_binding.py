"""The Rust binding include/voxhip.rs against the C header include/voxhip.h.

The binding is generated from the header by render_rust() below; after a header
change, regenerate it with

    python tests/test_rust_binding.py --write

and test_binding_is_the_rendered_header checks that the committed file is that
output.

The reference engine is Rust (src/baselm.rs, src/local.rs, src/acoustic.rs call
the Vulkan layer in src/vulkan.rs); a maintainer swaps that layer for these
extern "C" declarations. No Rust toolchain exists here, so the binding is checked
structurally instead: every function of the header is declared with the same
parameter count and the Rust spelling of each C type, every #[repr(C)] struct
has the header's fields in the header's order with the same types and array
lengths, and the status codes and #define constants carry the header's values.
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "voxhip.h"
RUST = ROOT / "include" / "voxhip.rs"

SCALARS = {
    "void": "c_void", "char": "c_char", "int": "c_int", "float": "f32", "double": "f64",
    "uint8_t": "u8", "uint16_t": "u16", "uint32_t": "u32", "uint64_t": "u64",
    "int8_t": "i8", "int16_t": "i16", "int32_t": "i32", "int64_t": "i64", "size_t": "usize",
}


def _strip(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return "\n".join(l for l in text.splitlines() if not l.strip().startswith("#"))


def rust_name(c: str) -> str:
    """vx_baselm_config -> VxBaselmConfig."""
    return "".join(p[:1].upper() + p[1:] for p in c.split("_"))


def rust_type(base: str, const: bool, ptr: int, enums: set[str]) -> str:
    """Rust spelling of a C type: base name, const qualifier of the pointee, pointer depth."""
    base = base.strip()
    if base in enums:
        t = "c_int"
    elif base in SCALARS:
        t = SCALARS[base]
    elif base.startswith("vx_"):
        t = rust_name(base)
    else:
        raise ValueError(f"no Rust spelling for C type {base!r}")
    for level in range(ptr):
        qual = "*const " if (const and level == 0) else "*mut "
        t = qual + t
    return t


def _decl(decl: str):
    """'const vx_buf *x' -> (name, base, const, ptr, array)."""
    decl = " ".join(decl.split())
    const = decl.startswith("const ")
    if const:
        decl = decl[len("const "):]
    m = re.match(r"(unsigned\s+\w+|\w+)\s*(\**)\s*(\w+)?\s*(?:\[(\w+)\])?$", decl)
    if not m:
        raise ValueError(f"cannot parse declaration {decl!r}")
    return m.group(3), m.group(1), const, len(m.group(2)), m.group(4)


def parse_header(text: str):
    """Functions, structs, enum constants and #define constants of voxhip.h."""
    defines = {}
    for m in re.finditer(r"^#define\s+(VX_\w+)\s+(.+?)\s*(?:/\*.*)?$", text, flags=re.M):
        defines[m.group(1)] = m.group(2).strip()
    s = _strip(text)
    enums, enum_values = set(), {}
    for m in re.finditer(r"typedef\s+enum\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", s, flags=re.S):
        enums.add(m.group(3))
        for item in m.group(2).split(","):
            if item.strip():
                k, v = item.split("=")
                enum_values[k.strip()] = int(v.strip())
    structs = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", s, flags=re.S):
        fields = []
        for decl in m.group(2).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            head = re.match(r"((?:const\s+)?(?:unsigned\s+)?\w+)\s+(.*)$", decl)
            base, rest = head.group(1), head.group(2)
            for d in rest.split(","):
                name, b, const, ptr, arr = _decl(f"{base} {d.strip()}")
                fields.append((name, b, const, ptr, arr))
        structs[m.group(3)] = fields
    opaque = set(re.findall(r"typedef\s+struct\s+(\w+)\s+\1\s*;", s))
    body = re.sub(r"typedef\s+(?:struct|enum)\s+\w+\s*\{.*?\}\s*\w+\s*;", " ", s, flags=re.S)
    body = re.sub(r"typedef\s+struct\s+\w+\s+\w+\s*;", " ", body)
    body = body.replace('extern "C" {', " ")
    funcs = {}
    for m in re.finditer(r"((?:const\s+)?\w+)\s*(\**)\s*\b(vx_\w+)\s*\(([^)]*)\)\s*;", body):
        ret_base, ret_ptr, name, args = m.group(1), len(m.group(2)), m.group(3), m.group(4)
        ret_const = ret_base.startswith("const ")
        params = []
        if args.strip() != "void":
            for a in args.split(","):
                params.append(_decl(a))
        funcs[name] = (ret_base.replace("const ", ""), ret_const, ret_ptr, params)
    return funcs, structs, enums, enum_values, opaque, defines


def parse_rust(text: str):
    """extern fns, #[repr(C)] structs and constants of voxhip.rs."""
    text = re.sub(r"//[^\n]*", "", text)
    funcs = {}
    for m in re.finditer(r"pub\s+fn\s+(vx_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", text, flags=re.S):
        params = []
        for p in m.group(2).split(","):
            p = " ".join(p.split())
            if p:
                name, ty = p.split(":", 1)
                params.append((name.strip(), ty.strip()))
        funcs[m.group(1)] = (params, (m.group(3) or "()").strip())
    structs = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub\s+struct\s+(\w+)\s*\{(.*?)\}", text,
                         flags=re.S):
        fields = []
        for f in m.group(2).split(","):
            f = " ".join(f.split())
            if f:
                name, ty = f.split(":", 1)
                fields.append((name.replace("pub ", "").strip(), ty.strip()))
        structs[m.group(1)] = fields
    consts = {m.group(1): (m.group(2).strip(), m.group(3).strip())
              for m in re.finditer(r"pub\s+const\s+(VX_\w+)\s*:\s*(\w+)\s*=\s*([^;]+);", text)}
    return funcs, structs, consts


def c_value(v: str, defines: dict) -> int:
    v = v.strip()
    v = re.sub(r"\b(VX_\w+)\b", lambda m: f"({c_value(defines[m.group(1)], defines)})", v)
    return int(eval(re.sub(r"(\d+)[uU]\b", r"\1", v), {"__builtins__": {}}))


def rust_value(v: str) -> int:
    return int(eval(v.replace("_", ""), {"__builtins__": {}}))


@pytest.fixture(scope="module")
def both():
    return parse_header(HEADER.read_text()), parse_rust(RUST.read_text())


def test_every_function_is_declared_with_matching_types(both):
    (hf, _, enums, _, _, _), (rf, _, _) = both
    assert len(hf) >= 130
    assert set(hf) == set(rf), (sorted(set(hf) - set(rf)), sorted(set(rf) - set(hf)))
    for name, (ret_base, ret_const, ret_ptr, params) in hf.items():
        rparams, rret = rf[name]
        assert len(params) == len(rparams), name
        for (pname, base, const, ptr, arr), (_, rty) in zip(params, rparams):
            assert arr is None, (name, pname)
            assert rty == rust_type(base, const, ptr, enums), (name, pname, rty)
        want_ret = "()" if (ret_base == "void" and ret_ptr == 0) else rust_type(ret_base, ret_const, ret_ptr, enums)
        assert rret == want_ret, (name, rret, want_ret)


def test_every_struct_has_the_header_layout(both):
    (_, hs, enums, _, opaque, defines), (_, rs, _) = both
    assert len(hs) >= 40
    for cname, fields in hs.items():
        rname = rust_name(cname)
        assert rname in rs, rname
        rfields = rs[rname]
        assert [f[0] for f in fields] == [f[0] for f in rfields], rname
        for (fname, base, const, ptr, arr), (_, rty) in zip(fields, rfields):
            t = rust_type(base, const, ptr, enums)
            if arr is not None:
                n = c_value(arr, defines) if not arr.isdigit() else int(arr)
                t = f"[{t}; {n}]"
            assert rty == t, (rname, fname, rty, t)
    for cname in opaque:
        assert re.search(rf"pub\s+struct\s+{rust_name(cname)}\s*\{{\s*_p:\s*\[u8;\s*0\]", RUST.read_text()), cname


def test_status_codes_and_constants_carry_the_header_values(both):
    (_, _, _, enum_values, _, defines), (_, _, consts) = both
    for k, v in enum_values.items():
        assert k in consts and rust_value(consts[k][1]) == v, k
    for k, v in defines.items():
        if k in ("VOXHIP_H",):
            continue
        assert k in consts, k
        assert rust_value(consts[k][1]) == c_value(v, defines), k


# ------------------------------------------------------------ the generator
RUST_KEYWORDS = {
    "type", "ref", "in", "match", "move", "fn", "loop", "use", "mod", "impl", "self", "box", "where", "async",
    "await", "dyn", "final", "override", "priv", "pub", "static", "struct", "trait", "true", "false", "unsafe",
    "virtual", "yield", "crate", "super", "const", "enum", "extern", "let", "mut", "return", "while", "for", "if",
    "else", "break", "continue", "as", "macro", "abstract", "become", "do", "typeof", "unsized", "try",
}

RUST_PREAMBLE = """// voxhip.rs: Rust declarations of the C ABI in voxhip.h (libvoxhip.so).
//
// The drop-in for VoxGen's Vulkan layer (src/vulkan.rs) on the BaseLM compute
// path: src/hip.rs of the reference crate can be this file. Every function and
// struct of voxhip.h appears here in the header's order, with the same parameter
// types and #[repr(C)] field layout. Generated from the header by
// `python tests/test_rust_binding.py --write`; do not edit by hand. Status codes
// are c_int (VX_OK = 0, negative = error; the message is vx_last_error()). Link
// with build.rs:
//     println!("cargo:rustc-link-lib=dylib=voxhip");
//     println!("cargo:rustc-link-search=native=<dir of libvoxhip.so>");
#![allow(non_camel_case_types, non_upper_case_globals, dead_code)]

use std::os::raw::{c_char, c_int, c_void};
"""


def _rid(n: str) -> str:
    return f"r#{n}" if n in RUST_KEYWORDS else n


def render_rust(text: str) -> str:
    """include/voxhip.rs for the header text: status codes, #define constants,
    opaque handles, then structs and functions in the header's order."""
    funcs, structs, enums, enum_values, opaque, defines = parse_header(text)
    s = _strip(text)
    items = []
    for m in re.finditer(r"typedef\s+struct\s+\w+\s*\{.*?\}\s*(\w+)\s*;", s, flags=re.S):
        items.append((m.start(), m.group(1)))
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s+\1\s*;", s):
        items.append((m.start(), m.group(1)))
    body = re.sub(r"typedef\s+(?:struct|enum)\s+\w+\s*\{.*?\}\s*\w+\s*;", lambda m: " " * len(m.group(0)), s,
                  flags=re.S)
    for m in re.finditer(r"\b(vx_\w+)\s*\(", body):
        items.append((m.start(), m.group(1)))
    order = [n for _, n in sorted(items)]
    out = [RUST_PREAMBLE, "// Status codes (vx_status).", "pub type VxStatus = c_int;"]
    out += [f"pub const {k}: c_int = {v};" for k, v in enum_values.items()]
    out += ["", "// Constants (#define)."]
    out += [f"pub const {k}: u32 = {c_value(v, defines)};" for k, v in defines.items()]
    out += ["", "// Opaque handles."]
    out += [f"#[repr(C)] pub struct {rust_name(n)} {{ _p: [u8; 0] }}" for n in order if n in opaque]
    out.append("")
    emitted, pending = set(), []

    def flush():
        if pending:
            out.extend(['#[link(name = "voxhip")]', 'extern "C" {', *pending, "}", ""])
            pending.clear()

    for n in order:
        if n in structs and n not in emitted:
            flush()
            emitted.add(n)
            out += ["#[repr(C)]", "#[derive(Clone, Copy)]", f"pub struct {rust_name(n)} {{"]
            for (fname, base, const, ptr, arr) in structs[n]:
                ty = rust_type(base, const, ptr, enums)
                if arr is not None:
                    ty = f"[{ty}; {c_value(arr, defines) if not arr.isdigit() else int(arr)}]"
                out.append(f"    pub {_rid(fname)}: {ty},")
            out += ["}", ""]
        elif n in funcs and n not in emitted:
            emitted.add(n)
            ret_base, ret_const, ret_ptr, params = funcs[n]
            ps = [f"{_rid(pname)}: {rust_type(base, const, ptr, enums)}" for (pname, base, const, ptr, _) in params]
            ret = "" if (ret_base == "void" and ret_ptr == 0) else " -> " + rust_type(ret_base, ret_const, ret_ptr,
                                                                                       enums)
            line = f"    pub fn {n}({', '.join(ps)}){ret};"
            if len(line) > 110:
                line = f"    pub fn {n}(\n        " + ",\n        ".join(ps) + f",\n    ){ret};"
            pending.append(line)
    flush()
    missing = (set(funcs) | set(structs)) - emitted
    assert not missing, missing
    return "\n".join(out).rstrip() + "\n"


def test_binding_is_the_rendered_header():
    assert RUST.read_text() == render_rust(HEADER.read_text()), \
        "include/voxhip.rs is stale: run python tests/test_rust_binding.py --write"


if __name__ == "__main__":
    if sys.argv[1:] != ["--write"]:
        sys.exit("usage: python tests/test_rust_binding.py --write")
    RUST.write_text(render_rust(HEADER.read_text()))
    print(f"wrote {RUST}")
