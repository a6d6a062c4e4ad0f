"""Writes rnn-sys/src/lib.rs, the Rust FFI declarations of include/rnn.h.

    python rnn-sys/gen_bindings.py

The header is the single source: its enum and #define constants, opaque
handles, #[repr(C)] structs and every prototype become Rust declarations with
the C types mapped one to one (int -> c_int, size_t -> usize, uint32_t -> u32,
float -> f32, T * -> *mut T, const T * -> *const T).  tests/test_rnn_sys.py
parses the committed lib.rs on its own and diffs it against the header.
"""
from __future__ import annotations

import os
import re
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rnn.h")
OUT = os.path.join(ROOT, "rnn-sys", "src", "lib.rs")

SCALARS = {"int": "c_int", "unsigned": "u32", "uint32_t": "u32", "int32_t": "i32",
           "uint64_t": "u64", "int64_t": "i64", "size_t": "usize", "float": "f32",
           "double": "f64", "char": "c_char", "void": "c_void"}


def strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def parse_header(path=HEADER):
    """(consts, opaque, structs, funcs) of the header:
    consts [(name, value, ctype)], opaque [name], structs {name: [(field,
    ctype)]}, funcs [(name, ret ctype, [(param, ctype)])]."""
    raw = open(path).read()
    text = strip_comments(raw)
    consts = []
    for m in re.finditer(r"enum\s*\{(.*?)\}\s*;", text, re.S):
        for item in m.group(1).split(","):
            item = item.strip()
            if item:
                name, val = [x.strip() for x in item.split("=")]
                consts.append((name, int(val), "int"))
    for m in re.finditer(r"^#define\s+(RNN_\w+)\s+(\(?[^\n]+)$", raw, re.M):
        name, val = m.group(1), m.group(2).strip()
        if name == "RNN_H":
            continue
        mu = re.fullmatch(r"(\d+)u", val)
        if mu:
            consts.append((name, int(mu.group(1)), "uint32_t"))
            continue
        ms = re.fullmatch(r"\(\(size_t\)(\d+)\s*<<\s*(\d+)\)", val)
        if ms:
            consts.append((name, int(ms.group(1)) << int(ms.group(2)), "size_t"))
            continue
        raise ValueError(f"unparsed #define {name} {val}")
    opaque = re.findall(r"typedef\s+struct\s+(\w+)\s+\1\s*;", text)
    structs = {}
    for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", text, re.S):
        fields = []
        for decl in m.group(1).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            base, names = split_decl_list(decl)
            for nm in names:
                stars = len(nm) - len(nm.lstrip("*"))
                fields.append((nm.lstrip("*"), base + " " + "*" * stars if stars else base))
        structs[m.group(2)] = [(f, norm(t)) for f, t in fields]
    funcs = []
    body = re.sub(r"^\s*#[^\n]*$", " ", text, flags=re.M)   # preprocessor lines
    body = body.replace('extern "C" {', " ")
    body = re.sub(r"typedef[^;]*;", " ", body)
    body = re.sub(r"enum\s*\{.*?\}\s*;", " ", body, flags=re.S)
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(rnn_\w+)\s*\(([^;{]*?)\)\s*;", body, re.S):
        ret, name, params = norm(m.group(1)), m.group(2), " ".join(m.group(3).split())
        plist = []
        if params and params != "void":
            for p in params.split(","):
                p = p.strip()
                pm = re.fullmatch(r"(.*?)(\w+)", p)
                plist.append((pm.group(2), norm(pm.group(1))))
        funcs.append((name, ret, plist))
    return consts, opaque, structs, funcs


def split_decl_list(decl):
    """'const uint32_t *relidx' -> ('const uint32_t', ['*relidx']);
    'float *v, *g' -> ('float', ['*v', '*g'])."""
    first, *rest = [x.strip() for x in decl.split(",")]
    m = re.fullmatch(r"(.*?)(\**\s*\w+)", first)
    base = m.group(1).strip()
    names = [m.group(2).replace(" ", "")] + [r.replace(" ", "") for r in rest]
    return base, names


def norm(ctype):
    """Canonical spelling: 'const float *', 'rnn_ctx **', 'size_t'."""
    t = " ".join(ctype.replace("*", " * ").split())
    return t.replace("* *", "**").replace(" *", " *").strip()


def rust_type(ctype):
    t = norm(ctype)
    stars = t.count("*")
    base = t.replace("*", "").strip()
    const = base.startswith("const ")
    base = base[6:] if const else base
    r = SCALARS.get(base, base)
    if stars == 0:
        return "()" if r == "c_void" else r
    ptr = ("*const " if const else "*mut ") + r
    for _ in range(stars - 1):
        ptr = "*mut " + ptr
    return ptr


def render():
    consts, opaque, structs, funcs = parse_header()
    out = ["// Generated from include/rnn.h by rnn-sys/gen_bindings.py; do not edit.",
           "// The C ABI of librnn.so (the MI355X GEMM core of rustnn).",
           "#![allow(non_camel_case_types)]",
           "use std::os::raw::{c_char, c_int, c_void};", ""]
    for name, val, ctype in consts:
        out.append(f"pub const {name}: {rust_type(ctype)} = {val};")
    out.append("")
    for name in opaque:
        out.append(f"#[repr(C)] pub struct {name} {{ _p: [u8; 0] }}")
    out.append("")
    for name, fields in structs.items():
        out.append("#[repr(C)] #[derive(Clone, Copy)]")
        out.append(f"pub struct {name} {{")
        for f, t in fields:
            out.append(f"    pub {f}: {rust_type(t)},")
        out.append("}")
        out.append("")
    out.append('#[link(name = "rnn")]')
    out.append('extern "C" {')
    for name, ret, params in funcs:
        args = ", ".join(f"{p}: {rust_type(t)}" for p, t in params)
        r = rust_type(ret)
        tail = "" if r == "()" else f" -> {r}"
        out.append(f"    pub fn {name}({args}){tail};")
    out.append("}")
    out.append("")
    out.append("// Hand-written safe layer (src/safe.rs): the reference's call-site")
    out.append("// signatures over the *_host entry points.")
    out.append("pub mod safe;")
    return "\n".join(out) + "\n"


if __name__ == "__main__":
    text = render()
    if "--check" in sys.argv:
        sys.exit(0 if open(OUT).read() == text else 1)
    open(OUT, "w").write(text)
    print(f"wrote {OUT}")
