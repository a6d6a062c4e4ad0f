"""The Rust FFI crate (rnn-sys/) against include/rnn.h and librnn.so, on the
CPU (cargo is not in this image, so the crate is checked as text): every
prototype, struct and constant of the header appears in src/lib.rs with the
mapped Rust types, nothing else does, and the library exports every
declared function."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "rnn-sys"))
import gen_bindings as gb  # noqa: E402

LIB_RS = os.path.join(ROOT, "rnn-sys", "src", "lib.rs")

# C spelling -> Rust spelling, written out here rather than taken from the
# generator, so a wrong mapping there fails this test
C2RUST = {"int": "c_int", "uint32_t": "u32", "uint64_t": "u64", "size_t": "usize",
          "float": "f32", "double": "f64", "void": "c_void", "char": "c_char"}


def expect(ctype):
    t = " ".join(ctype.replace("*", " * ").split())
    stars = t.count("*")
    base = t.replace("*", "").strip()
    const = base.startswith("const ")
    base = base[len("const "):] if const else base
    r = C2RUST.get(base, base)
    if stars == 0:
        return "()" if r == "c_void" else r
    out = ("*const " if const else "*mut ") + r
    return "*mut " * (stars - 1) + out


def parse_lib_rs():
    text = open(LIB_RS).read()
    fns = {}
    for m in re.finditer(r"pub fn (\w+)\(([^)]*)\)(?:\s*->\s*([^;]+))?;", text):
        args = [a.strip() for a in m.group(2).split(",") if a.strip()]
        fns[m.group(1)] = ([tuple(x.strip() for x in a.split(":", 1)) for a in args],
                           (m.group(3) or "()").strip())
    structs = {}
    for m in re.finditer(r"pub struct (\w+) \{\n(.*?)\n\}", text, re.S):
        structs[m.group(1)] = [tuple(x.strip().rstrip(",").replace("pub ", "", 1).split(": ", 1))
                               for x in m.group(2).splitlines()]
    opaque = re.findall(r"pub struct (\w+) \{ _p: \[u8; 0\] \}", text)
    consts = {m.group(1): (m.group(2), int(m.group(3)))
              for m in re.finditer(r"pub const (\w+): (\w+) = (-?\d+);", text)}
    return fns, structs, opaque, consts, text


def test_functions_match_header():
    _, _, _, funcs = gb.parse_header()
    fns, _, _, _, _ = parse_lib_rs()
    assert len(funcs) > 100
    assert sorted(f[0] for f in funcs) == sorted(fns)
    for name, ret, params in funcs:
        args, rret = fns[name]
        assert [a[0] for a in args] == [p for p, _ in params], name
        assert [a[1] for a in args] == [expect(t) for _, t in params], name
        assert rret == expect(ret), name


def test_structs_and_constants_match_header():
    consts, opaque, structs, _ = gb.parse_header()
    _, rstructs, ropaque, rconsts, _ = parse_lib_rs()
    assert sorted(opaque) == sorted(ropaque) == ["rnn_conv_packs", "rnn_ctx", "rnn_optim",
                                                 "rnn_resnet"]
    assert sorted(structs) == sorted(rstructs)
    for name, fields in structs.items():
        assert rstructs[name] == [(f, expect(t)) for f, t in fields], name
    assert {n: v for n, v, _ in consts} == {n: v for n, (_, v) in rconsts.items()}
    assert rconsts["RNN_OK"] == ("c_int", 0) and rconsts["RNN_ATTN_SET_DKV"] == ("u32", 2)


def test_header_parse_sees_known_layouts():
    """The parser itself, on declarations whose layout is known."""
    _, _, structs, funcs = gb.parse_header()
    assert structs["rnn_attn_desc"][:4] == [("h", "uint32_t"), ("dh", "uint32_t"),
                                            ("tq", "uint32_t"), ("tk", "uint32_t")]
    assert ("relidx", "const uint32_t *") in structs["rnn_attn_desc"]
    assert [f for f, _ in structs["rnn_param"]] == ["v", "g", "m", "v2", "len", "rows",
                                                    "cols", "decay"]
    f = {n: (r, p) for n, r, p in funcs}
    assert f["rnn_ctx_create"] == ("int", [("device", "int"), ("out", "rnn_ctx **")])
    assert f["rnn_ctx_last_error"][0] == "const char *"


def test_lib_rs_is_current():
    assert open(LIB_RS).read() == gb.render(), "run python rnn-sys/gen_bindings.py"


def test_library_exports_every_declared_function():
    so = os.path.join(ROOT, "rustnn_amd", "librnn.so")
    if not os.path.exists(so):
        pytest.skip("librnn.so not built")
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    fns, _, _, _, _ = parse_lib_rs()
    assert not (set(fns) - exported)


def test_build_script_links_rnn():
    b = open(os.path.join(ROOT, "rnn-sys", "build.rs")).read()
    assert "rustc-link-lib=dylib=rnn" in b
    toml = open(os.path.join(ROOT, "rnn-sys", "Cargo.toml")).read()
    assert 'name = "rnn-sys"' in toml and 'links = "rnn"' in toml


SAFE_RS = os.path.join(ROOT, "rnn-sys", "src", "safe.rs")

# The reference's call-site signatures the safe layer keeps, written out from
# the reference files (parameter name: type, in order):
#   gemm.rs:434-444 matmul, gemm.rs:500-512 gemm_small, gemm.rs:555 matmul_dw,
#   attn.rs:148-160 Core::forward, attn.rs:226-242 Core::backward.
REF_SIGS = {
    "matmul": [("m", "usize"), ("n", "usize"), ("k", "usize"), ("a", "&[f32]"), ("at", "bool"),
               ("b", "&[f32]"), ("bt", "bool"), ("c", "&mut [f32]"), ("acc", "bool")],
    "gemm_small": [("m", "usize"), ("n", "usize"), ("k", "usize"), ("a", "&[f32]"),
                   ("at", "bool"), ("b", "&[f32]"), ("bt", "bool"), ("c", "&mut [f32]"),
                   ("acc", "bool"), ("_ap", "&mut PackedA"), ("_bp", "&mut PackedB")],
    "matmul_dw": [("m", "usize"), ("n", "usize"), ("k", "usize"), ("a", "&[f32]"),
                  ("b", "&[f32]"), ("c", "&mut [f32]")],
    "forward": [("&self", None), ("q", "&[f32]"), ("qstride", "usize"), ("qoff", "usize"),
                ("kv", "&[f32]"), ("kvstride", "usize"), ("koff", "usize"), ("voff", "usize"),
                ("tau", "&[f32]"), ("rel", "&[f32]"), ("p", "&mut [f32]"), ("o", "&mut [f32]")],
    "backward": [("&self", None), ("q", "&[f32]"), ("qstride", "usize"), ("qoff", "usize"),
                 ("kv", "&[f32]"), ("kvstride", "usize"), ("koff", "usize"),
                 ("voff", "usize"), ("tau", "&[f32]"), ("p", "&[f32]"), ("dobuf", "&[f32]"),
                 ("dq", "&mut [f32]"), ("dkv", "&mut [f32]"), ("dtau", "&mut [f32]"),
                 ("drel", "&mut [f32]")],
}
# safe fn -> the *_host entry point it must call
SAFE_CALLS = {"matmul": "rnn_matmul_host", "gemm_small": "rnn_gemm_small_batched_host",
              "matmul_dw": "rnn_matmul_dw_host", "conv2d_forward": "rnn_conv2d_forward_host",
              "conv2d_backward_w": "rnn_conv2d_backward_w_host",
              "conv2d_backward_x": "rnn_conv2d_backward_x_host",
              "forward": "rnn_attn_forward_host", "backward": "rnn_attn_backward_host",
              "linear_forward": "rnn_linear_forward_host",
              "linear_backward": "rnn_linear_backward_host"}


def _safe_fns():
    """{name: (params [(name, type)], body)} of the `pub fn`s of safe.rs."""
    text = open(SAFE_RS).read()
    out = {}
    for m in re.finditer(r"pub fn (\w+)\(([^)]*)\)[^{]*\{", text):
        params = []
        for a in [x.strip() for x in m.group(2).replace("\n", " ").split(",") if x.strip()]:
            if ":" in a:
                n, t = a.split(":", 1)
                params.append((n.strip(), " ".join(t.split())))
            else:
                params.append((a, None))
        depth, i = 1, m.end()
        while depth:
            depth += {"{": 1, "}": -1}.get(text[i], 0)
            i += 1
        out.setdefault(m.group(1), (params, text[m.end():i]))
    return out, text


def test_safe_layer_keeps_reference_signatures():
    fns, text = _safe_fns()
    for name, want in REF_SIGS.items():
        assert fns[name][0] == want, name
    assert "pub struct Core {" in text and "pub relidx: Vec<u32>," in text
    assert "pub mod safe;" in open(LIB_RS).read()


def test_safe_layer_calls_host_entry_points():
    """Each safe function calls its *_host entry point (declared in lib.rs and
    exported by librnn.so) and no device-pointer entry point."""
    fns, text = _safe_fns()
    decl, _, _, _, _ = parse_lib_rs()
    for name, host in SAFE_CALLS.items():
        body = fns[name][1]
        called = set(re.findall(r"\b(rnn_\w+)\(", body))
        assert called == {host}, (name, called)
        assert host in decl
    every = set(re.findall(r"\b(rnn_\w+)\(", text))
    assert every <= set(decl)
    assert {c for c in every if not c.endswith("_host")} == {
        "rnn_ctx_create", "rnn_ctx_last_error", "rnn_status_string"}
