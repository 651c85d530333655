"""The reference-side Rust binding (crates/qx-hip) against include/qx_hip.h.

The crate is what a qx maintainer adds beside crates/qx-metal; this image has
no Rust toolchain, so it is checked here by parsing: every header function is
declared in src/ffi.rs with the same name and the Rust counterpart of each
parameter type, every header struct has the same fields in the same order,
the constants agree, and src/lib.rs offers the qx-metal encoder methods the
attention call sites use, with the reference's parameter names
(crates/qx-metal/src/lib.rs:1918-2096, :7959-8382, :9404-9514, :9819-9999,
:14373-14599).
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qx_hip.h")
CRATE = os.path.join(ROOT, "crates", "qx-hip")

C_SCALARS = {"int32_t": "i32", "uint32_t": "u32", "uint64_t": "u64", "size_t": "usize", "float": "f32",
             "double": "f64", "uint16_t": "u16", "uint8_t": "u8", "char": "c_char", "void": "c_void"}


def rust_name(c_type_name):
    return "".join(part.capitalize() for part in c_type_name.split("_"))


def rust_type(c_type):
    """The Rust spelling of a C parameter or field type."""
    t = " ".join(c_type.split())
    const = t.startswith("const ")
    if const:
        t = t[len("const "):]
    stars = t.count("*")
    base = t.replace("*", "").strip()
    r = C_SCALARS.get(base, rust_name(base) if base.startswith("qxh_") else None)
    assert r is not None, f"no Rust mapping for C type {c_type!r}"
    if stars == 0:
        return r
    r = ("*const " if const else "*mut ") + r
    for _ in range(stars - 1):
        r = "*mut " + r
    return r


def strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def header_functions():
    body = strip_c_comments(open(HEADER).read())
    out = {}
    for ret, name, params in re.findall(r"QXH_API\s+(\w+)\s+(qxh_\w+)\s*\(([^;]*?)\)\s*;", body, flags=re.S):
        ps = [p.strip() for p in " ".join(params.split()).split(",") if p.strip() and p.strip() != "void"]
        args = []
        for p in ps:
            m = re.match(r"(.*?)(\w+)$", p)
            args.append((m.group(2), rust_type(m.group(1))))
        out[name] = (rust_type(ret), args)
    return out


def header_structs():
    body = strip_c_comments(open(HEADER).read())
    out = {}
    for fields, name in re.findall(r"typedef struct\s*\{(.*?)\}\s*(qxh_\w+)\s*;", body, flags=re.S):
        fs = []
        for f in [x.strip() for x in fields.split(";") if x.strip()]:
            m = re.match(r"(.*?)(\w+)$", " ".join(f.split()))
            fs.append((m.group(2), rust_type(m.group(1))))
        out[rust_name(name)] = fs
    return out


def rust_source(name):
    text = open(os.path.join(CRATE, "src", name)).read()
    return re.sub(r"//[^\n]*", "", text)


def ffi_functions():
    src = rust_source("ffi.rs")
    block = src[src.index('extern "C"'):]
    out = {}
    for name, params, ret in re.findall(r"pub fn (qxh_\w+)\s*\((.*?)\)\s*->\s*([^;]+);", block, flags=re.S):
        args = []
        for p in [x.strip() for x in " ".join(params.split()).split(",") if x.strip()]:
            n, t = p.split(":", 1)
            args.append((n.strip(), " ".join(t.split())))
        out[name] = (ret.strip(), args)
    return out


def ffi_structs():
    src = rust_source("ffi.rs")
    out = {}
    for name, fields in re.findall(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct (\w+)\s*\{(.*?)\}", src,
                                   flags=re.S):
        fs = []
        for f in [x.strip() for x in fields.split(",") if x.strip()]:
            n, t = f.split(":", 1)
            fs.append((n.replace("pub", "").strip(), " ".join(t.split())))
        out[name] = fs
    return out


def test_every_header_function_is_bound_with_the_same_types():
    h, r = header_functions(), ffi_functions()
    assert len(h) >= 58
    assert sorted(h) == sorted(r), (sorted(set(h) ^ set(r)))
    for name, (ret, args) in h.items():
        rret, rargs = r[name]
        assert rret == ret, (name, rret, ret)
        assert [t for _, t in rargs] == [t for _, t in args], (name, rargs, args)
        assert [n for n, _ in rargs] == [n for n, _ in args], (name, rargs, args)


def test_every_header_struct_has_the_same_fields():
    h, r = header_structs(), ffi_structs()
    for name, fields in h.items():
        assert name in r, name
        assert r[name] == fields, (name, r[name], fields)
    body = strip_c_comments(open(HEADER).read())
    for opaque in re.findall(r"typedef struct (qxh_\w+) qxh_\w+;", body):
        assert r.get(rust_name(opaque)) == [("_private", "[u8; 0]")], opaque


def test_constants_agree():
    body = strip_c_comments(open(HEADER).read())
    src = rust_source("ffi.rs")
    consts = dict(re.findall(r"pub const (QXH_\w+): i32 = (\d+);", src))
    for name, value in re.findall(r"(QXH_\w+)\s*=\s*(\d+)", body):
        assert consts.get(name) == value, name
    assert consts["QXH_ABI_VERSION"] == re.search(r"#define QXH_ABI_VERSION (\d+)", body).group(1)


# qx-metal methods of this path and their parameter names after `&mut self` /
# `&self` (crates/qx-metal/src/lib.rs line ranges in the module docstring)
REFERENCE_METHODS = {
    "encode_rope_kv_for_layer": ["context", "query", "key", "value", "query_output", "key_cache", "value_cache",
                                 "layer", "position"],
    "encode_rope_kv_batch": ["context", "query", "key", "value", "query_output", "key_cache", "value_cache",
                             "start_position", "tokens"],
    "encode_attention_batch_with_plan": ["context", "query", "key_cache", "value_cache", "output", "start_position",
                                         "tokens", "use_batch_simd"],
    "encode_attention": ["context", "query", "key_cache", "value_cache", "output", "length"],
    "encode_attention_three_stage_for_layer": ["context", "query", "key_cache", "value_cache", "scores", "output",
                                               "layer", "length"],
    "encode_qwen_qk_norm_rope": ["context", "query", "key", "query_norm", "key_norm", "position"],
    "encode_qwen_store_kv": ["context", "key", "value", "key_cache", "value_cache", "position"],
    "encode_qwen_gqa_attention": ["context", "query", "key_cache", "value_cache", "output", "context_len"],
    "run_qwen_qk_norm_rope": ["query", "key", "query_norm", "key_norm", "position"],
    "run_qwen_gqa_attention": ["query", "key_cache", "value_cache"],
    "allocate_runtime_buffer": ["length"],
    "write_runtime_buffer": ["buffer", "bytes"],
    "read_runtime_u32": ["buffer"],
    "read_runtime_f32": ["buffer", "elements"],
    "read_runtime_f16": ["buffer", "elements"],
    "begin_decode": [],
    "finish": ["context"],
    "wait": ["context"],
}


@pytest.mark.parametrize("method", sorted(REFERENCE_METHODS))
def test_shim_keeps_the_reference_method_signatures(method):
    src = rust_source("lib.rs")
    m = re.search(r"pub fn " + method + r"\s*\((.*?)\)\s*->", src, flags=re.S)
    assert m, method
    params = [p.strip() for p in " ".join(m.group(1).split()).split(",") if p.strip()]
    assert params and params[0] in ("&self", "&mut self", "self"), (method, params)
    names = [p.split(":")[0].strip().lstrip("_") for p in params[1:]]
    assert names == REFERENCE_METHODS[method], (method, names)


def test_shim_calls_only_declared_functions():
    declared = set(ffi_functions())
    called = set(re.findall(r"ffi::(qxh_\w+)\(", rust_source("lib.rs")))
    assert called and called <= declared, called - declared


def test_only_the_context_owner_holds_the_raw_context():
    """Arenas, graphs and submitted graphs keep the context alive through the
    Rc of its owner, so safe code cannot destroy a context that a cache or a
    graph still reads (qxh_kv_cache_destroy and qxh_graph_wait use it)."""
    src = rust_source("lib.rs")
    structs = dict(re.findall(r"pub struct (\w+)\s*\{(.*?)\n\}", src, flags=re.S))
    raw_holders = [name for name, body in structs.items() if "*mut ffi::QxhContext" in body]
    assert raw_holders == ["ContextInner"], raw_holders
    for name in ("HipContext", "ArenaInner", "DecodeGraph", "SubmittedDecode"):
        assert "Rc<ContextInner>" in structs[name], name
    assert "qxh_context_destroy" in src.split("impl Drop for ContextInner")[1].split("\n}\n")[0]
