"""The Rust binding (crates/attn-hip-ffi, source only: no Rust toolchain here) against the C
header and the ctypes binding:
- the repr(C) EmaKvCacheDesc has the header struct's fields, in order, with matching
  types, and so does ema_attn.KvCacheDesc;
- every #define constant of include/ema_attn.h is a `pub const` of the crate, same value;
- every EMA_API function is declared in the crate's extern block with the same
  parameter types and return type;
- the crate's link name and the safe layer's reference-shaped API are present.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ema_attn.h")
CRATE = os.path.join(ROOT, "crates", "attn-hip-ffi")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")


def _strip_c_comments(s):
    return re.sub(r"/\*.*?\*/", " ", s, flags=re.S)


def _strip_rs_comments(s):
    return re.sub(r"//[^\n]*", "", s)


@pytest.fixture(scope="module")
def header():
    return _strip_c_comments(open(HEADER).read())


@pytest.fixture(scope="module")
def rust():
    return _strip_rs_comments(open(LIB_RS).read())


C_TO_RS = {
    "void*": "*mut c_void", "const void*": "*const c_void",
    "int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64", "float": "f32",
    "int32_t*": "*mut i32", "const int32_t*": "*const i32", "uint64_t*": "*mut u64",
    "float*": "*mut f32", "const float*": "*const f32", "const uint32_t*": "*const u32",
    "ema_stream_t": "EmaStream", "ema_kvcache_desc*": "*mut EmaKvCacheDesc",
    "const ema_kvcache_desc*": "*const EmaKvCacheDesc", "const char*": "*const c_char",
}


def _norm_c_type(t):
    return re.sub(r"\s*\*", "*", " ".join(t.split()))


def _c_struct(header):
    body = re.search(r"typedef struct ema_kvcache_desc \{(.*?)\} ema_kvcache_desc;", header, re.S).group(1)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        m = re.match(r"(.+?)\s*(\w+)$", decl)
        fields.append((m.group(2), _norm_c_type(m.group(1))))
    return fields


def _rs_struct(rust):
    body = re.search(r"pub struct EmaKvCacheDesc \{(.*?)\}", rust, re.S).group(1)
    return [(m.group(1), " ".join(m.group(2).split()))
            for m in re.finditer(r"pub (\w+):\s*([^,]+),", body)]


def test_desc_fields_match_header_and_ctypes(header, rust):
    import sys

    sys.path.insert(0, os.path.join(ROOT, "engine-mlx_amd"))
    import ema_attn

    c = _c_struct(header)
    r = _rs_struct(rust)
    assert [n for n, _ in r] == [n for n, _ in c], "field order"
    for (name, ct), (_, rt) in zip(c, r):
        assert C_TO_RS[ct] == rt, (name, ct, rt)
    py = [n for n, _ in ema_attn.KvCacheDesc._fields_]
    assert py == [n for n, _ in c]
    ptypes = dict(ema_attn.KvCacheDesc._fields_)
    size = {"i32": ctypes.c_int32, "i64": ctypes.c_int64, "*mut c_void": ctypes.c_void_p}
    for name, rt in r:
        assert ctypes.sizeof(ptypes[name]) == ctypes.sizeof(size[rt]), name
    assert "#[repr(C)]" in rust.split("pub struct EmaKvCacheDesc")[0][-200:]


def _c_defines(header):
    out = {}
    for m in re.finditer(r"^#define (EMA_[A-Z0-9_]+)\s+(.+?)\s*$", header, re.M):
        v = m.group(2).strip()
        v = re.sub(r"(?<=\d)(ull|ul|u|ll)\b", "", v, flags=re.I)
        try:
            out[m.group(1)] = int(eval(v, {}))  # integer literals, shifts and parentheses only
        except Exception:
            continue
    return out


def test_every_constant_is_in_the_crate(header, rust):
    consts = {m.group(1): int(eval(m.group(3), {}))
              for m in re.finditer(r"pub const (EMA_\w+):\s*(\w+)\s*=\s*([^;]+);", rust)}
    defines = _c_defines(header)
    names = set(re.findall(r"^#define (EMA_\w+)", header, re.M)) - {"EMA_ATTN_H", "EMA_API"}
    assert set(defines) == names, names - set(defines)  # every value constant parsed
    for name, value in defines.items():
        assert name in consts, f"{name} missing from the crate"
        assert consts[name] == value, (name, consts[name], value)


def _c_functions(header):
    fns = {}
    for m in re.finditer(r"EMA_API\s+([\w\s\*]+?)\s*(ema_\w+)\s*\(([^)]*)\)\s*;", header):
        ret = _norm_c_type(m.group(1))
        params = []
        args = m.group(3).strip()
        if args and args != "void":
            for p in args.split(","):
                pm = re.match(r"(.+?)\s*(\w+)$", " ".join(p.split()))
                params.append(_norm_c_type(pm.group(1)))
        fns[m.group(2)] = (ret, params)
    return fns


def _rs_functions(rust):
    block = re.search(r'pub mod sys \{.*?extern "C" \{(.*?)\n    \}\n\}', rust, re.S).group(1)
    fns = {}
    for m in re.finditer(r"pub fn (ema_\w+)\((.*?)\)\s*->\s*([^;]+);", block, re.S):
        params = []
        args = " ".join(m.group(2).split())
        if args:
            for p in args.split(","):
                p = p.strip()
                if p:
                    params.append(" ".join(p.split(":", 1)[1].split()))
        fns[m.group(1)] = (" ".join(m.group(3).split()), params)
    return fns


def test_every_export_is_declared_with_matching_types(header, rust):
    c = _c_functions(header)
    r = _rs_functions(rust)
    assert len(c) >= 20
    assert set(c) == set(r), (set(c) ^ set(r))
    for name, (ret, params) in c.items():
        rret, rparams = r[name]
        assert C_TO_RS[ret] == rret, (name, ret, rret)
        assert [C_TO_RS[p] for p in params] == rparams, name


def test_crate_links_the_library_and_mirrors_the_reference_api(rust):
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert re.search(r'^links = "ema_attn"', toml, re.M)
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=ema_attn" in build
    for item in ("pub trait KvCache: Send", "fn append(&mut self, ctx: &HipCtx", "fn get(&self, ctx: &HipCtx)",
                 "fn len(&self) -> usize", "fn reset(&mut self)", "fn memory_bytes(&self) -> usize",
                 "impl KvCache for StaticCache", "pub struct QuantWeights", "pub struct GqaWeights",
                 "pub struct GqaConfig", "pub q_norm: Option<DeviceArray>",
                 # the layer functions are generic over the cache, as gqa.rs:62-69 is
                 "pub trait HipKvCache: KvCache", "fn desc(&self) -> &sys::EmaKvCacheDesc",
                 "fn position(&self, ctx: &HipCtx, p: i64) -> Result<*const i32>",
                 "pub fn gqa_attention<C: HipKvCache>(", "pub fn sliding_window_attention<C: HipKvCache>(",
                 "pub fn gqa_workspace_bytes_for<C: HipKvCache>("):
        assert item in rust, item
    for cache in ("StaticCache", "RotatingCache", "Fp8Cache"):
        assert f"impl KvCache for {cache}" in rust and f"impl HipKvCache for {cache}" in rust, cache
        assert f"unsafe impl Send for {cache}" in rust, cache
    # the ring flag, the slot write and the FP8 conversions are what the types rest on
    assert "cache.desc.flags = sys::EMA_KV_ROTATING" in rust
    assert "sys::ema_position_write(ctx.stream, self.slot" in rust
    assert rust.count("sys::ema_kvcache_convert(") == 2
    assert "sys::ema_kvcache_alloc_fp8(" in rust and "sys::ema_prefill_attention_ws(" in rust


def test_crate_source_is_balanced(rust):
    """No Rust toolchain here: at least the delimiters of the crate source pair up."""
    text = re.sub(r'"(\\.|[^"\\])*"', '""', rust)  # string literals
    text = re.sub(r"'(\\.|[^'\\])'", "' '", text)  # char literals
    stack = []
    pairs = {")": "(", "]": "[", "}": "{"}
    for i, ch in enumerate(text):
        if ch in "([{":
            stack.append((ch, i))
        elif ch in pairs:
            assert stack and stack[-1][0] == pairs[ch], f"unbalanced {ch} at {i}: {text[max(0, i - 80):i + 1]}"
            stack.pop()
    assert not stack, stack[-1]
