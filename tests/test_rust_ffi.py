"""The Rust FFI crate (crates/webyiq-hip-sys, the binding webyIQ's engine
would link in place of its WGSL dispatches, graph.rs:190-222) against the C
header, on the CPU: no Rust toolchain exists in this image, so the crate is
checked as text.  Every function declared in include/webyiq_q4q8.h appears
in the crate's extern "C" block with the same name, arity, argument types
and return type (C type -> Rust type by the standard FFI mapping), and
every #define constant has a Rust const of the same value."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "webyiq_q4q8.h")
CRATE = os.path.join(ROOT, "crates", "webyiq-hip-sys")

C_TO_RUST = {
    "void*": "*mut c_void", "const void*": "*const c_void",
    "const char*": "*const c_char",
    "float": "f32", "const float*": "*const f32", "float*": "*mut f32",
    "int8_t*": "*mut i8", "const int8_t*": "*const i8",
    "int32_t": "i32", "int32_t*": "*mut i32", "const int32_t*": "*const i32",
    "uint32_t*": "*mut u32", "const uint32_t*": "*const u32",
    "int64_t": "i64", "size_t": "usize", "int": "i32",
    "const wq_params*": "*const WqParams",
}


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", re.sub(r"//[^\n]*", "", text, flags=re.S), flags=re.S)


def c_declarations():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"((?:const\s+)?\w+\s*\*?)\s*(wq_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        types = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p in ("", "void"):
                continue
            # drop the parameter name: the last identifier
            t = re.sub(r"\s*\b\w+$", "", p).replace(" *", "*").strip()
            types.append(t)
        out[name] = (" ".join(ret.split()).replace(" *", "*"), types)
    return out


def rust_declarations():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (wq_\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        name, params, ret = m.group(1), m.group(2), (m.group(3) or "()").strip()
        types = []
        for p in params.split(","):
            p = " ".join(p.split())
            if not p:
                continue
            types.append(p.split(":", 1)[1].strip())
        out[name] = (ret, types)
    return out


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs")):
        assert os.path.isfile(os.path.join(CRATE, f)), f
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'links = "webyiq_q4q8"' in cargo
    assert "rustc-link-lib=dylib=webyiq_q4q8" in open(os.path.join(CRATE, "build.rs")).read()


def test_every_header_function_bound_with_the_same_signature():
    c = c_declarations()
    r = rust_declarations()
    assert len(c) == 20
    assert set(c) == set(r), (set(c) ^ set(r))
    for name, (cret, cargs) in c.items():
        rret, rargs = r[name]
        assert len(cargs) == len(rargs), f"{name}: arity {len(cargs)} vs {len(rargs)}"
        want_ret = C_TO_RUST[cret]
        assert rret == want_ret, f"{name}: returns {rret}, header {cret}"
        for i, (ct, rt) in enumerate(zip(cargs, rargs)):
            assert C_TO_RUST[ct] == rt, f"{name} argument {i}: {rt} vs header {ct}"


def test_constants_match_the_header():
    defs = dict(re.findall(r"#define\s+(WQ_\w+)\s+\(?(-?\d+)\)?", open(HEADER).read()))
    consts = dict(re.findall(r"pub const (WQ_\w+): i32 = (-?\d+);", open(os.path.join(CRATE, "src", "lib.rs")).read()))
    assert defs and set(defs) == set(consts)
    for k, v in defs.items():
        assert int(consts[k]) == int(v), k


def test_params_struct_matches_the_header():
    """wq_params and the crate's #[repr(C)] WqParams: the same u32 fields in
    the same order (the layout the kernels read, word 0 pos, word 2 m)."""
    hdr = _strip_c_comments(open(HEADER).read())
    cfields = re.findall(r"uint32_t\s+(\w+);", re.search(r"typedef struct wq_params \{(.*?)\}", hdr, re.S).group(1))
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    body = re.search(r"#\[repr\(C\)\][^{]*pub struct WqParams \{(.*?)\}", text, re.S).group(1)
    rfields = re.findall(r"pub (\w+): u32,", body)
    assert cfields == ["pos", "seq_len", "m", "slot"]
    assert rfields == cfields


def test_header_parser_catches_a_mismatch():
    """The checker itself: a planted change in a signature is detected."""
    c = c_declarations()
    ret, args = c["wq_gemv"]
    args = list(args)
    args[3], args[4] = "int32_t", "int64_t"   # swapped n / k types
    assert [C_TO_RUST[t] for t in args] != rust_declarations()["wq_gemv"][1]
