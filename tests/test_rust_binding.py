"""The Rust side of the boundary, checked against the C header without a Rust toolchain:
every function include/ppocr_rechead.h declares is declared in the ppocr-hip-sys crate's
extern "C" block with the same parameter and return types (C type -> Rust type mapping
below), nothing else is declared there, and every call the reference-side wrapper makes
through the crate names a declared function with its number of arguments."""
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ppocr_rechead.h")
CRATE = os.path.join(ROOT, "rust-ppocrv6_amd", "ppocr-hip-sys")
PATCH = os.path.join(ROOT, "rust-ppocrv6_amd", "reference_patch")

C_TO_RUST = {
    "void": None, "int": "c_int", "size_t": "usize", "int64_t": "i64", "int32_t": "i32",
    "const char*": "*const c_char", "char*": "*mut c_char", "void*": "*mut c_void",
    "const float*": "*const f32", "float*": "*mut f32", "const int8_t*": "*const i8", "int8_t*": "*mut i8",
    "const int32_t*": "*const i32", "int32_t*": "*mut i32", "const int64_t*": "*const i64", "int64_t*": "*mut i64",
    "int*": "*mut c_int", "const ppocr_rh_t*": "*const ppocr_rh_t", "ppocr_rh_t*": "*mut ppocr_rh_t",
    "ppocr_rh_t**": "*mut *mut ppocr_rh_t", "float": "f32", "const ppocr_rn_block_t*": "*const ppocr_rn_block_t",
    "const ppocr_rn_t*": "*const ppocr_rn_t", "ppocr_rn_t*": "*mut ppocr_rn_t", "ppocr_rn_t**": "*mut *mut ppocr_rn_t",
}


def _norm_c(t):
    t = " ".join(t.replace("*", " * ").split())
    return t.replace(" *", "*").replace("* *", "**")


def header_decls():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"([\w\s\*]+?)\b(ppocr_\w+)\s*\(([^)]*)\)\s*;", text):
        ret = _norm_c(m.group(1).strip())
        params = [] if m.group(3).strip() in ("", "void") else [p.strip() for p in m.group(3).split(",")]
        types = [_norm_c(re.sub(r"\s*\b\w+$", "", p)) for p in params]
        out[m.group(2)] = (ret, types)
    return out


def rust_decls():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = re.search(r'extern "C" \{(.*)\n\}', text, flags=re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        types = [" ".join(p.split(":", 1)[1].split()) for p in params]
        ret = " ".join(m.group(4).split()) if m.group(4) else None
        out[m.group(1)] = (ret, types)
    return out


def test_extern_block_declares_exactly_the_header():
    h, r = header_decls(), rust_decls()
    assert len(h) >= 28
    assert set(h) == set(r), set(h) ^ set(r)


@pytest.mark.parametrize("name", sorted(header_decls()))
def test_extern_types_match_the_header(name):
    hret, htypes = header_decls()[name]
    rret, rtypes = rust_decls()[name]
    assert C_TO_RUST[hret] == rret, (name, hret, rret)
    assert len(htypes) == len(rtypes), (name, htypes, rtypes)
    for i, (c, rs) in enumerate(zip(htypes, rtypes)):
        assert C_TO_RUST[c] == rs, (name, i, c, rs)


def test_crate_constants_match_the_header():
    h = open(HEADER).read()
    rs = open(os.path.join(CRATE, "src", "lib.rs")).read()
    consts = dict(re.findall(r"#define (PPOCR_\w+) (\d+)", h))
    consts.update({k: v for k, v in re.findall(r"(PPOCR_MODE_\w+) = (\d+)", h)})
    assert len(consts) >= 9
    for k, v in consts.items():
        assert re.search(rf"pub const {k}: c_int = {v};", rs), k


def test_build_script_compiles_every_library_source_for_gfx950_only():
    b = open(os.path.join(CRATE, "build.rs")).read()
    mk = open(os.path.join(ROOT, "rust-ppocrv6_amd", "csrc", "Makefile")).read().replace("\\\n", " ")
    srcs = re.findall(r"(\w+\.(?:hip|cpp))", re.search(r"HIP_SRCS = ([^\n]*)\nCPP_SRCS = ([^\n]*)", mk).group(0))
    listed = re.findall(r'"(\w+\.(?:hip|cpp))"', b)
    assert sorted(srcs) == sorted(listed)
    assert re.findall(r"--offload-arch=(\w+)", b) == ["gfx950"]
    assert "-packed-fp32-ops" in b


def test_reference_side_calls_match_the_declarations():
    decls = rust_decls()
    calls = 0
    for dirpath, _, files in os.walk(PATCH):
        for f in files:
            if not f.endswith(".rs"):
                continue
            text = open(os.path.join(dirpath, f)).read()
            for m in re.finditer(r"sys::(ppocr_\w+)\(", text):
                name = m.group(1)
                assert name in decls, (f, name)
                # the argument list up to the matching parenthesis
                depth, i, args, cur = 1, m.end(), [], ""
                while depth:
                    ch = text[i]
                    if ch in "([{":
                        depth += 1
                    elif ch in ")]}":
                        depth -= 1
                    if depth == 1 and ch == ",":
                        args.append(cur)
                        cur = ""
                    elif depth:
                        cur += ch
                    i += 1
                if cur.strip():
                    args.append(cur)
                assert len(args) == len(decls[name][1]), (f, name, len(args))
                calls += 1
    assert calls >= 10
