"""The Rust side of the boundary, checked against the C header without a Rust toolchain:
every function include/ppocr_rechead.h declares is declared in the ppocr-hip-sys crate's
extern "C" block with the same parameter and return types (C type -> Rust type mapping
below), nothing else is declared there, and every call the reference-side wrapper makes
through the crate names a declared function with its number of arguments.  The edits of the
reference's executor and pipeline (reference_patch/patches/*.patch) apply to the reference's
files, are what make_patches.py writes, and call only wrapper and Model methods that exist,
with their number of arguments."""
import os
import re
import shutil
import subprocess
import sys

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
    "void* const*": "*const *mut c_void", "const char**": "*mut *const c_char",
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
    block = re.search(r"const SOURCES: &\[&str\] = &\[(.*?)\];", b, re.S).group(1)
    listed = re.findall(r'"(\w+\.(?:hip|cpp))"', block)
    assert sorted(srcs) == sorted(listed)
    assert re.findall(r"--offload-arch=(\w+)", b) == ["gfx950"]
    assert "-packed-fp32-ops" in b
    # the same per-file flags as the Makefile
    mk_file = dict(re.findall(r"\$\(OBJDIR\)/(\w+)\.o: FILE_FLAGS = ([^\n]*)", mk))
    rs_file = {m.group(1).split(".")[0]: " ".join(re.findall(r'"([^"]+)"', m.group(2)))
               for m in re.finditer(r'if src == "(\w+\.hip)" \{\s*&\[([^\]]*)\]', b)}
    assert mk_file == rs_file and mk_file


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


REF = "/root/reference"
PATCHES = {"engine_model.patch": "src/engine/model.rs", "pipeline.patch": "src/pipeline.rs"}


def _call_args(text, start):
    """Arguments of the call whose '(' ends at text[start - 1]: split at top-level commas."""
    depth, i, args, cur = 1, start, [], ""
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
    return [a for a in args if a.strip()]


def _rust_fns(text):
    """pub fn name(params) -> number of parameters other than self."""
    out = {}
    for m in re.finditer(r"pub(?:\(crate\))? fn (\w+)\s*(?:<[^>]*>)?\(", text):
        params = _call_args(text, m.end())
        out[m.group(1)] = len([p for p in params if not re.match(r"\s*&?\s*(mut\s+)?self\b", p)])
    return out


def _added(patch):
    return "\n".join(l[1:] for l in open(os.path.join(PATCH, "patches", patch)).read().splitlines()
                     if l.startswith("+") and not l.startswith("+++"))


@pytest.mark.skipif(not os.path.isdir(REF) or not shutil.which("patch"), reason="the reference crate is not here")
def test_patches_apply_to_the_reference_and_are_current(tmp_path):
    for patch, rel in PATCHES.items():
        dst = tmp_path / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copy(os.path.join(REF, rel), dst)
        r = subprocess.run(["patch", "-p1", "--dry-run", "-i", os.path.join(PATCH, "patches", patch)],
                           cwd=tmp_path, capture_output=True, text=True)
        assert r.returncode == 0 and "FAILED" not in r.stdout and "fuzz" not in r.stdout, (patch, r.stdout, r.stderr)
    # regenerate into a scratch copy of the generator's folder: the committed diffs are its output
    scratch = tmp_path / "gen"
    shutil.copytree(PATCH, scratch, ignore=shutil.ignore_patterns("patches"))
    subprocess.run([sys.executable, str(scratch / "make_patches.py"), REF], check=True, capture_output=True)
    for patch in PATCHES:
        assert (scratch / "patches" / patch).read_text() == open(os.path.join(PATCH, "patches", patch)).read(), patch


def test_patch_calls_name_existing_methods_with_their_arity():
    head = _rust_fns(open(os.path.join(PATCH, "src", "ops", "gpu_head.rs")).read())
    ctc = _rust_fns(open(os.path.join(PATCH, "src", "postprocess", "ctc", "gpu.rs")).read())
    model_added = _added("engine_model.patch")
    model = _rust_fns(model_added)
    assert {"attach_gpu_heads", "rec_head", "forward_until"} <= set(model)
    expect = {
        # receiver pattern -> the methods it may call, with where they are defined
        r"\bhead\.(\w+)\(": head,
        r"GpuHead::(\w+)\(": head,
        r"self\.ctc_decoder\.(\w+)\(": ctc,
        r"(?:self\.)?rec_model\.(\w+)\(": model,
    }
    seen = 0
    for patch in PATCHES:
        text = _added(patch)
        for pat, defs in expect.items():
            for m in re.finditer(pat, text):
                name = m.group(1)
                if defs is model and name not in model:
                    continue  # the reference's own Model methods (quantize_matmul_weights, ...)
                assert name in defs, (patch, name)
                assert len(_call_args(text, m.end())) == defs[name], (patch, name)
                seen += 1
    assert seen >= 8
