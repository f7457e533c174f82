"""The bindings above the C ABI agree with include/mvr_attn.h (CPU only, no launch).

* The Rust module a maintainer drops into the reference (mini-vllm-rs_amd/rust/mvr_attn.rs): every #[repr(C)]
  struct has its C struct's fields in the same order with the same widths, and every extern fn the C
  prototype's argument and return types.  (No Rust toolchain exists in this image, so the source is checked
  against the header by parsing both.)
* The Python ctypes mirror (mvr_attn.py): the same field names at the offsets gcc gives the C structs, and the
  same struct sizes.
"""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

import mvr_attn as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mvr_attn.h")
RUST = os.path.join(ROOT, "mini-vllm-rs_amd", "rust", "mvr_attn.rs")

STRUCTS = {  # C typedef -> (Rust struct, ctypes mirror)
    "mvr_paged_attention_args": ("MvrPagedAttentionArgs", M.PagedAttentionArgs),
    "mvr_cascade_groups": ("MvrCascadeGroups", M.CascadeGroups),
    "mvr_attention_dimensions": ("MvrAttentionDimensions", M.AttentionDimensions),
    "mvr_paged_cache_layout": ("MvrPagedCacheLayout", M.PagedCacheLayoutC),
    "mvr_rope_append_args": ("MvrRopeAppendArgs", M.RopeAppendArgs),
}

# C type -> Rust type (both sides of an FFI boundary must agree on width and pointer-ness).
C_TO_RUST = {
    "int32_t": "i32", "int64_t": "i64", "float": "f32", "size_t": "usize", "int": "c_int",
    "const void*": "*const c_void", "void*": "*mut c_void", "const int32_t*": "*const i32",
    "const uint8_t*": "*const u8", "const char*": "*const c_char", "void": "()",
}


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def _norm_c_type(t):
    t = " ".join(t.split())
    t = re.sub(r"\s*\*", "*", t)
    return t


def c_structs():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for body, name in re.findall(r"typedef struct \w+ \{(.*?)\} (\w+);", text, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            m = re.match(r"^(const )?(\w+)\s*(\*?)\s*(.*)$", decl)
            const, base, star, names = m.groups()
            ctype = _norm_c_type(f"{const or ''}{base}{star}")
            for n in names.split(","):
                n = n.strip()
                if n.startswith("*"):  # "T *a" style
                    ctype, n = _norm_c_type(ctype + "*"), n[1:]
                fields.append((n, ctype))
        out[name] = fields
    return out


def c_functions():
    text = _strip_c_comments(open(HEADER).read())
    funcs = {}
    for ret, name, args in re.findall(r"\n\s*([\w ]+?\*?)\s*\b(mvr_\w+)\s*\(([^)]*)\)\s*;", text):
        types = []
        for a in args.split(","):
            a = " ".join(a.split())
            if not a or a == "void":
                continue
            m = re.match(r"^(.*?)(\w+)$", a)
            types.append(_norm_c_type(m.group(1)))
        funcs[name] = (_norm_c_type(ret), types)
    return funcs


def rust_structs():
    text = open(RUST).read()
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+) \{(.*?)\n\}", text, flags=re.S):
        fields = []
        for line in body.splitlines():
            line = line.split("//")[0].strip()
            if not line:
                continue
            m = re.match(r"^pub (\w+): (.+?),$", line)
            assert m, line
            fields.append((m.group(1), " ".join(m.group(2).split())))
        out[name] = fields
    return out


def rust_functions():
    text = open(RUST).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, flags=re.S).group(1)
    funcs = {}
    for name, args, ret in re.findall(r"pub fn (\w+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        types = []
        for a in args.split(","):
            a = " ".join(a.split())
            if a:
                types.append(a.split(":", 1)[1].strip())
        funcs[name] = ((ret or "()").strip(), types)
    return funcs


def test_header_parses():
    s = c_structs()
    assert set(STRUCTS) <= set(s)
    assert ("cu_q_lens_host", "const int32_t*") in s["mvr_paged_attention_args"]
    assert ("q_stride_token", "int64_t") in s["mvr_rope_append_args"]
    assert set(c_functions()) == set(M.EXPORTED_SYMBOLS)


@pytest.mark.parametrize("c_name", sorted(STRUCTS))
def test_rust_structs_match_the_header(c_name):
    rust_name = STRUCTS[c_name][0]
    c_fields = c_structs()[c_name]
    r_fields = rust_structs()[rust_name]
    assert [n for n, _ in r_fields] == [n for n, _ in c_fields]
    for (n, ct), (_, rt) in zip(c_fields, r_fields):
        assert C_TO_RUST[ct] == rt, (c_name, n, ct, rt)


def test_rust_extern_functions_match_the_header():
    cf, rf = c_functions(), rust_functions()
    assert set(rf) == set(cf)
    struct_map = {f"const {c}*": f"*const {r}" for c, (r, _) in STRUCTS.items()}
    for name, (cret, cargs) in cf.items():
        rret, rargs = rf[name]
        mapped = [struct_map.get(t, C_TO_RUST.get(t)) for t in cargs]
        assert mapped == rargs, (name, cargs, rargs)
        assert C_TO_RUST[cret] == rret, (name, cret, rret)


def test_rust_constants_match_the_header():
    text = open(RUST).read()
    header = _strip_c_comments(open(HEADER).read())
    assert f"MVR_ATTN_ABI_VERSION: c_int = {M.ABI_VERSION};" in text
    assert f"#define MVR_ATTN_ABI_VERSION {M.ABI_VERSION}" in header
    for name, value in re.findall(r"\b(MVR_E_\w+|MVR_OK)\s*=\s*(-?\d+)", header):
        assert re.search(rf"pub const {name}: c_int = {value};", text), name


@pytest.mark.skipif(subprocess.run(["which", "gcc"], capture_output=True).returncode != 0, reason="no gcc")
def test_ctypes_mirror_has_the_c_layout():
    """gcc's offsetof / sizeof for every field against the Python ctypes structs."""
    structs = c_structs()
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "mvr_attn.h"', "int main(void) {"]
    for c_name in STRUCTS:
        lines.append(f'  printf("{c_name} sizeof %zu\\n", sizeof({c_name}));')
        for n, _ in structs[c_name]:
            lines.append(f'  printf("{c_name} {n} %zu\\n", offsetof({c_name}, {n}));')
    lines.append("  return 0;\n}")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), src, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {}
    for line in out:
        if line:
            s, f, v = line.split()
            got[(s, f)] = int(v)
    for c_name, (_, mirror) in STRUCTS.items():
        assert [n for n, _ in mirror._fields_] == [n for n, _ in structs[c_name]], c_name
        assert ctypes.sizeof(mirror) == got[(c_name, "sizeof")], c_name
        for n, _ in mirror._fields_:
            assert getattr(mirror, n).offset == got[(c_name, n)], (c_name, n)
