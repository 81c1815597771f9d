"""Generates src/bindings.rs (the raw Rust FFI of libtqkv) from include/tqkv.h.

The reference's host code is Rust; this crate is the thin -sys layer its
turboquant-cache / lumen-mlx callers would link against. There is no Rust
toolchain in this build's image, so the bindings are generated here from the
C header (C types mapped one for one: fixed-width integers, const/mut
pointers, #[repr(C)] structs, opaque handles) and tests/test_rust_sys.py
checks that the committed file matches the header.

    python3 gen_bindings.py            # rewrite src/bindings.rs
"""
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(HERE, "..", "..", "..", "include", "tqkv.h")
OUT = os.path.join(HERE, "src", "bindings.rs")

BASE = {
    "int32_t": "i32", "int64_t": "i64", "uint64_t": "u64", "uint32_t": "u32",
    "uint16_t": "u16", "uint8_t": "u8", "size_t": "usize", "float": "f32", "double": "f64",
    "char": "c_char", "void": "c_void",
}
RUST_KEYWORDS = {"type", "ref", "match", "fn", "mod", "use", "where", "loop", "move", "box",
                 "self", "in", "impl", "trait", "struct", "enum", "crate", "super", "dyn"}


def strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def rust_type(ctype, opaque):
    """C type text (no declarator name) -> Rust type."""
    toks = re.findall(r"\*|const|[A-Za-z_][A-Za-z0-9_]*", ctype)
    toks = [t for t in toks if t != "struct"]
    base_const = False
    i = 0
    if toks and toks[0] == "const":
        base_const, i = True, 1
    base = toks[i]
    i += 1
    if i < len(toks) and toks[i] == "const":  # "T const*"
        base_const, i = True, i + 1
    out = BASE.get(base, base)
    pending_const = base_const
    while i < len(toks):
        assert toks[i] == "*", ctype
        out = f"*{'const' if pending_const else 'mut'} {out}"
        i += 1
        pending_const = False
        if i < len(toks) and toks[i] == "const":
            pending_const, i = True, i + 1
    return out


def split_decl(decl):
    """'const uint16_t* q' -> ('const uint16_t*', 'q'); arrays 'void* slot[6]'."""
    decl = decl.strip()
    m = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)\s*(\[\s*(\d+)\s*\])?$", decl, flags=re.S)
    ctype, name, _, n = m.group(1).strip(), m.group(2), m.group(3), m.group(4)
    return ctype, name, (int(n) if n else None)


def ident(name):
    return f"r#{name}" if name in RUST_KEYWORDS else name


def generate(header_text):
    src = strip_comments(header_text)
    lines = ["// Generated from include/tqkv.h by gen_bindings.py; do not edit.",
             "#![allow(non_camel_case_types, non_snake_case, dead_code)]", "",
             "use core::ffi::{c_char, c_void};", "",
             "/// hipStream_t: the HIP stream work is queued on (null: the default stream).",
             "pub type tqkv_stream = *mut c_void;", ""]
    for name, value in re.findall(r"#define\s+(TQKV_[A-Z0-9_]+)\s+(-?\d+)", src):
        lines.append(f"pub const {name}: i32 = {value};")
    lines.append("")
    opaque = set(re.findall(r"typedef\s+struct\s+(\w+)\s+\1\s*;", src))
    for name in sorted(opaque):
        lines += ["#[repr(C)]", f"pub struct {name} {{", "    _private: [u8; 0],", "}", ""]
    for body, name in re.findall(r"typedef\s+struct\s+\w+\s*\{(.*?)\}\s*(\w+)\s*;", src, flags=re.S):
        lines += ["#[repr(C)]", "#[derive(Debug, Copy, Clone)]", f"pub struct {name} {{"]
        for field in [f for f in body.split(";") if f.strip()]:
            ctype, fname, n = split_decl(field)
            rt = rust_type(ctype, opaque)
            lines.append(f"    pub {ident(fname)}: {f'[{rt}; {n}]' if n else rt},")
        lines += ["}", ""]
    lines.append('extern "C" {')
    protos = re.findall(r"\n\s*((?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**)\s*(tqkv_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;",
                        src, flags=re.S)
    for ret, name, params in protos:
        args = []
        params = " ".join(params.split())
        if params and params != "void":
            for p in params.split(","):
                ctype, pname, n = split_decl(p)
                assert n is None, p
                args.append(f"{ident(pname)}: {rust_type(ctype, opaque)}")
        rret = rust_type(ret, opaque)
        lines.append(f"    pub fn {name}({', '.join(args)}) -> {rret};")
    lines += ["}", ""]
    return "\n".join(lines)


def header_functions(header_text):
    return sorted(set(re.findall(r"\b(tqkv_[a-z0-9_]+)\s*\(", strip_comments(header_text))))


if __name__ == "__main__":
    text = generate(open(HEADER).read())
    with open(OUT, "w") as f:
        f.write(text)
    print(f"wrote {OUT}", file=sys.stderr)
