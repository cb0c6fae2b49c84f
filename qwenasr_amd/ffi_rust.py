"""Rust FFI module for include/qasr_hip.h, generated from the header.

    python -m qwenasr_amd.ffi_rust > hip.rs

Emits what the reference crate would add as `src/kernels/hip.rs` (behind its
`hip` feature): the status and mode constants, one opaque `#[repr(C)]` type
per handle, one `#[repr(C)]` struct per configuration / weight table with the
header's field order, and one `extern "C"` declaration per entry point, with
the header's argument names.  The integration notes embed this output, and
tests/test_abi.py checks that the embedded copy is current.
"""
import os
import re
import sys

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "qasr_hip.h")

SCALARS = {"int": "c_int", "int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "uint16_t": "u16",
           "int8_t": "i8", "uint8_t": "u8", "float": "f32", "double": "f64", "size_t": "usize", "char": "c_char",
           "void": "c_void", "unsigned": "u32"}


def camel(name):
    return "".join(p.capitalize() for p in name.split("_"))


def strip_comments(src):
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    return re.sub(r"//[^\n]*", " ", src)


def rust_type(ctype, structs):
    """A C type spelled as in the header ('const float *', 'qasr_hip **',
    'const float *const *') -> its Rust FFI spelling."""
    t = " ".join(ctype.replace("*", " * ").split())
    toks = t.split(" ")
    # base type and its qualifier
    base_const = toks[0] == "const"
    if base_const:
        toks = toks[1:]
    base = toks[0]
    rest = toks[1:]
    rb = SCALARS.get(base) or (camel(base) if base in structs else None)
    if rb is None:
        raise ValueError(f"unknown C type {ctype!r}")
    # pointer levels, innermost first: each '*' may be followed by 'const'
    levels = []
    i = 0
    while i < len(rest):
        if rest[i] == "*":
            const_after = i + 1 < len(rest) and rest[i + 1] == "const"
            levels.append(const_after)
            i += 2 if const_after else 1
        else:
            raise ValueError(f"cannot parse C type {ctype!r}")
    if not levels:
        return "()" if rb == "c_void" else rb
    out = rb
    # the pointee of the first '*' is the base (const if base_const); the
    # pointee of later '*'s is the previous pointer (const if that '*' was
    # followed by const)
    pointee_const = base_const
    for k, const_after in enumerate(levels):
        out = f"*{'const' if pointee_const else 'mut'} {out}"
        pointee_const = const_after
    return out


def parse(src):
    text = strip_comments(src)
    consts = re.findall(r"#define\s+(QASR_[A-Z0-9_]+)\s+\(?(-?\d+)\)?", text)
    opaque = re.findall(r"typedef\s+struct\s+(\w+)\s+\1\s*;", text)
    structs_raw = re.findall(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S)
    names = set(opaque) | {n for _, n in structs_raw}
    structs = []
    for body, name in structs_raw:
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            m = re.match(r"((?:const\s+)?\w+)\s*(.*)", decl)
            base, declarators = m.group(1), m.group(2)
            for d in declarators.split(","):
                d = d.strip()
                stars = d.count("*")
                fname = d.replace("*", "").strip()
                arr = re.match(r"(\w+)\[(\d+)\]", fname)
                ctype = base + " " + "*" * stars
                rt = rust_type(ctype, names)
                if arr:
                    fields.append((arr.group(1), f"[{rt}; {arr.group(2)}]"))
                else:
                    fields.append((fname, rt))
        structs.append((name, fields))
    # function prototypes: flatten whitespace, drop preprocessor lines
    flat = " ".join(l for l in text.splitlines() if not l.strip().startswith("#"))
    flat = re.sub(r"typedef\s+struct\s*\{.*?\}\s*\w+\s*;", " ", flat)
    flat = re.sub(r"typedef\s+struct\s+\w+\s+\w+\s*;", " ", flat)
    flat = re.sub(r'extern\s+"C"\s*\{|\}', " ", flat)
    funcs = []
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(qasr_hip_\w+)\s*\(([^)]*)\)\s*;", flat):
        ret, name, args = " ".join(m.group(1).split()), m.group(2), m.group(3).strip()
        params = []
        if args and args != "void":
            for a in args.split(","):
                a = " ".join(a.split())
                pm = re.match(r"(.*?)(\w+)$", a)
                ctype, pname = pm.group(1).strip(), pm.group(2)
                params.append((pname, rust_type(ctype, names)))
        funcs.append((name, params, rust_type(ret, names)))
    return consts, opaque, structs, funcs


RUST_KEYWORDS = {"type", "ref", "in", "fn", "loop", "match", "move", "mut", "self", "super", "use", "where"}


def render(src):
    consts, opaque, structs, funcs = parse(src)
    out = ['#![cfg(feature = "hip")]',
           "// Generated from include/qasr_hip.h by `python -m qwenasr_amd.ffi_rust`.",
           "#![allow(non_camel_case_types, dead_code)]",
           "use std::ffi::{c_char, c_int, c_void};", ""]
    for n, v in consts:
        out.append(f"pub const {n}: c_int = {v};")
    out.append("")
    for n in opaque:
        out.append(f"#[repr(C)] pub struct {camel(n)} {{ _p: [u8; 0] }}")
    out.append("")
    for n, fields in structs:
        out.append("#[repr(C)] #[derive(Clone, Copy)]")
        out.append(f"pub struct {camel(n)} {{")
        for f, t in fields:
            out.append(f"    pub {f}: {t},")
        out.append("}")
    out.append("")
    out.append('extern "C" {')
    for name, params, ret in funcs:
        ps = ", ".join(f"{p + '_' if p in RUST_KEYWORDS else p}: {t}" for p, t in params)
        r = "" if ret == "()" else f" -> {ret}"
        out.append(f"    pub fn {name}({ps}){r};")
    out.append("}")
    return "\n".join(out) + "\n"


if __name__ == "__main__":
    sys.stdout.write(render(open(sys.argv[1] if len(sys.argv) > 1 else HEADER).read()))
