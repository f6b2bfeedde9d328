"""The Rust `sys` module in INTEGRATION.md is a complete transcription of
include/hx.h: every constant, enum, struct and entry point, with each C type
mapped to its Rust FFI equivalent.  The expected text is generated here from
the header, so a declaration added to or changed in hx.h without the matching
change in the guide fails this test (CPU only; no toolchain for Rust is
needed to check it).

To refresh the guide after changing hx.h, print `rust_sys_module()` and paste
it between the markers in INTEGRATION.md.
"""
from __future__ import annotations

import re
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "hx.h"
GUIDE = REPO / "INTEGRATION.md"
BEGIN = "// ---- begin: generated from include/hx.h ----"
END = "// ---- end: generated from include/hx.h ----"

SCALARS = {"void": "c_void", "char": "c_char", "int32_t": "i32", "uint32_t": "u32", "int64_t": "i64",
           "uint64_t": "u64", "float": "f32", "double": "f64"}
RUST_KEYWORDS = {"in": "input", "type": "kind", "ref": "reference", "fn": "func"}


def _strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _base(name: str) -> str:
    return SCALARS.get(name, name)


def rust_type(c: str) -> str:
    """A C parameter or return type of hx.h as its Rust FFI type."""
    c = " ".join(c.replace("*", " * ").split())
    toks = c.split(" ")
    const_first = toks[0] == "const"
    if const_first:
        toks = toks[1:]
    base, rest = _base(toks[0]), toks[1:]
    if not rest:
        assert not const_first, c
        return "()" if base == "c_void" else base
    # rest is a sequence of '*' and 'const' qualifiers read left to right:
    # the innermost pointee first.
    ptrs = []  # for each '*', whether the pointee is const
    pointee_const = const_first
    i = 0
    while i < len(rest):
        assert rest[i] == "*", c
        ptrs.append(pointee_const)
        pointee_const = False
        if i + 1 < len(rest) and rest[i + 1] == "const":
            pointee_const = True  # `T *const *`: the next level points at a const pointer
            i += 1
        i += 1
    assert not pointee_const, c  # a const pointer parameter itself is not a type distinction here
    out = base
    for is_const in ptrs:
        out = ("*const " if is_const else "*mut ") + out
    return out


def _split_params(params: str):
    params = params.strip()
    if params == "void":
        return []
    out = []
    for p in params.split(","):
        p = " ".join(p.replace("*", " * ").split())
        m = re.match(r"^(.*?)([A-Za-z_][A-Za-z0-9_]*)$", p)
        ctype, name = m.group(1).strip(), m.group(2)
        out.append((RUST_KEYWORDS.get(name, name), rust_type(ctype)))
    return out


def parse_header():
    text = _strip_comments(HEADER.read_text())
    items = []  # in header order: ("define"|"enum"|"struct"|"opaque"|"alias"|"fnptr"|"fn", ...)
    pos = 0
    pattern = re.compile(
        r"#define\s+(HX_[A-Z0-9_]+)\s+(\d+)u?\s*\n"
        r"|typedef\s+enum\s+(\w+)\s*\{(.*?)\}\s*\w+\s*;"
        r"|typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*\w+\s*;"
        r"|typedef\s+struct\s+(\w+)\s+\w+\s*;"
        r"|typedef\s+void\s*\*\s*(\w+)\s*;"
        r"|typedef\s+const\s+char\s*\*\s*\(\s*\*\s*(\w+)\s*\)\s*\(([^)]*)\)\s*;"
        r"|\n\s*((?:const\s+)?[a-z_][a-z0-9_]*\s*\**)\s*(hx_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;",
        re.S)
    for m in pattern.finditer(text, pos):
        if m.group(1):
            items.append(("define", m.group(1), int(m.group(2))))
        elif m.group(3):
            consts = []
            for entry in m.group(4).split(","):
                entry = entry.strip()
                if entry:
                    k, v = [s.strip() for s in entry.split("=")]
                    consts.append((k, int(v)))
            items.append(("enum", m.group(3), consts))
        elif m.group(5):
            fields = []
            for decl in m.group(6).split(";"):
                decl = " ".join(decl.split())
                if not decl:
                    continue
                fm = re.match(r"^(\w+)\s+(\w+)(?:\[(\w+)\])?$", decl)
                fields.append((fm.group(2), _base(fm.group(1)), fm.group(3)))
            items.append(("struct", m.group(5), fields))
        elif m.group(7):
            items.append(("opaque", m.group(7)))
        elif m.group(8):
            items.append(("alias", m.group(8)))
        elif m.group(9):
            items.append(("fnptr", m.group(9), _split_params(m.group(10))))
        else:
            items.append(("fn", m.group(12), rust_type(m.group(11)), _split_params(m.group(13))))
    return items


def rust_sys_module() -> str:
    items = parse_header()
    defines = {name: value for kind, name, value in (i for i in items if i[0] == "define")}
    lines = [BEGIN, "#![allow(non_camel_case_types, dead_code)]", "use std::os::raw::{c_char, c_void};", ""]
    fns = []
    for it in items:
        kind = it[0]
        if kind == "define":
            lines.append(f"pub const {it[1]}: u32 = {it[2]};")
        elif kind == "enum":
            lines.append("")
            lines.append(f"pub type {it[1]} = i32;")
            for k, v in it[2]:
                lines.append(f"pub const {k}: {it[1]} = {v};")
        elif kind == "struct":
            lines.append("")
            lines.append("#[repr(C)]")
            lines.append("#[derive(Clone, Copy)]")
            lines.append(f"pub struct {it[1]} {{")
            for name, ty, dim in it[2]:
                if dim is not None:
                    n = defines.get(dim, dim)
                    lines.append(f"    pub {name}: [{ty}; {n}],")
                else:
                    lines.append(f"    pub {name}: {ty},")
            lines.append("}")
        elif kind == "opaque":
            lines.append(f"#[repr(C)] pub struct {it[1]} {{ _p: [u8; 0] }}")
        elif kind == "alias":
            lines.append(f"pub type {it[1]} = *mut c_void;")
        elif kind == "fnptr":
            args = ", ".join(f"{n}: {t}" for n, t in it[2])
            lines.append(f"pub type {it[1]} = Option<unsafe extern \"C\" fn({args}) -> *const c_char>;")
        else:
            fns.append(it)
    lines += ["", "#[link(name = \"hephaestus_amd\")]", "extern \"C\" {"]
    for _, name, ret, params in fns:
        args = ", ".join(f"{n}: {t}" for n, t in params)
        tail = "" if ret == "()" else f" -> {ret}"
        lines.append(f"    pub fn {name}({args}){tail};")
    lines += ["}", END]
    return "\n".join(lines)


def _guide_block() -> str:
    text = GUIDE.read_text()
    a, b = text.index(BEGIN), text.index(END) + len(END)
    return text[a:b]


def test_rust_types_of_c_declarations():
    assert rust_type("const void *") == "*const c_void"
    assert rust_type("void **") == "*mut *mut c_void"
    assert rust_type("hx_plan *const *") == "*const *mut hx_plan"
    assert rust_type("void *const *") == "*const *mut c_void"
    assert rust_type("const hx_layout *") == "*const hx_layout"
    assert rust_type("hx_device **") == "*mut *mut hx_device"
    assert rust_type("const char *") == "*const c_char"
    assert rust_type("uint64_t") == "u64" and rust_type("void") == "()"


def test_every_header_entry_point_is_transcribed():
    fns = [it for it in parse_header() if it[0] == "fn"]
    declared = set(re.findall(r"\b(hx_[a-z0-9_]+)\s*\(", _strip_comments(HEADER.read_text())))
    declared -= {"hx_kernel_source_fn"}
    assert {it[1] for it in fns} == declared
    assert len(fns) == len(declared)


def test_guide_carries_the_generated_sys_module():
    assert _guide_block() == rust_sys_module()


if __name__ == "__main__":
    print(rust_sys_module())
