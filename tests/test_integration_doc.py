"""The Rust binding that INTEGRATION.md tells a maintainer to paste into the
reference's FFI crate must match the C ABI it binds: every `#[repr(C)]` struct
field for field (name, type, order), and every `fn axh_*` parameter for
parameter, against the declarations in include/*.h.

The reference-side counterparts are the structs the binding replaces:
VulkanContextOptions (crates/axc-runtime/src/context.rs:76-109) and the
strategy holes (crates/axc-hir/src/hir.rs:62-68).

Types are compared in one canonical spelling: the base type first, then each
pointer level as " *" preceded by " const" when the pointee is const (C
`const void *const *` and Rust `*const *const c_void` are both
`void const * const *`), arrays as `T[N]`.
"""
from __future__ import annotations

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
DOC = ROOT / "INTEGRATION.md"
HEADERS = sorted((ROOT / "include").glob("*.h"))

RUST_BASE = {
    "u8": "uint8_t", "u16": "uint16_t", "u32": "uint32_t", "u64": "uint64_t",
    "i8": "int8_t", "i16": "int16_t", "i32": "int32_t", "i64": "int64_t",
    "usize": "size_t", "f32": "float", "f64": "double", "c_char": "char", "c_void": "void",
    "c_int": "int", "axh_status": "int",
}
C_BASE = {"axh_status": "int"}


def _strip_c(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return "\n".join(ln for ln in text.splitlines() if not ln.lstrip().startswith("#"))


def c_type(decl: str, is_param: bool) -> tuple[str, str]:
    """(name, canonical type) of one C declaration such as
    `const void *const *inputs` or `uint32_t workgroup_size[3]`."""
    decl = decl.strip()
    dims = re.findall(r"\[\s*(\w*)\s*\]", decl)
    decl = re.sub(r"\[[^\]]*\]", "", decl)
    toks = re.findall(r"\w+|\*", decl)
    name = ""
    if len(toks) > 1 and re.fullmatch(r"\w+", toks[-1]) and toks[-1] != "const":
        name = toks.pop()
    # east const: a leading const qualifies the base type
    lead_const = False
    while toks and toks[0] == "const":
        lead_const = True
        toks.pop(0)
    base = toks.pop(0)
    if base in ("unsigned", "signed", "struct", "enum") and toks and toks[0] not in ("*", "const"):
        base = f"{base} {toks.pop(0)}"
    out = [C_BASE.get(base, base)] + (["const"] if lead_const else []) + toks
    t = " ".join(out)
    if dims:
        t = t + " *" if is_param else t + "".join(f"[{d}]" for d in dims)
    return name, t


def rust_type(t: str) -> str:
    t = t.strip()
    m = re.fullmatch(r"\[\s*(.+?)\s*;\s*(\w+)\s*\]", t)
    if m:
        return f"{rust_type(m.group(1))}[{m.group(2)}]"
    quals = []
    while True:
        m = re.match(r"\*\s*(const|mut)\s+", t)
        if not m:
            break
        quals.append(m.group(1))
        t = t[m.end():]
    out = RUST_BASE.get(t, t)
    for q in reversed(quals):
        out += (" const" if q == "const" else "") + " *"
    return out


def header_structs() -> dict[str, list[tuple[str, str]]]:
    out = {}
    for h in HEADERS:
        text = _strip_c(h.read_text())
        for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*\1\s*;", text, flags=re.S):
            fields = []
            for stmt in m.group(2).split(";"):
                stmt = stmt.strip()
                if not stmt:
                    continue
                # `uint32_t n_rows, units, batch` declares three fields of one type
                first, *rest = [s.strip() for s in stmt.split(",")]
                name, t = c_type(first, is_param=False)
                fields.append((name, t))
                base = re.sub(r"\s*\*+.*$", "", t.split("[")[0])
                for r in rest:
                    fields.append(c_type(f"{base} {r}", is_param=False))
            out[m.group(1)] = fields
    return out


def header_functions() -> dict[str, tuple[str, list[str]]]:
    out = {}
    for h in HEADERS:
        text = _strip_c(h.read_text())
        text = text.replace('extern "C" {', " ")
        for stmt in re.split(r"[;{}]", text):
            stmt = " ".join(stmt.split())
            if stmt.startswith("typedef"):
                continue
            m = re.fullmatch(r"(.*?)\b(axh_\w+)\s*\((.*)\)", stmt)
            if not m or not m.group(1).strip():
                continue
            ret = c_type(m.group(1), is_param=True)[1] if m.group(1).strip() != "void" else "void"
            params = [p for p in (s.strip() for s in m.group(3).split(",")) if p and p != "void"]
            out[m.group(2)] = (ret, [c_type(p, is_param=True)[1] for p in params])
    return out


def _split_top(s: str) -> list[str]:
    parts, depth, cur = [], 0, ""
    for ch in s:
        depth += ch in "[("
        depth -= ch in "])"
        if ch == "," and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += ch
    parts.append(cur)
    return [p.strip() for p in parts if p.strip()]


def doc_structs(text: str) -> dict[str, list[list[tuple[str, str]]]]:
    """Every `#[repr(C)] [pub] struct NAME { fields }` in the document (a name
    may appear more than once); opaque handles (`_p: [u8; 0]`) are left out."""
    out: dict[str, list] = {}
    pat = r"#\[repr\(C\)\]\s*(?:pub\s+)?struct\s+(\w+)\s*\{(.*?)\}"
    for m in re.finditer(pat, text, flags=re.S):
        fields = []
        for f in _split_top(m.group(2)):
            fm = re.fullmatch(r"(?:pub\s+)?(\w+)\s*:\s*(.+)", f, flags=re.S)
            assert fm, f"unparsed field {f!r} of {m.group(1)}"
            fields.append((fm.group(1), rust_type(" ".join(fm.group(2).split()))))
        if [n for n, _ in fields] == ["_p"]:
            continue
        out.setdefault(m.group(1), []).append(fields)
    return out


def doc_functions(text: str) -> dict[str, list[tuple[str, list[str]]]]:
    out: dict[str, list] = {}
    pat = r"\bfn\s+(axh_\w+)\s*\((.*?)\)\s*(?:->\s*([^;{]+?))?\s*;"
    for m in re.finditer(pat, text, flags=re.S):
        params = []
        for p in _split_top(" ".join(m.group(2).split())):
            pm = re.fullmatch(r"(\w+)\s*:\s*(.+)", p)
            assert pm, f"unparsed parameter {p!r} of {m.group(1)}"
            params.append(rust_type(pm.group(2)))
        ret = rust_type(m.group(3)) if m.group(3) else "void"
        out.setdefault(m.group(1), []).append((ret, params))
    return out


def test_canonical_spellings_agree():
    """The two spellings meet on the forms the binding uses."""
    assert c_type("const void *const *inputs", True) == ("inputs", "void const * const *")
    assert rust_type("*const *const c_void") == "void const * const *"
    assert c_type("void *const *outputs", True)[1] == rust_type("*const *mut c_void")
    assert c_type("axh_context **out", True)[1] == rust_type("*mut *mut axh_context")
    assert c_type("const uint32_t workgroups[3]", True)[1] == rust_type("*const u32")
    assert c_type("uint32_t workgroup_size[3]", False)[1] == rust_type("[u32; 3]")
    assert c_type("const char *dir", False)[1] == rust_type("*const c_char")
    assert c_type("int32_t device_index", False)[1] != rust_type("u32")
    assert c_type("axh_status", True)[1] == rust_type("axh_status")


def test_every_documented_struct_matches_the_header():
    doc = doc_structs(DOC.read_text())
    hdr = header_structs()
    for name in ("axh_context_options", "axh_binding_plan", "axh_q4_variant",
                 "axh_q4_matmul_variant"):
        assert name in doc, f"INTEGRATION.md declares no #[repr(C)] {name}"
    for name, decls in doc.items():
        assert name in hdr, f"INTEGRATION.md declares {name}, which no header defines"
        for fields in decls:
            assert fields == hdr[name], (
                f"INTEGRATION.md's {name} {fields} differs from the header's {hdr[name]}")


def test_every_documented_function_matches_the_header():
    doc = doc_functions(DOC.read_text())
    hdr = header_functions()
    assert len(doc) >= 10
    for name, decls in doc.items():
        assert name in hdr, f"INTEGRATION.md binds {name}, which no header declares"
        for ret, params in decls:
            assert (ret, params) == hdr[name], (
                f"INTEGRATION.md's {name} {ret} {params} differs from the header's {hdr[name]}")


def test_documented_abi_version_matches(axc):
    m = re.search(r"pub const AXH_ABI_VERSION: u32 = (\d+);", DOC.read_text())
    h = re.search(r"#define AXH_ABI_VERSION (\d+)u", (ROOT / "include" / "axh.h").read_text())
    assert m and h and int(m.group(1)) == int(h.group(1))
    assert axc.load_library().axh_abi_version() == int(h.group(1))


def test_the_four_field_variant_is_rejected():
    """The check catches the slip it was written for: the 4-field
    axh_q4_variant of an older binding."""
    old = ("#[repr(C)]\npub struct axh_q4_variant { pub rows_per_wave: u32, "
           "pub waves_per_workgroup: u32,\n pub prefetch: u32, pub nontemporal: u32 }\n")
    fields = doc_structs(old)["axh_q4_variant"][0]
    assert fields != header_structs()["axh_q4_variant"]
    assert [n for n, _ in header_structs()["axh_q4_variant"]][-2:] == ["family", "sb_per_lane"]


@pytest.mark.parametrize("name", ["axh_bench_op", "axh_check_report", "axh_gguf_tensor_info"])
def test_header_struct_parser_reads_every_field(name):
    """Multi-name declarations and arrays are split into single fields."""
    fields = header_structs()[name]
    assert len(fields) >= 3 and all(n and t for n, t in fields)
    if name == "axh_bench_op":
        assert [n for n, _ in fields][8:11] == ["n_rows", "units", "batch"]
