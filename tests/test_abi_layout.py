"""The C ABI's struct layouts agree across the header and its two bindings.

tests/abi_layout.c is compiled against include/tatara_hip.h with the host C
compiler: its static assertions pin sizes and offsets, and it prints every
field's offset and size.  Those are compared with
  - the fields the header declares (so the program misses none),
  - the ctypes structs of tatara_amd/_lib.py (the Python host mirror),
  - the Rust #[repr(C)] structs the integration guide gives a maintainer: field
    names, order and the layout repr(C) gives them on x86-64 Linux;
and every Rust `extern "C"` function the integration guide binds is checked against
the header's parameter list, type by type.
CPU only.
"""
from __future__ import annotations

import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from tatara_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tatara_hip.h"


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    exe = tmp_path_factory.mktemp("abi") / "abi_layout"
    subprocess.run([cc, "-std=c11", "-Wall", "-Werror", "-o", str(exe), str(ROOT / "tests" / "abi_layout.c")],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    layout: dict[str, dict] = {}
    for line in out.splitlines():
        struct, field, off, size = line.split()
        s = layout.setdefault(struct, {"fields": []})
        if field == "sizeof":
            s["size"] = int(size)
        else:
            s["fields"].append((field, int(off), int(size)))
    return layout


def header_structs() -> dict[str, list[str]]:
    """Field names, in order, of every `typedef struct X { ... } X;` in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, body in re.findall(r"typedef struct (\w+) \{(.*?)\}\s*\1;", text, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            # "float a, b, c" / "const int32_t* p" / "char run_id[257]" / "const struct X* next"
            head, *rest = [d.strip() for d in decl.split(",")]
            first = re.findall(r"(\w+)\s*(?:\[\d+\])?$", head)[0]
            fields += [first] + [re.findall(r"(\w+)", r)[0] for r in rest]
        out[name] = fields
    return out


RUST_TYPES = {"i32": C.c_int32, "u32": C.c_uint32, "i64": C.c_int64, "u64": C.c_uint64, "f32": C.c_float,
              "f64": C.c_double, "u8": C.c_uint8}


def rust_structs() -> dict[str, list[tuple[str, str]]]:
    """(field, type) lists of the #[repr(C)] structs in the integration guide's Rust blocks."""
    text = (ROOT / "INTEGRATION.md").read_text()
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+)\s*\{([^{}]*)\}", text):
        body = re.sub(r"//[^\n]*", "", body)
        fields = re.findall(r"(\w+)\s*:\s*([^,]+?)\s*(?:,|$)", body.replace("\n", " "))
        out[name] = [(f.replace("pub ", "").strip(), t.strip()) for f, t in fields]
    return out


def rust_ctype(t: str):
    if t.startswith("*const") or t.startswith("*mut"):
        return C.c_void_p
    m = re.fullmatch(r"\[\s*(\w+)\s*;\s*(\d+)\s*\]", t)
    if m:
        elem = C.c_char if m.group(1) == "c_char" else RUST_TYPES[m.group(1)]
        return elem * int(m.group(2))
    return RUST_TYPES[t]


def test_layout_program_covers_every_header_field(c_layout):
    for name, fields in header_structs().items():
        assert name in c_layout, f"tests/abi_layout.c does not print {name}"
        assert [f for f, _, _ in c_layout[name]["fields"]] == fields, name


def test_python_ctypes_structs_match_the_header(c_layout):
    checked = 0
    for name, lay in c_layout.items():
        cls = getattr(_lib, name, None)
        assert cls is not None, f"tatara_amd/_lib.py has no {name}"
        assert [f[0] for f in cls._fields_] == [f for f, _, _ in lay["fields"]], name
        for field, off, size in lay["fields"]:
            d = getattr(cls, field)
            assert (d.offset, d.size) == (off, size), f"{name}.{field}"
        assert C.sizeof(cls) == lay["size"], name
        checked += 1
    assert checked >= 9


def test_integration_doc_rust_structs_match_the_header(c_layout):
    rust = rust_structs()
    assert {"TataraTrainerConfig", "TataraLoss", "TataraBatch", "TataraCkptHeader"} <= set(rust), set(rust)
    for name, fields in rust.items():
        if [f for f, _ in fields] == ["_p"]:  # opaque handle
            continue
        lay = c_layout[name]
        assert [f for f, _ in fields] == [f for f, _, _ in lay["fields"]], \
            f"INTEGRATION.md {name}: fields differ from include/tatara_hip.h"
        cls = type(name, (C.Structure,), {"_fields_": [(f, rust_ctype(t)) for f, t in fields]})
        for field, off, size in lay["fields"]:
            d = getattr(cls, field)
            assert (d.offset, d.size) == (off, size), f"INTEGRATION.md {name}.{field}"
        assert C.sizeof(cls) == lay["size"], f"INTEGRATION.md {name}: {C.sizeof(cls)} bytes vs {lay['size']}"


_RUST_SCALARS = {"i32": "int32_t", "u32": "uint32_t", "u64": "uint64_t", "u8": "uint8_t", "f32": "float",
                 "f64": "double", "c_void": "void", "c_char": "char"}


def _rust_param(t: str) -> str:
    """A Rust FFI parameter type as the C type it binds (const-ness kept on the pointee)."""
    t = t.strip()
    if t.startswith("*const "):
        inner = _rust_param(t[len("*const "):])
        return ("const " + inner if "*" not in inner else inner) + "*"
    if t.startswith("*mut "):
        return _rust_param(t[len("*mut "):]) + "*"
    return _RUST_SCALARS.get(t, t)


def _c_param(decl: str) -> str:
    """A C parameter declaration without its name; an array parameter is a pointer."""
    decl = " ".join(decl.split())
    m = re.fullmatch(r"(.*?)(\w+)\s*\[\s*\d*\s*\]", decl)
    if m:
        return _c_param(m.group(1) + "* " + m.group(2))
    return re.sub(r"\b\w+$", "", decl)  # without the parameter name


def _header_functions() -> dict[str, list[str]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"TATARA_API\s+[\w\s\*]+?\b(tatara_\w+)\s*\(([^)]*)\)\s*;", text):
        ps = [p for p in params.split(",") if p.strip() and p.strip() != "void"]
        out[name] = [_c_param(p) for p in ps]
    return out


def test_integration_doc_rust_functions_match_the_header():
    """Every `pub fn tatara_*` the integration guide gives a maintainer has the
    header's parameter list: count, and each type as repr(C) binds it."""
    text = (ROOT / "INTEGRATION.md").read_text()
    header = _header_functions()
    fns = re.findall(r"pub fn (tatara_\w+)\s*\((.*?)\)\s*(?:->\s*([\w\s\*]+?))?\s*;", text, re.S)
    assert len(fns) >= 30, len(fns)
    for name, params, _ in fns:
        assert name in header, f"INTEGRATION.md binds {name}, which the header does not declare"
        rust = [_rust_param(p.split(":", 1)[1]) for p in params.split(",") if p.strip()]
        want = [p.replace(" ", "") for p in header[name]]
        got = [p.replace(" ", "") for p in rust]
        assert got == want, f"{name}: INTEGRATION.md {got} vs header {want}"
