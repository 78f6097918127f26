"""The Rust binding documented in INTEGRATION.md matches the C ABI it binds: the `HosPeftCfg` struct has the
fields of include/hos_hip.h's `hos_peft_cfg` in the same order with the same C types, and so does the ctypes
mirror (hos_amd/_lib.py PeftCfg) the tests use; every `extern "C"` function the document declares exists in
the header. A binding written from the document therefore passes a struct of the library's size and layout
(no reads or writes past it). CPU only."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")
HEADER = os.path.join(ROOT, "include", "hos_hip.h")

C_OF_RUST = {"c_int": "int", "f32": "float", "u32": "uint32_t", "i32": "int"}
CTYPES_OF_C = {"int": ctypes.c_int, "float": ctypes.c_float, "uint32_t": ctypes.c_uint32}


def rust_struct():
    text = open(DOC).read()
    m = re.search(r"pub struct HosPeftCfg \{(.*?)\n\}", text, re.S)
    assert m, "INTEGRATION.md declares no HosPeftCfg"
    return [(n, C_OF_RUST[t]) for n, t in re.findall(r"pub (\w+): (\w+)", m.group(1))]


def c_struct():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    m = re.search(r"typedef struct \{(.*?)\} hos_peft_cfg;", text, re.S)
    fields = []
    for decl in m.group(1).split(";"):
        decl = decl.strip()
        if not decl:
            continue
        typ, names = decl.split(None, 1)
        fields += [(n.strip(), typ) for n in names.split(",")]
    return fields


def test_rust_struct_matches_header():
    rust, c = rust_struct(), c_struct()
    assert len(c) == 23
    assert rust == c


def test_ctypes_mirror_matches_header():
    from hos_amd._lib import PeftCfg
    got = [(n, t) for n, t in PeftCfg._fields_]
    want = [(n, CTYPES_OF_C[t]) for n, t in c_struct()]
    assert got == want
    assert ctypes.sizeof(PeftCfg) == 4 * len(want)


def test_documented_functions_exist_in_header():
    text = open(DOC).read()
    header = open(HEADER).read()
    names = set(re.findall(r"\bfn (hos_\w+)\(", text))
    assert names, "no extern functions documented"
    missing = sorted(n for n in names if not re.search(r"\b" + n + r"\s*\(", header))
    assert not missing, missing
