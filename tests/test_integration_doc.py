"""The Rust backend source integration/hip_be.rs (the `src/hip_be.rs` a HOS maintainer adds) matches
the C ABI it binds and the `Gpu` surface it replaces:
- its `HosPeftCfg` has the fields of include/hos_hip.h's `hos_peft_cfg` in the same order with the same C types,
  and so does the ctypes mirror (hos_amd/_lib.py PeftCfg) the tests use;
- its `extern "C"` block declares every function of the header with the same argument names and C types, in
  order, and the same return type;
- every method of the reference stub's `impl Gpu` / `impl GpuRunner` (src/metal_be_stub.rs:35-208, 213-236) and its
  free functions exist with the same parameter types and return type (checked when the reference tree is present);
- every `fn hos_*` quoted in INTEGRATION.md exists in the header.
A binding built from the file therefore passes arguments of the library's layout. CPU only."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = os.path.join(ROOT, "INTEGRATION.md")
RS = os.path.join(ROOT, "integration", "hip_be.rs")
HEADER = os.path.join(ROOT, "include", "hos_hip.h")
STUB = "/root/reference/src/metal_be_stub.rs"

C_OF_RUST = {"c_int": "int", "f32": "float", "u32": "uint32_t", "i32": "int32_t", "usize": "size_t", "u64": "uint64_t",
             "f64": "double", "i64": "long long", "c_char": "char", "c_void": "void", "u8": "uint8_t",
             "HosCtx": "hos_ctx", "HosPeft": "hos_peft", "HosFt": "hos_ft", "HosPeftCfg": "hos_peft_cfg"}
CTYPES_OF_C = {"int": ctypes.c_int, "float": ctypes.c_float, "uint32_t": ctypes.c_uint32}


def c_of_rust(t):
    """'*const f32' -> 'const float*', '*mut *mut HosCtx' -> 'hos_ctx**', 'c_int' -> 'int'."""
    t = t.strip()
    stars, const = 0, False
    while t.startswith("*"):
        stars += 1
        if t.startswith("*const "):
            const = stars == 1 if not const else const
            t = t[7:]
        else:
            t = t[5:]
        t = t.strip()
    # only the innermost pointer's constness is expressible as a leading `const`
    inner_const = const and stars >= 1
    return ("const " if inner_const else "") + C_OF_RUST[t] + "*" * stars


def norm_c(t):
    return " ".join(t.replace("*", " * ").split()).replace(" *", "*")


def rust_struct():
    text = open(RS).read()
    m = re.search(r"pub struct HosPeftCfg \{(.*?)\n\}", text, re.S)
    assert m, "hip_be.rs declares no HosPeftCfg"
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


def c_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    text = re.sub(r"typedef struct \{.*?\}\s*\w+;", "", text, flags=re.S)
    text = re.sub(r"enum \{.*?\};", "", text, flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"([\w\s\*]+?)\b(hos_\w+)\s*\(([^)]*)\)\s*;", text):
        ret = norm_c(ret.strip().split("\n")[-1])
        params = []
        for a in " ".join(args.split()).split(","):
            m = re.match(r"(.*?)(\w+)$", a.strip())
            params.append((m.group(2), norm_c(m.group(1))))
        out[name] = (ret, params)
    return out


def rust_externs():
    text = open(RS).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, re.S).group(1)
    out = {}
    for name, args, ret in re.findall(r"pub fn (hos_\w+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        params = []
        for a in " ".join(args.split()).split(","):
            if not a.strip():
                continue
            n, t = a.split(":", 1)
            n = n.strip()
            params.append(("in" if n == "in_" else n, norm_c(c_of_rust(t))))
        out[name] = (norm_c(c_of_rust(ret)) if ret else "void", params)
    return out


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


def test_rust_externs_match_header_signatures():
    c, r = c_functions(), rust_externs()
    assert set(c) == set(r), (sorted(set(c) - set(r)), sorted(set(r) - set(c)))
    for name in c:
        assert r[name] == c[name], f"{name}: rust {r[name]} vs header {c[name]}"


def _methods(text, impl):
    """pub fn name -> (param types, return type) of `impl <impl> {...}` (or free functions when impl is None)."""
    if impl:
        m = re.search(r"\nimpl " + impl + r" \{\n(.*?)\n\}", text, re.S)
        body = m.group(1)
    else:
        body = re.sub(r"\nimpl \w+ \{\n.*?\n\}", "", text, flags=re.S)
        body = "\n".join(line for line in body.splitlines() if line.startswith("pub fn"))
    out = {}
    for name, args, ret in re.findall(r"pub fn (\w+)(?:<[^>]*>)?\((.*?)\)\s*(?:->\s*(.*?))?\s*\{", body, re.S):
        types = []
        for a in " ".join(args.split()).split(","):
            a = a.strip()
            if not a or a in ("&self", "self", "&mut self"):
                continue
            types.append(" ".join(a.split(":", 1)[1].split()))
        out[name] = (types, " ".join((ret or "()").split()))
    return out


@pytest.mark.skipif(not os.path.exists(STUB), reason="reference tree not present")
def test_gpu_surface_matches_the_reference_stub():
    stub, ours = open(STUB).read(), open(RS).read()
    for impl in ("Gpu", "GpuRunner", None):
        want, got = _methods(stub, impl), _methods(ours, impl)
        assert want, impl
        for name, sig in want.items():
            assert name in got, f"{impl or 'free fn'}::{name} missing from hip_be.rs"
            assert got[name] == sig, f"{impl or 'free fn'}::{name}: {got[name]} vs the stub's {sig}"


def test_documented_functions_exist_in_header():
    text = open(DOC).read()
    header = open(HEADER).read()
    names = set(re.findall(r"\bfn (hos_\w+)\(", text))
    missing = sorted(n for n in names if not re.search(r"\b" + n + r"\s*\(", header))
    assert not missing, missing


def test_integration_doc_points_at_the_source_file():
    assert "integration/hip_be.rs" in open(DOC).read()
