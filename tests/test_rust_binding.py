"""The Rust binding hardshell-hip/src/ffi.rs (source only: no cargo here) against the C header
include/hardshell_hip.h: every function the header declares is declared in ffi.rs under the same
name with the same number of parameters, and nothing else is; the status values agree."""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hardshell_hip.h")
FFI = os.path.join(ROOT, "hardshell-hip", "src", "ffi.rs")


def _strip_c_comments(s):
    return re.sub(r"/\*.*?\*/", "", re.sub(r"//[^\n]*", "", s, flags=re.S), flags=re.S)


def _count_params(params):
    params = params.strip()
    if params in ("", "void"):
        return 0
    depth, n = 0, 1
    for ch in params:
        if ch in "([":
            depth += 1
        elif ch in ")]":
            depth -= 1
        elif ch == "," and depth == 0:
            n += 1
    return n


def header_functions():
    src = _strip_c_comments(open(HEADER).read())
    src = re.sub(r"typedef[^;]*;", "", src)  # typedefs (incl. the mixer function pointer type)
    out = {}
    for m in re.finditer(r"\b(hs_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", src):
        out[m.group(1)] = _count_params(m.group(2))
    return out


def rust_functions():
    src = open(FFI).read()
    block = src[src.index('unsafe extern "C" {'):]
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (hs_[a-z0-9_]+)\s*\((.*?)\)\s*(->\s*[^;]+)?;", block, flags=re.S):
        out[m.group(1)] = _count_params(m.group(2).strip().rstrip(","))
    return out


def test_every_header_function_has_its_rust_declaration():
    h, r = header_functions(), rust_functions()
    assert len(h) > 60, sorted(h)
    assert sorted(set(h) - set(r)) == [], "declared in the header, missing in ffi.rs"
    assert sorted(set(r) - set(h)) == [], "declared in ffi.rs, not in the header"
    bad = {k: (h[k], r[k]) for k in h if h[k] != r[k]}
    assert not bad, f"parameter counts differ (header, ffi.rs): {bad}"


def test_status_values_agree():
    src = _strip_c_comments(open(HEADER).read())
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"HS_([A-Z_]+)\s*=\s*(\d+)", src)}
    rs = open(FFI).read()
    enum = rs[rs.index("pub enum Status"):]
    enum = enum[:enum.index("}")]
    r = {m.group(1): int(m.group(2)) for m in re.finditer(r"(\w+)\s*=\s*(\d+)", enum)}
    camel = {"OK": "Ok", "NO_DEVICE": "NoDevice", "DEVICE_ERROR": "DeviceError", "UNSUPPORTED": "Unsupported",
             "MODEL_ERROR": "ModelError", "BAD_SLOT": "BadSlot", "LENGTH_MISMATCH": "LengthMismatch",
             "INVALID_ARGUMENT": "InvalidArgument"}
    for name, rust in camel.items():
        assert c[name] == r[rust], (name, c[name], r[rust])
    for name in ("MIX_NONE", "MIX_PLAIN"):
        cv = int(re.search(r"#define HS_%s (0x[0-9A-Fa-f]+)u" % name, open(HEADER).read()).group(1), 16)
        rv = int(re.search(r"pub const HS_%s: u32 = (0x[0-9A-F_]+);" % name, rs).group(1).replace("_", ""), 16)
        assert cv == rv, name
