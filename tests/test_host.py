"""Host-side checks that need no GPU: the C-ABI libraries load and export every entry point the
headers declare, the model loader accepts and refuses .hsm files as the reference reader does
(the cases of crates/hardshell/tests/hsm.rs, on conformance/tiny.hsm), the Python .hsm writer
rewrites tiny.hsm byte for byte, and the synthetic workload is pinned by its hashes."""

import ctypes as C
import hashlib
import json
import os
import re

import numpy as np
import pytest

from tests.conftest import GOLDEN

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TINY = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()

HS_OK, HS_NO_DEVICE, HS_MODEL_ERROR = 0, 1, 4
KIND = dict(INVALID_SHAPE=1, BAD_MAGIC=4, UNSUPPORTED_VERSION=5, TRUNCATED=6, HEADER_NOT_UTF8=7,
            HEADER_JSON=8, INVALID_HEADER=9, LAYOUT=10, NON_ZERO_PADDING=11, VOCABULARY=12,
            MISSING_TENSOR=13, UNEXPECTED_TENSOR=14, TENSOR_MISMATCH=15)


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:hs|tc)_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("lib,header", [("libhardshell_hip.so", "hardshell_hip.h"),
                                        ("libtaco_hip.so", "taco_hip.h")])
def test_library_exports_every_declared_symbol(lib, header):
    path = os.path.join(ROOT, "taco_amd", lib)
    if not os.path.exists(path):
        pytest.fail(f"{lib} is not built (run __graft_entry__.build())")
    if lib == "libtaco_hip.so":
        C.CDLL(os.path.join(ROOT, "taco_amd", "libhardshell_hip.so"))
    L = C.CDLL(path)
    names = declared(header)
    assert len(names) > (40 if lib.startswith("libhardshell") else 2)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def hs():
    from taco_amd import hip
    return hip.lib()


def test_no_device_is_reported_as_no_device():
    """NoDevice means "use another backend" (crates/taco/src/backend.rs:288-309)."""
    h = C.c_void_p()
    st = hs().hs_device_open(0, C.byref(h))
    if st == HS_OK:
        hs().hs_device_close(h)
        pytest.skip("a GPU is present")
    assert st == HS_NO_DEVICE


def validate(data: bytes):
    """(status, model error kind, sha256) of hs_model_validate."""
    buf = np.frombuffer(data or b"\0", np.uint8).copy()
    out = (C.c_uint8 * 32)()
    st = hs().hs_model_validate(buf.ctypes.data_as(C.c_void_p), len(data), out)
    return st, (hs().hs_last_error_code() if st == HS_MODEL_ERROR else 0), bytes(out)


def refused(data: bytes, *kinds):
    st, kind, _ = validate(data)
    assert st == HS_MODEL_ERROR, "accepted"
    assert kind in [KIND[k] for k in kinds], (kind, kinds)


def header_len(f):
    return int.from_bytes(f[12:16], "little")


def header_value(f):
    return json.loads(f[16:16 + header_len(f)])


def rebuild(orig, edit_value=lambda v: None, edit_text=lambda t: t):
    """orig with a changed header; every section moves by a multiple of 64 bytes, so the layout
    stays canonical unless the edit changes it."""
    base = header_value(orig)
    voff = base["vocabulary"]["offset"]
    for k in range(64):
        v = json.loads(json.dumps(base))
        sh = 64 * k
        v["vocabulary"]["offset"] += sh
        if "merges" in v:
            v["merges"]["offset"] += sh
        for t in v["tensors"]:
            t["offset"] += sh
        edit_value(v)
        text = edit_text(json.dumps(v, separators=(",", ":"), ensure_ascii=False)).encode()
        room = voff + sh - 16
        if len(text) <= room:
            return (orig[:12] + room.to_bytes(4, "little") + text + b" " * (room - len(text))
                    + orig[voff:])
    raise AssertionError("the header does not fit")


def test_tiny_hsm_is_accepted_with_its_hash():
    st, _, h = validate(TINY)
    assert st == HS_OK
    assert h.hex() == hashlib.sha256(TINY).hexdigest()
    assert h.hex().startswith("eb78b89a")
    assert validate(rebuild(TINY))[0] == HS_OK


def test_bad_magic_and_version():
    f = bytearray(TINY)
    f[0] = ord("X")
    refused(bytes(f), "BAD_MAGIC")
    f = bytearray(TINY)
    f[8] = 3
    refused(bytes(f), "UNSUPPORTED_VERSION")
    v = header_value(TINY)
    assert TINY[8] == 1 and "ln_f_bits" not in v["model"]["constants"]
    f = bytearray(TINY)
    f[8] = 2  # version 2 with no part that needs it
    refused(bytes(f), "INVALID_HEADER")


def test_every_truncation_is_refused():
    n = len(TINY)
    lengths = sorted(set(list(range(0, 300)) + list(range(0, n, 997)) + [n - 64, n - 2, n - 1]))
    for k in lengths:
        assert validate(TINY[:k])[0] == HS_MODEL_ERROR, k


def test_trailing_bytes_are_refused():
    refused(TINY + b"\0", "LAYOUT")


def test_floats_and_negatives_in_the_header_are_refused():
    refused(rebuild(TINY, lambda v: v["model"].__setitem__("n_layer", 2.0)), "HEADER_JSON")
    refused(rebuild(TINY, edit_text=lambda t: t.replace('"eot_token":299', '"eot_token":299e0')),
            "HEADER_JSON")
    eps = header_value(TINY)["model"]["constants"]["ln_eps"]
    refused(rebuild(TINY, edit_text=lambda t: t.replace(f'"ln_eps":{eps}', f'"ln_eps":{eps}.0')),
            "HEADER_JSON")
    refused(rebuild(TINY, lambda v: v["tensors"][0].__setitem__(
        "shape", [float(x) for x in v["tensors"][0]["shape"]])), "HEADER_JSON")
    refused(rebuild(TINY, lambda v: v["model"].__setitem__("n_head", -4)), "HEADER_JSON")
    refused(rebuild(TINY, edit_text=lambda t: t.replace('"n_head":4', '"n_head":18446744073709551616')),
            "HEADER_JSON")


def test_unknown_missing_and_duplicate_fields_are_refused():
    refused(rebuild(TINY, lambda v: v["model"].__setitem__("dropout", 0)), "HEADER_JSON")
    refused(rebuild(TINY, lambda v: v.__setitem__("extra", 1)), "HEADER_JSON")
    refused(rebuild(TINY, lambda v: v["model"].pop("d_ff")), "HEADER_JSON")
    refused(rebuild(TINY, edit_text=lambda t: t.replace('"n_layer":2', '"n_layer":2,"n_layer":2')),
            "HEADER_JSON")
    refused(rebuild(TINY, lambda v: v["tensors"][1].__setitem__("scale", 1)), "HEADER_JSON")


def test_a_header_that_is_not_utf8_is_refused():
    g = rebuild(TINY, edit_text=lambda t: t.replace('"gpt2"', '"gpté"'))
    pos = g.index(b"\xc3\xa9")
    g2 = bytearray(g)
    g2[pos] = 0xFF
    refused(bytes(g2), "HEADER_NOT_UTF8")
    refused(g, "INVALID_HEADER")  # the valid UTF-8 form is refused for its name


def test_bad_model_fields_are_refused():
    for edit in (lambda v: v["model"].__setitem__("eot_token", 300),
                 lambda v: v["model"].__setitem__("vocab_size", 0),
                 lambda v: v["model"]["constants"].__setitem__("ln_k", 49),
                 lambda v: v["model"]["constants"].__setitem__("ln_eps", 0),
                 lambda v: v["model"]["constants"].__setitem__("softmax_p", 31),
                 lambda v: v["model"].__setitem__("architecture", "GPT2"),
                 lambda v: v["tensors"][0].__setitem__("name", "")):
        refused(rebuild(TINY, edit), "INVALID_HEADER")


def test_bad_tensor_entries_are_refused():
    t0 = header_value(TINY)["tensors"][0]  # wte [300, 64] i8
    assert t0["name"] == "wte" and t0["shape"] == [300, 64]
    bad = ("TENSOR_MISMATCH", "INVALID_SHAPE")
    refused(rebuild(TINY, lambda v: v["tensors"][0].__setitem__("dtype", "f32")), *bad)
    refused(rebuild(TINY, lambda v: v["tensors"][0].__setitem__("shape", [300, 32, 2]),
                    lambda t: t.replace("[300,32,2]", "[300,32,3]")), *bad)
    refused(rebuild(TINY, lambda v: v["tensors"][0].__setitem__("shape", [19200, 0])), *bad)
    refused(rebuild(TINY, lambda v: v["tensors"][0].__setitem__("shape", [])), *bad)
    refused(rebuild(TINY, lambda v: v["tensors"][0].__setitem__("shift", 3)), *bad)
    refused(rebuild(TINY, lambda v: v["tensors"][1].__setitem__("length", 4)), *bad, "LAYOUT")
    refused(rebuild(TINY, lambda v: v["tensors"][1].__setitem__("name", "wte")),
            "UNEXPECTED_TENSOR")


def test_a_non_canonical_layout_is_refused():
    def move(i, dlt):
        def f(v):
            v["tensors"][i]["offset"] += dlt
        return f
    refused(rebuild(TINY, move(1, 64)), "LAYOUT")
    refused(rebuild(TINY, move(1, -64)), "LAYOUT")
    refused(rebuild(TINY, lambda v: v["vocabulary"].__setitem__("offset", v["vocabulary"]["offset"] + 64)),
            "LAYOUT")
    refused(rebuild(TINY, move(3, 1)), "LAYOUT")


def test_non_zero_padding_is_refused():
    v = header_value(TINY)
    t = v["tensors"][1]  # the gap after wte.rescale_embed
    end = t["offset"] + t["length"]
    nxt = v["tensors"][2]["offset"]
    assert end < nxt
    g = bytearray(TINY)
    g[end] = 1
    refused(bytes(g), "NON_ZERO_PADDING")
    hl = header_len(TINY)
    if 16 + hl < v["vocabulary"]["offset"]:
        g = bytearray(TINY)
        g[16 + hl] = 1
        refused(bytes(g), "NON_ZERO_PADDING")


def test_a_bad_vocabulary_is_refused():
    voff = header_value(TINY)["vocabulary"]["offset"]
    g = bytearray(TINY)
    g[voff] = 200  # a token length that runs past the section
    g[voff + 1] = 200
    refused(bytes(g), "VOCABULARY", "LAYOUT")
    refused(rebuild(TINY, lambda v: v["model"].__setitem__("vocab_size", 299)),
            "VOCABULARY", "LAYOUT", "INVALID_HEADER", "TENSOR_MISMATCH")


def read_hsm(data):
    from tests.test_oracle import read_hsm as rd
    return rd(data)


def test_python_writer_rewrites_tiny_hsm():
    """crates/hardshell/tests/hsm_merges.rs:246-261: parse and rewrite give the same bytes."""
    from taco_amd.hsm_writer import HsmWriter
    hdr, tensors = read_hsm(TINY)
    m = hdr["model"]
    c = m["constants"]
    w = HsmWriter(n_layer=m["n_layer"], n_head=m["n_head"], d_model=m["d_model"], d_ff=m["d_ff"],
                  vocab_size=m["vocab_size"], n_ctx=m["n_ctx"], eot_token=m["eot_token"],
                  ln_k=c["ln_k"], ln_j=c["ln_j"], ln_eps=c["ln_eps"], softmax_p=c["softmax_p"],
                  architecture=m["architecture"])
    vo, vl = hdr["vocabulary"]["offset"], hdr["vocabulary"]["length"]
    toks, p = [], vo
    while p < vo + vl:
        n = int.from_bytes(TINY[p:p + 2], "little")
        toks.append(TINY[p + 2:p + 2 + n])
        p += 2 + n
    w.set_vocabulary(toks)
    if "merges" in hdr:
        mo, ml = hdr["merges"]["offset"], hdr["merges"]["length"]
        raw = np.frombuffer(TINY, "<u4", count=ml // 4, offset=mo).reshape(-1, 2)
        w.set_merges([(int(a), int(b)) for a, b in raw])
    for t in hdr["tensors"]:
        arr, shift = tensors[t["name"]]
        w.add_tensor(t["name"], arr.copy(), shift)
    assert w.finish() == TINY


def test_synthetic_workload_is_pinned():
    """The bench workload: the GPT-2-small-shape model and the 16,384-token Zipf(1.1) stream."""
    from taco_amd import synth
    b = synth.build_model(synth.GPT2_SMALL)
    assert hashlib.sha256(b).hexdigest() == \
        "013358b7e8f7799a6c4cbc2220264b6c4957e4a9e69f5c042d3ae6b543fb795c"
    assert synth.sha256_tokens(synth.zipf_tokens(16384)) == \
        "dd627cc10d96abd5e4f8649b46f3ac1ef238f0415636c7f33a3d51f15b6cc6ce"
    assert validate(b)[0] == HS_OK


SHA_CHECK = r"""
import ctypes as C, hashlib, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from taco_amd import fold
L = fold.lib()
P = lambda a: a.ctypes.data_as(C.c_void_p)
rng = np.random.default_rng(5)
bad = 0
for n in list(range(0, 200)) + [1000, 4095, 4096, 65537, 1 << 20]:
    orig = rng.integers(0, 256, max(n, 1), dtype=np.uint8)
    cnt = (n + 1023) // 1024
    kinds = np.zeros(max(cnt, 1), np.uint8)
    offa = np.zeros(cnt + 1, np.uint64)
    out = np.zeros(200 + 5 * cnt + n, np.uint8)
    L.tc_container_build(P(np.zeros(32, np.uint8)), P(orig), n, 1024, 0, P(kinds), P(orig), P(offa),
                         P(out), len(out))
    bad += out[48:80].tobytes() != hashlib.sha256(orig[:n].tobytes()).digest()
print(bad)
"""


@pytest.mark.parametrize("portable", [False, True])
def test_sha256_of_the_container_equals_hashlib(portable):
    """The original-bytes checksum of the container (crates/taco-format/src/header.rs), with the
    x86 SHA extensions where the CPU has them and with the portable compression."""
    import subprocess
    import sys
    env = dict(os.environ)
    if portable:
        env["HS_SHA256_PORTABLE"] = "1"
    r = subprocess.run([sys.executable, "-c", SHA_CHECK, ROOT], capture_output=True, text=True,
                       env=env, timeout=300)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "0"
