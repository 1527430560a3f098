"""Pins the oracle (oracle/oracle.cpp) to the reference's own golden vectors and to closed
forms. Every oracle function used as a checker has at least one check here that a plausible
mistake (a dropped term, a wrong sign, a transposed operand, an off-by-one) would fail."""

import hashlib
import os
import random

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import GOLDEN, splitmix_tokens

# crates/hardshell/tests/gpt2.rs:224-226
GOLDEN_MODEL = "e3055785bc4509abf7b017e52a0f99030a508cfe0810293e7a5efdccdf2d7bb9"
GOLDEN_OUTPUT = "d4063522517854fdcab605c3d3159bd3ac9a15eb92fa6721ff4a276658f90078"
# crates/hardshell/tests/context.rs:351-353
GOLDEN_OVERLAP_OUTPUT = "5a79928200ad35bb7e7a1be2a0a35e05dcecc001a89cf3cf0765dfc7e5304a83"
# crates/hardshell/tests/wide.rs:275-277
GOLDEN_V2_MODEL = "201f9fd6df4aa0467657380c3890bdb25330510d7253d0fcf5f6cd9211e6af04"
GOLDEN_V2_OUTPUT = "64108429f3ce999899c1df4da4d8c364138b1315143d08d2ab01ab7b2dde2eb8"
# crates/taco-coder/tests/golden.rs:23-27
TABLE_A_SHA256 = "6dce098f222c6f262440d5def6ca5bbb7f1cb34c4cef5a26a19835b77c56ff4d"
STREAM_SHA256 = "91676cdc669fca0eb22ed18f5f629882212523261f41d0d5c568b647e78d798f"
STREAM_LEN = 15_689
# conformance/README.md:12
TINY_HSM_SHA256 = "eb78b89a4f0f17c7245865aed22f86512a49e0272b7583a831c47e1a401418f8"


@pytest.fixture(scope="module")
def golden_model():
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64)
    return b, O.Model(b)


def weights_hash(rows):
    h = hashlib.sha256()
    for w in rows:
        h.update(np.asarray(w, dtype="<u8").tobytes())
    return h.hexdigest()


# ---------------------------------------------------------------------------------------------
# Integer rules: crates/hardshell/src/int.rs:299-363, plus exact big-integer arithmetic.
# ---------------------------------------------------------------------------------------------

def py_rescale(x, m, s, max_shift=95):
    p = x * m
    if s == 0:
        return p
    if s > max_shift:
        return 0
    return (p + (1 << (s - 1))) >> s  # Python >> on ints is a floor


def test_rescale_unit_vectors():
    assert O.rescale(3, 1, 1) == 2
    assert O.rescale(-3, 1, 1) == -1
    assert O.rescale(-5, 1, 1) == -2
    assert O.rescale(5, 1, 0) == 5
    assert O.rescale(7, 3, 2) == 5
    i64min, i32min, i64max, i32max = -(1 << 63), -(1 << 31), (1 << 63) - 1, (1 << 31) - 1
    assert O.rescale(i64min, i32min, 0) == i64min * i32min
    assert O.rescale(i64min, i32min, 94) == 1
    assert O.rescale(i64max, i32max, 255) == 0
    assert O.rescale(i64min, i32max, 200) == 0
    assert O.rescale_wide(-(1 << 94), i32min, 126) == 1
    assert O.rescale_wide(-(1 << 94), i32min, 127) == 0
    assert O.rescale(i64min, i32min, 95) == 1
    assert O.rescale(i64min, i32min, 96) == 0
    assert O.rescale_wide(1 << 94, i32min, 120) == -(1 << 5)


def test_rescale_matches_exact_arithmetic():
    r = random.Random(1)
    for _ in range(4000):
        x = r.choice([r.randrange(-(1 << 63), 1 << 63), r.randrange(-(1 << 33), 1 << 33),
                      r.randrange(-5, 6)])
        m = r.randrange(-(1 << 31), 1 << 31)
        s = r.choice([0, 1, 2, r.randrange(0, 96), r.randrange(0, 256), 62, 63, 64, 95])
        assert O.rescale(x, m, s) == py_rescale(x, m, s), (x, m, s)
        lo, hi = sorted([r.randrange(-(1 << 41), 1 << 41) for _ in range(2)])
        want = max(lo, min(py_rescale(x, m, s), hi))
        assert O.lib().or_rescale_clamp(x, m, s, lo, hi) == want


def test_floor_div_and_isqrt():
    assert O.lib().or_floor_div(-7, 3) == -3
    assert O.lib().or_floor_div(7, 3) == 2
    assert O.lib().or_floor_div(-(1 << 63), 1) == -(1 << 63)
    isq = lambda v: O.lib().or_isqrt_u128(v >> 64, v & ((1 << 64) - 1))
    assert isq(0) == 0 and isq(1) == 1 and isq(3) == 1 and isq(4) == 2
    assert isq((1 << 64) - 1) == (1 << 32) - 1
    assert isq((1 << 128) - 1) == (1 << 64) - 1
    for rr in [1, 2, 1000, 1 << 40, (1 << 63) - 1]:
        assert isq(rr * rr) == rr
        assert isq(rr * rr - 1) == rr - 1
    import math
    r = random.Random(2)
    for _ in range(2000):
        v = r.randrange(0, 1 << r.randrange(1, 128))
        assert isq(v) == math.isqrt(v)


def py_layernorm(x, g, b, m, s, k, j, eps, beta_frac=0, out_max=127):
    n = len(x)
    mean = sum(x) // n
    var = sum((v - mean) ** 2 for v in x) // n
    root = math.isqrt((var << (2 * j)) + eps)
    inv = (1 << k) // max(root, 1)
    out = []
    for v, gg, bb in zip(x, g, b):
        t = (v - mean) * inv * gg
        if beta_frac == 0:
            y = py_rescale(t, m, s, 126) + bb
        else:
            p = t * m + (bb << (s - beta_frac))
            y = 0 if s > 126 else ((p + (1 << (s - 1))) >> s if s else p)
        out.append(max(-out_max, min(out_max, y)))
    return out


import math  # noqa: E402


@pytest.mark.parametrize("beta_frac,bits", [(0, 8), (8, 8), (0, 16), (4, 16)])
def test_layernorm_matches_exact_arithmetic(beta_frac, bits):
    r = np.random.default_rng(3)
    for n in [1, 7, 64, 768]:
        for scale in [1, 1 << 10, (1 << 30) - 1]:
            x = r.integers(-scale, scale + 1, n).astype(np.int32)
            g = r.integers(-(1 << 15), 1 << 15, n).astype(np.int16)
            b = r.integers(-(1 << 20), 1 << 20, n).astype(np.int32)
            m = int(r.integers(1 << 30, 1 << 31))
            s = int(r.integers(60, 90))
            out = np.zeros(n, np.int8 if bits == 8 else np.int16)
            O.lib().or_layernorm(O.ptr(x), n, O.ptr(g), O.ptr(b), m, s, beta_frac, 48, 8,
                                 10_572_336_812_221, bits, O.ptr(out))
            want = py_layernorm([int(v) for v in x], [int(v) for v in g], [int(v) for v in b],
                                m, s, 48, 8, 10_572_336_812_221, beta_frac,
                                127 if bits == 8 else 32767)
            assert out.tolist() == want


def test_layernorm_constant_row_gives_beta():
    # layernorm.rs property: a constant row has x - mean = 0, so y = beta (v1).
    n = 16
    x = np.full(n, 12345, np.int32)
    g = np.arange(n, dtype=np.int16) + 100
    b = np.arange(n, dtype=np.int32) - 8
    out = np.zeros(n, np.int8)
    O.lib().or_layernorm(O.ptr(x), n, O.ptr(g), O.ptr(b), 1 << 30, 70, 0, 48, 8, 1, 8,
                         O.ptr(out))
    assert out.tolist() == list(range(-8, 8))


def test_softmax_and_logit_weights():
    table = np.array([1 << 30, 1 << 29, 1 << 28, 3], np.int32)
    scores = np.array([5, 3, 5, 4, -100], np.int64)
    out = np.zeros(5, np.int64)
    O.lib().or_softmax(O.ptr(scores), 5, O.ptr(table), 4, 30, O.ptr(out))
    e = [1 << 30, 1 << 28, 1 << 30, 1 << 29, 3]
    assert out.tolist() == [(v << 30) // sum(e) for v in e]
    assert out.sum() <= 1 << 30
    lt = np.array([1 << 40, 1 << 39, 7], np.uint64)
    lg = np.array([10, 9, 10, -(1 << 40)], np.int64)
    w = np.zeros(4, np.uint64)
    O.lib().or_logits_to_weights(O.ptr(lg), 4, O.ptr(lt), 3, O.ptr(w))
    assert w.tolist() == [1 << 40, 1 << 39, 1 << 40, 7]


def test_matmul_is_the_exact_product():
    r = np.random.default_rng(4)
    for rows, cols, n in [(1, 1, 1), (5, 17, 3), (33, 768, 7), (4, 65536, 2)]:
        w = r.integers(-128, 128, (rows, cols)).astype(np.int8)
        x = r.integers(-128, 128, (n, cols)).astype(np.int8)
        got = O.matmul_i8(w, x)
        want = x.astype(np.int64) @ w.astype(np.int64).T
        assert np.array_equal(got, want)
    # the worst case at the bound (kernels.rs:112-119): 2^16 products of -128 * -128 = 2^30
    w = np.full((1, 1 << 16), -128, np.int8)
    assert O.matmul_i8(w, w)[0, 0] == 1 << 30


# ---------------------------------------------------------------------------------------------
# Builder and reference session: the conformance hashes.
# ---------------------------------------------------------------------------------------------

def test_golden_model_and_output_hash(golden_model):
    b, m = golden_model
    assert hashlib.sha256(b).hexdigest() == GOLDEN_MODEL
    s = O.Session(m)
    rows = [s.start_block()] + [s.step(t) for t in splitmix_tokens(0x7AC0_0002, 150, 300)]
    assert weights_hash(rows) == GOLDEN_OUTPUT


def test_golden_overlap_hash(golden_model):
    _, m = golden_model
    s = O.Session(m, overlap=32)
    rows = [s.start_block()] + [s.step(t) for t in splitmix_tokens(0x7AC0_0002, 300, 300)]
    assert weights_hash(rows) == GOLDEN_OVERLAP_OUTPUT


def test_golden_version_2_hashes():
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64, wide=True)
    assert hashlib.sha256(b).hexdigest() == GOLDEN_V2_MODEL
    m = O.Model(b)
    assert m.wide
    s = O.Session(m)
    rows = [s.start_block()] + [s.step(t) for t in splitmix_tokens(0x7AC0_0002, 150, 300)]
    assert weights_hash(rows) == GOLDEN_V2_OUTPUT


def test_restart_position_and_refusals(golden_model):
    # crates/hardshell/tests/gpt2.rs:80-99: token 63 restarts; after 2*n_ctx tokens pos is 3.
    _, m = golden_model
    toks = splitmix_tokens(7, 128, 300)
    s = O.Session(m)
    all_rows = [s.start_block()] + [s.step(t) for t in toks]
    fresh = O.Session(m)
    fresh.start_block()
    assert np.array_equal(all_rows[64], fresh.step(toks[63]))
    assert s.position() == 3
    with pytest.raises(ValueError):
        O.Session(m).step(300)


# ---------------------------------------------------------------------------------------------
# Frequency tables and the range coder: taco-coder/src/freq.rs tests and tests/golden.rs.
# ---------------------------------------------------------------------------------------------

def test_freq_unit_vectors():
    assert O.freq_from_weights([1, 2, 3, 4], 4).tolist() == [2, 3, 4, 7]
    assert O.freq_from_weights([3, 3, 1], 3).tolist() == [4, 3, 1]
    assert O.freq_from_weights([0, 0, 0], 2).tolist() == [2, 1, 1]
    assert O.freq_from_weights([0, (1 << 64) - 1, 0], 32).tolist() == [1, (1 << 32) - 2, 1]
    assert O.freq_from_weights([9] * 16, 4).tolist() == [1] * 16
    assert O.freq_from_weights([5], 32).tolist() == [1 << 32]
    with pytest.raises(ValueError):
        O.freq_from_weights([1] * 17, 4)


def py_from_weights(w, bits):
    total = 1 << bits
    W = sum(w)
    largest, best = 0, 0
    for i, v in enumerate(w):
        if v > best:
            best, largest = v, i
    if W == 0:
        w = [1] * len(w)
        W = len(w)
    spare = total - len(w)
    f = [1 + v * spare // W for v in w]
    f[largest] += total - sum(f)
    return f


def test_freq_matches_exact_arithmetic():
    r = random.Random(5)
    for _ in range(200):
        n = r.randrange(1, 300)
        w = [r.choice([0, r.randrange(1 << 40), r.randrange(1 << 64), 7]) for _ in range(n)]
        bits = r.choice([32, 24, max(9, n.bit_length())])
        assert O.freq_from_weights(w, bits).tolist() == py_from_weights(w, bits)
        f = py_from_weights(w, bits)
        starts = np.concatenate([[0], np.cumsum(f)[:-1]]).tolist()
        sym = r.randrange(n)
        assert O.freq_interval(w, bits, sym) == (starts[sym], f[sym])
        t = r.randrange(1 << bits)
        i = max(k for k in range(n) if starts[k] <= t)
        assert O.freq_find(w, bits, t) == (i, starts[i], f[i])


def splitmix_state(s):
    mask = (1 << 64) - 1
    s = (s + 0x9E3779B97F4A7C15) & mask
    z = s
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
    return s, z ^ (z >> 31)


def test_coder_golden_stream():
    # taco-coder/tests/golden.rs:38-102
    s = 0x7AC0_C0DE
    w = []
    for _ in range(1000):
        s, a = splitmix_state(s)
        s, b = splitmix_state(s)
        w.append(a >> (b % 64))
    fa = O.freq_from_weights(w, 24)
    assert hashlib.sha256(fa.astype("<u8").tobytes()).hexdigest() == TABLE_A_SHA256
    fa = fa.tolist()
    sa = np.concatenate([[0], np.cumsum(fa)[:-1]]).tolist()
    ends = np.cumsum(fa).tolist()
    fb = [1, (1 << 32) - 2, 1]
    sb = [0, 1, (1 << 32) - 1]
    ops, s = [], 0x5EED
    import bisect
    script = []
    for _ in range(20000):
        s, x = splitmix_state(s)
        k = x % 8
        if k <= 4:
            t = (x >> 8) % (1 << 24)
            sym = bisect.bisect_right(ends, t)
            ops.append(("A", sym))
            script.append([0, sa[sym], fa[sym], 24])
        elif k == 5:
            sym = (x >> 8) % 3
            ops.append(("B", sym))
            script.append([0, sb[sym], fb[sym], 32])
        else:
            p = (x >> 8) % 4095 + 1
            bit = (x >> 40) % 4096 < p
            ops.append(("bit", p, bit))
            script.append([1, p, int(bit), 0])
    data = O.encode_script(script)
    assert len(data) == STREAM_LEN
    assert hashlib.sha256(data).hexdigest() == STREAM_SHA256
    d = O.Decoder(data)
    for op in ops:
        if op[0] == "bit":
            assert d.decode_bit(op[1]) == op[2]
        else:
            st, fr, bits = (sa, fa, 24) if op[0] == "A" else (sb, fb, 32)
            t = d.target(bits)
            sym = bisect.bisect_right(st, t) - 1
            assert sym == op[1]
            d.decode_interval(st[sym], fr[sym], bits)


# ---------------------------------------------------------------------------------------------
# The committed conformance data: tiny.hsm and the coded conformance/v2 containers.
# ---------------------------------------------------------------------------------------------

def read_container(data):
    """Container v2 (crates/taco-format/src/lib.rs:14-36): header, table, blocks."""
    assert data[:4] == b"TACO" and int.from_bytes(data[4:6], "little") == 2
    block_size = int.from_bytes(data[80:84], "little")
    count = int.from_bytes(data[84:88], "little")
    overlap = int.from_bytes(data[94:96], "little")
    table = [(data[104 + 5 * i], int.from_bytes(data[105 + 5 * i:109 + 5 * i], "little"))
             for i in range(count)]
    pos = 104 + 5 * count
    blocks = []
    for kind, ln in table:
        blocks.append((kind, data[pos:pos + ln]))
        pos += ln
    return dict(block_size=block_size, overlap=overlap, blocks=blocks,
                model_hash=data[8:40], orig_len=int.from_bytes(data[40:48], "little"),
                checksum=data[48:80])


def vocab_of(hsm: bytes):
    import json
    hl = int.from_bytes(hsm[12:16], "little")
    h = json.loads(hsm[16:16 + hl])
    off, n = h["vocabulary"]["offset"], h["model"]["vocab_size"]
    out, p = [], off
    for _ in range(n):
        ln = int.from_bytes(hsm[p:p + 2], "little")
        out.append(hsm[p + 2:p + 2 + ln])
        p += 2 + ln
    return out


@pytest.mark.parametrize("name", ["predicted_text_k0", "predicted_text_k32", "all_kinds_text"])
def test_conformance_coded_blocks_decode_and_reencode(name):
    hsm = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()
    assert hashlib.sha256(hsm).hexdigest() == TINY_HSM_SHA256
    m = O.Model(hsm)
    vocab = vocab_of(hsm)
    data = open(os.path.join(GOLDEN, name + ".taco"), "rb").read()
    original = open(os.path.join(GOLDEN, name + ".in"), "rb").read()
    c = read_container(data)
    assert c["model_hash"] == hashlib.sha256(hsm).digest()
    assert c["checksum"] == hashlib.sha256(original).digest()
    coded = 0
    for i, (kind, payload) in enumerate(c["blocks"]):
        piece = original[i * c["block_size"]:(i + 1) * c["block_size"]]
        if kind != 1:
            continue
        coded += 1
        toks = O.decode_block(m, payload, overlap=c["overlap"])
        assert b"".join(vocab[t] for t in toks) == piece
        again = O.encode_block(m, toks, overlap=c["overlap"])
        assert again == payload
    assert coded >= 2


def test_fast_engine_equals_reference(golden_model):
    _, m = golden_model
    toks = splitmix_tokens(11, 64, 300)
    s = O.Session(m)
    want = [s.start_block()] + [s.step(t) for t in toks[:63]]
    for chunk in [1, 3, 32, 64]:
        got = O.fast_window_weights(m, toks, chunk=chunk)
        assert np.array_equal(got, np.array(want)), chunk


def test_fast_engine_equals_reference_version_2():
    # the golden version-2 model (i16 GELU outputs, 16-bit ln_f, ln_beta_frac), whose reference
    # session output is pinned by GOLDEN_V2_OUTPUT
    m = O.Model(O.build_model(O.tiny_dims(), 0x7AC0_0001, 64, wide=True))
    toks = splitmix_tokens(14, 60, 300)
    s = O.Session(m)
    want = [s.start_block()] + [s.step(t) for t in toks[:-1]]
    for chunk in [1, 5, 32]:
        assert np.array_equal(O.fast_window_weights(m, toks, chunk=chunk), np.array(want)), chunk


@pytest.mark.parametrize("dims", [(1, 3, 60, 100, 300, 40), (2, 1, 33, 47, 270, 20),
                                  (1, 2, 40, 64, 260, 30)])
def test_fast_engine_equals_reference_odd_dims(dims):
    # odd head widths (20, 33) and widths that are not multiples of 16 (fast_paths.rs:140-150)
    m = O.Model(O.build_model(dims, 9, 16))
    toks = splitmix_tokens(12, dims[5], dims[4])
    s = O.Session(m)
    want = [s.start_block()] + [s.step(t) for t in toks[:-1]]
    assert np.array_equal(O.fast_window_weights(m, toks, chunk=7), np.array(want))
    iv = O.fast_window_intervals(m, toks, chunk=5)
    for i, w in enumerate(want):
        assert tuple(iv[i]) == (toks[i],) + O.freq_interval(w, 32, toks[i])


def test_fold_payloads_equal_encode_block(golden_model):
    _, m = golden_model
    toks = np.array(splitmix_tokens(13, 3 * 40, 299), np.uint32)
    got = O.fold_payloads(m, toks, 3, 40, chunk=32, threads=2)
    for w in range(3):
        assert got[w] == O.encode_block(m, toks[w * 40:(w + 1) * 40])


def read_hsm(data: bytes):
    """The header and the tensors of a .hsm file (layout of crates/hardshell/src/hsm/mod.rs):
    8-byte magic, u32 version, u32 header length, the JSON header, aligned sections."""
    import json
    hl = int.from_bytes(data[12:16], "little")
    hdr = json.loads(data[16:16 + hl])
    dts = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "u64": np.uint64}
    tensors = {}
    for t in hdr["tensors"]:
        dt = np.dtype(dts[t["dtype"]])
        a = np.frombuffer(data, dt, count=t["length"] // dt.itemsize, offset=t["offset"])
        tensors[t["name"]] = (a.reshape(t["shape"]), t.get("shift"))
    return hdr, tensors


def test_linear_act_ref_equals_the_session(golden_model):
    """The op-level reference of the C1 GEMM (i8 x i8 -> i32, bias, per-channel rescale, clamp
    to +-127) against block 0's c_attn in the golden-hash-pinned reference session: its input is
    the session's ln_1 output and its output the session's q, k, v."""
    b, om = golden_model
    _, ts = read_hsm(b)
    w, _ = ts["h.0.attn.c_attn.w"]
    bias, _ = ts["h.0.attn.c_attn.b"]
    mult, shift = ts["h.0.attn.c_attn.rescale"]
    s = O.Session(om)
    for i, tok in enumerate([om.eot] + splitmix_tokens(5, 20, om.vocab)):
        pr = s.probe(tok)
        got = O.linear_act_ref(w, pr["ln1"][None, :], bias, mult, shift)[0]
        assert np.array_equal(got, pr["qkv"]), i


def test_attend_decode_ref_equals_the_session(golden_model):
    """The op-level reference of decode attention (config 3) against block 0's attention in the
    reference session: q, k, v of every position from the session's own c_attn output, the
    cache of positions 0..t, the block's score and output rescales and attn_exp."""
    b, om = golden_model
    hdr, ts = read_hsm(b)
    H, d = hdr["model"]["n_head"], hdr["model"]["d_model"]
    hd = d // H
    p = hdr["model"]["constants"]["softmax_p"]
    sm, ss = ts["h.0.attn.score.rescale"]
    omul, osh = ts["h.0.attn.out.rescale"]
    table, _ = ts["attn_exp"]
    toks = [om.eot] + splitmix_tokens(6, 40, om.vocab)
    cap = 48
    kc = np.zeros((1, H, cap, hd), np.int8)
    vc = np.zeros((1, H, cap, hd), np.int8)
    s = O.Session(om)
    for t, tok in enumerate(toks):
        pr = s.probe(tok)
        qkv = pr["qkv"]
        kc[0, :, t, :] = qkv[d:2 * d].reshape(H, hd)
        vc[0, :, t, :] = qkv[2 * d:].reshape(H, hd)
        q = qkv[:d].reshape(1, H, hd)
        got = O.attend_decode_ref(q, kc, vc, np.array([t + 1], np.uint32), int(sm[0]), ss,
                                  int(omul[0]), osh, table, p)[0]
        assert np.array_equal(got, pr["att"]), t
