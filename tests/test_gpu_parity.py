"""GPU parity: the HIP path through the C ABI against the oracle and the reference's golden
vectors. Every comparison is bit-exact."""

import hashlib
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import GOLDEN, splitmix_tokens
from tests.test_oracle import (GOLDEN_MODEL, GOLDEN_OUTPUT, GOLDEN_OVERLAP_OUTPUT, read_container,
                               vocab_of, weights_hash)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from taco_amd import hip
    return hip.HipDevice.open(0)


@pytest.fixture(scope="module")
def golden(dev):
    from taco_amd import hip
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64)
    assert hashlib.sha256(b).hexdigest() == GOLDEN_MODEL
    return b, hip.HipModel.load(dev, b), O.Model(b)


# The CUDA matmul test shapes (crates/hardshell-cuda/tests/ops.rs:29-60): (rows, cols, inputs).
GEMM_SHAPES = [(1, 1, 1), (3, 5, 2), (64, 64, 1), (65, 63, 7), (128, 128, 128), (300, 64, 17),
               (768, 768, 9), (2304, 768, 256), (1000, 64, 513), (50, 3072, 33)]


@pytest.mark.parametrize("n,k,m", GEMM_SHAPES)
def test_gemm_i8_is_the_exact_product(dev, n, k, m):
    from taco_amd import hip
    print(f"gemm n={n} k={k} m={m}", flush=True)
    r = np.random.default_rng(n * 7919 + k * 31 + m)
    w = r.integers(-128, 128, (n, k)).astype(np.int8)
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    got = hip.matmul_i8(dev, w, a)
    want = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(got, want)


def test_gemm_i8_worst_case_at_the_bound(dev):
    # kernels.rs:112-119: 2^16 products of (-128) * (-128) sum to exactly 2^30.
    from taco_amd import hip
    k = 1 << 16
    w = np.full((3, k), -128, np.int8)
    a = np.full((2, k), -128, np.int8)
    a[1, ::2] = 127
    got = hip.matmul_i8(dev, w, a)
    assert got[0].tolist() == [1 << 30] * 3
    assert got[1].tolist() == [(k // 2) * (-128 * 127) + (k // 2) * (1 << 14)] * 3


@pytest.mark.parametrize("n,k,m,splits", [
    (2304, 768, 256, 3), (1024, 4096, 256, 16), (768, 3072, 100, 7), (65, 63, 7, 2),
    (3, 1000, 2, 16), (300, 64 * 9 + 1, 17, 4), (2304, 768, 512, 2), (50, 3072, 33, 1)])
def test_gemm_i8_split_is_the_exact_product(dev, n, k, m, splits):
    """matmul_i8_split (crates/hardshell-cuda/src/ops.rs:163-184): K in `splits` slices, the
    i32 partials summed on the GPU, equal to the exact product (slices of unequal length, K
    below 64 per slice, the worst case of one slice)."""
    from taco_amd import hip
    print(f"gemm split n={n} k={k} m={m} splits={splits}", flush=True)
    r = np.random.default_rng(n * 131 + k * 7 + m + splits)
    w = r.integers(-128, 128, (n, k)).astype(np.int8)
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    got = hip.matmul_i8_split(dev, w, a, splits)
    want = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(got, want)


def test_gemm_i8_split_worst_case_at_the_bound(dev):
    """kernels.rs:112-119: 2^16 products of (-128) * (-128) sum to exactly 2^30 in 16 slices."""
    from taco_amd import hip
    k = 1 << 16
    w = np.full((70, k), -128, np.int8)
    a = np.full((3, k), -128, np.int8)
    a[1, ::2] = 127
    got = hip.matmul_i8_split(dev, w, a, 16)
    assert got[0].tolist() == [1 << 30] * 70
    assert got[1].tolist() == [(k // 2) * (-128 * 127) + (k // 2) * (1 << 14)] * 70


@pytest.mark.parametrize("n,k,m,splits", [(64, 64, 1, 1), (300, 768, 40, 1), (1024, 3072, 256, 8),
                                          (77, 1000, 5, 3)])
def test_gemm_i8_i16_is_the_exact_product(dev, n, k, m, splits):
    """matmul_i8_i16 (ops.rs:220-282, kernels::matvec_i8_i16): i16 activations as two i8 planes,
    one product of 2m rows, exact i64 (the i16 extremes included)."""
    from taco_amd import hip
    r = np.random.default_rng(n + 3 * k + m)
    w = r.integers(-128, 128, (n, k)).astype(np.int8)
    a = r.integers(-32768, 32768, (m, k)).astype(np.int16)
    a[0, :3] = [-32768, 32767, -1]
    got = hip.matmul_i8_i16(dev, w, a, splits)
    want = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(got, want)


def test_gemm_requant_c1_shape(dev):
    # The c_attn linear at GPT-2-small shape: A [256, 768], W [2304, 768], per-channel m, one s.
    from taco_amd import hip
    r = np.random.default_rng(1)
    a = r.integers(-127, 128, (256, 768)).astype(np.int8)
    w = r.integers(-127, 128, (2304, 768)).astype(np.int8)
    bias = r.integers(-(1 << 16), 1 << 16, 2304).astype(np.int32)
    mult = r.integers(1 << 30, 1 << 31, 2304).astype(np.int64).astype(np.int32)
    for shift in (42, 0, 1, 30, 31, 32, 62, 63, 64, 95, 96):
        got = hip.gemm_requant_i8(dev, w, a, bias, mult, shift)
        want = O.linear_act_ref(w, a, bias, mult, shift)
        assert np.array_equal(got, want), shift
    # negative multipliers and extremes
    mult2 = r.integers(-(1 << 31), 1 << 31, 2304).astype(np.int64).astype(np.int32)
    mult2[:4] = [-(1 << 31), (1 << 31) - 1, 0, -1]
    got = hip.gemm_requant_i8(dev, w, a, bias, mult2, 40)
    assert np.array_equal(got, O.linear_act_ref(w, a, bias, mult2, 40))


@pytest.mark.parametrize("m,n,k", [(1, 100, 64), (130, 700, 128), (700, 2304, 768), (16384, 768, 768),
                                   (257, 1000, 192), (512, 3072, 1024), (511, 1000, 4096),
                                   (300, 1030, 4100)])
def test_gemm_requant_tile_shapes(dev, m, n, k):
    # Shapes whose rounds favour the 128 x 192 tiles (partial tiles in M and N included) and the
    # 256 x 128 ones, the 64 x 64 tiles of passes of at most 512 rows (K up to 4,096, partial
    # tiles in M and N), and a K just past them (split into slices), against the exact rule.
    from taco_amd import hip
    r = np.random.default_rng(m * 7 + n)
    a = r.integers(-127, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    bias = r.integers(-(1 << 16), 1 << 16, n).astype(np.int32)
    mult = r.integers(-(1 << 31), 1 << 31, n).astype(np.int64).astype(np.int32)
    rows = min(m, 1024)  # the oracle's rows (the first 1,024)
    got = hip.gemm_requant_i8(dev, w, a, bias, mult, 38)
    assert np.array_equal(got[:rows], O.linear_act_ref(w, a[:rows], bias, mult, 38))
    if m > rows:  # the last rows (the partial tiles) too
        assert np.array_equal(got[-rows:], O.linear_act_ref(w, a[-rows:], bias, mult, 38))


def test_gemm_requant_at_the_narrow_bound(dev):
    # The epilogue keeps rescaled values in i32 when the host shows |acc + bias| < 2^31 and the
    # shift is at least 31: operands at that bound (|acc| = 768 2^14, |bias| = 2^31 - 1 - 768 2^14)
    # with the extreme multipliers, at shifts 30 .. 33, against the exact rule.
    from taco_amd import hip
    k = 768
    a = np.zeros((4, k), np.int8)
    a[0], a[1], a[2], a[3] = 127, -128, 1, -1
    w = np.zeros((256, k), np.int8)
    w[0::4], w[1::4], w[2::4], w[3::4] = 127, -128, -127, 0
    big = (1 << 31) - 1 - k * (1 << 14)
    bias = np.resize(np.array([big, -big, big, -big, 0], np.int64), 256).astype(np.int32)
    mult = np.resize(np.array([-(1 << 31), (1 << 31) - 1, 1 << 30, -1, 12345], np.int64), 256).astype(np.int32)
    for shift in (30, 31, 32, 33):
        got = hip.gemm_requant_i8(dev, w, a, bias, mult, shift)
        assert np.array_equal(got, O.linear_act_ref(w, a, bias, mult, shift)), shift


def test_golden_output_hash_on_gpu(golden):
    # crates/hardshell/tests/gpt2.rs:203-226 through the GPU step path (150 tokens, 1 restart).
    from taco_amd import hip
    _, hm, _ = golden
    s = hip.HipSession(hm)
    rows = [s.start_block()] + [s.step(t) for t in splitmix_tokens(0x7AC0_0002, 150, 300)]
    assert weights_hash(rows) == GOLDEN_OUTPUT


def test_golden_overlap_hash_on_gpu(golden):
    # crates/hardshell/tests/context.rs:321-353: overlap 32, 300 tokens, 8 restarts.
    from taco_amd import hip
    _, hm, _ = golden
    s = hip.HipSession(hm, overlap=32)
    rows = [s.start_block()] + [s.step(t) for t in splitmix_tokens(0x7AC0_0002, 300, 300)]
    assert weights_hash(rows) == GOLDEN_OVERLAP_OUTPUT


@pytest.mark.parametrize("max_rows", [2, 5, 40, 64, 200])
def test_prefill_passes_equal_the_reference(golden, max_rows):
    # Prefill of 151 rows in passes of max_rows (crates/hardshell-cuda/tests/gpt2.rs:33-112).
    from taco_amd import hip
    _, hm, om = golden
    toks = splitmix_tokens(0x7AC0_0002, 150, 300)
    s = O.Session(om)
    want = np.array([s.start_block()] + [s.step(t) for t in toks])
    b = hip.HipBatch(hm, 1, max_rows)
    got = b.run_weights([(0, 299)] + [(0, t) for t in toks])
    assert np.array_equal(got, want)
    assert b.position(0) == s.position()  # two restarts at n_ctx 64


def test_batch_of_slots_equals_independent_sessions(golden):
    from taco_amd import hip
    _, hm, om = golden
    slots = 5
    seqs = [splitmix_tokens(100 + s, 40 + 7 * s, 299) for s in range(slots)]
    want = []
    for seq in seqs:
        s = O.Session(om)
        want.append([s.start_block()] + [s.step(t) for t in seq[:-1]])
    b = hip.HipBatch(hm, slots, 97)
    # interleave: each call gives every slot a run of its next tokens
    got = [[] for _ in range(slots)]
    done = [0] * slots
    while any(done[s] < len(seqs[s]) for s in range(slots)):
        inputs, owner = [], []
        for s in range(slots):
            take = min(len(seqs[s]) - done[s], 3 + s)
            for i in range(done[s], done[s] + take):
                tok = 299 if i == 0 else seqs[s][i - 1]
                inputs.append((s, tok))
                owner.append(s)
            done[s] += take
        w = b.run_weights(inputs)
        for o, row in zip(owner, w):
            got[o].append(row)
    for s in range(slots):
        assert np.array_equal(np.array(got[s]), np.array(want[s])), s


def test_coded_intervals_equal_from_weights(golden):
    from taco_amd import hip
    _, hm, om = golden
    toks = splitmix_tokens(0x5EED, 63, 300)
    s = O.Session(om)
    weights = [s.start_block()] + [s.step(t) for t in toks[:-1]]
    b = hip.HipBatch(hm, 1, 64)
    inputs = [(0, 299)] + [(0, t) for t in toks[:-1]]
    enc = b.run_coded(inputs, [(0, t) for t in toks], 32)
    for i, (w, iv) in enumerate(zip(weights, enc)):
        st, fr = O.freq_interval(w, 32, toks[i])
        assert (iv.symbol, iv.start, iv.freq) == (toks[i], st, fr), i
        assert iv.is_last == (st + fr == 1 << 32)
    # decode queries: targets 0, T/3, T-1 and random ones, and a smaller total (freq_bits 20)
    r = np.random.default_rng(2)
    for bits in (32, 20, 9):
        targets = [0, (1 << bits) // 3, (1 << bits) - 1] + [int(x) for x in r.integers(0, 1 << bits, 60)]
        b.reset(0)
        dec = b.run_coded(inputs, [(1, targets[i % len(targets)]) for i in range(len(inputs))], bits)
        for i, (w, iv) in enumerate(zip(weights, dec)):
            t = targets[i % len(targets)]
            assert (iv.symbol, iv.start, iv.freq) == O.freq_find(w, bits, t), (bits, i)


def test_refusals_keep_positions(golden):
    from taco_amd import hip
    _, hm, _ = golden
    b = hip.HipBatch(hm, 2, 8)
    b.run_weights([(0, 299), (0, 5)])
    with pytest.raises(hip.BadSlot):
        b.run_weights([(0, 1), (2, 1)])
    with pytest.raises(hip.ModelError) as e:
        b.run_weights([(0, 1), (1, 300)])
    assert e.value.kind == "TokenOutOfRange"
    with pytest.raises(hip.Unsupported):
        b.run_coded([(0, 1)], [(0, 300)], 32)
    with pytest.raises(hip.Unsupported):
        b.run_coded([(0, 1)], [(0, 1)], 8)  # 2^8 < vocab
    with pytest.raises(hip.ModelError):
        b.set_overlap(63)
    assert b.position(0) == 2 and b.position(1) == 0


@pytest.mark.parametrize("name", ["predicted_text_k0", "predicted_text_k32", "all_kinds_text"])
def test_conformance_blocks_through_the_gpu_coder(dev, name):
    """The coded blocks of conformance/v2 decode on the GPU (Decode queries, one row per step,
    as gpu_unfold.rs:143-160) and re-encode on the GPU to the same payload bytes."""
    from taco_amd import hip
    hsm = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()
    om = O.Model(hsm)
    hm = hip.HipModel.load(dev, hsm)
    vocab = vocab_of(hsm)
    data = open(os.path.join(GOLDEN, name + ".taco"), "rb").read()
    original = open(os.path.join(GOLDEN, name + ".in"), "rb").read()
    c = read_container(data)
    coded = [(i, p) for i, (k, p) in enumerate(c["blocks"]) if k == 1]
    b = hip.HipBatch(hm, len(coded), 64)
    b.set_overlap(c["overlap"])
    # decode all coded blocks in lockstep, one slot each
    decs, counts, toks = [], [], []
    for _, payload in coded:
        n, used = 0, 0
        shift = 0
        while True:
            byte = payload[used]
            n |= (byte & 0x7F) << shift
            used += 1
            shift += 7
            if byte < 0x80:
                break
        decs.append(O.Decoder(payload[used:]))
        counts.append(n)
        toks.append([])
    nxt = [299] * len(coded)
    while any(len(toks[s]) < counts[s] for s in range(len(coded))):
        live = [s for s in range(len(coded)) if len(toks[s]) < counts[s]]
        ans = b.run_coded([(s, nxt[s]) for s in live], [(1, decs[s].target(32)) for s in live], 32)
        for s, iv in zip(live, ans):
            decs[s].decode_interval(iv.start, iv.freq, 32)
            toks[s].append(iv.symbol)
            nxt[s] = iv.symbol
    for s, (i, payload) in enumerate(coded):
        piece = original[i * c["block_size"]:(i + 1) * c["block_size"]]
        assert b"".join(vocab[t] for t in toks[s]) == piece
        assert O.encode_block(om, toks[s], overlap=c["overlap"]) == payload
    # encode on the GPU: Encode queries over the whole block in one call (prefill)
    b2 = hip.HipBatch(hm, len(coded), 512)
    b2.set_overlap(c["overlap"])
    inputs, queries = [], []
    for s in range(len(coded)):
        seq = toks[s]
        inputs += [(s, 299)] + [(s, t) for t in seq[:-1]]
        queries += [(0, t) for t in seq]
    got = b2.run_coded_raw(inputs, queries, 32)
    pos = 0
    for s, (i, payload) in enumerate(coded):
        n = len(toks[s])
        ops = [[0, int(st), int(fr), 32] for _, st, fr in got[pos:pos + n]]
        pos += n
        body = O.encode_script(ops)
        head = bytearray()
        v = n
        while True:
            lo = v & 0x7F
            v >>= 7
            head.append(lo | (0x80 if v else 0))
            if not v:
                break
        assert bytes(head) + body == payload


@pytest.mark.parametrize("dims", [(1, 3, 60, 100, 300, 40), (1, 2, 40, 64, 260, 30),
                                  (3, 2, 128, 200, 1000, 48)])
def test_odd_dims_equal_the_reference(dev, dims):
    from taco_amd import hip
    b = O.build_model(dims, 9, 16)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    toks = splitmix_tokens(12, dims[5] + 5, dims[4])
    s = O.Session(om)
    want = np.array([s.start_block()] + [s.step(t) for t in toks])
    hb = hip.HipBatch(hm, 1, 13)
    got = hb.run_weights([(0, om.eot)] + [(0, t) for t in toks])
    assert np.array_equal(got, want)


def test_head_dim_not_multiple_of_4_is_unsupported(dev):
    from taco_amd import hip
    b = O.build_model((1, 1, 33, 47, 270, 20), 9, 8)
    with pytest.raises(hip.Unsupported):
        hip.HipModel.load(dev, b)


def _dev_buf(dev, arr):
    from taco_amd import hip
    import ctypes as C
    p = C.c_void_p()
    hip._check(hip.lib().hs_device_alloc(dev.h, arr.nbytes, C.byref(p)))
    hip._check(hip.lib().hs_device_upload(dev.h, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes))
    return p


@pytest.mark.parametrize("ctx_cap,hd,score_s", [
    (320, 64, 33), (1024, 64, 33), (1024, 64, 8), (1100, 64, 33), (1024, 16, 33), (256, 32, 33),
    (512, 128, 33), (700, 256, 33), (320, 48, 33)])
def test_attend_decode_op(dev, ctx_cap, hd, score_s):
    """The decode attention op, smaller than GPT-2's: 8 streams x 12 heads over caches of
    ctx_cap positions. head_dim 64 with at most 1,024 positions takes the one-launch kernel
    (score shift 8: scores clamped at +-2^40), other powers of two and longer caches the
    split-key kernels, 48 the row kernel."""
    import ctypes as C
    from taco_amd import hip
    r = np.random.default_rng(3 + hd)
    B, H = 8, 12
    q = r.integers(-127, 128, (B, H, hd)).astype(np.int8)
    kc = r.integers(-127, 128, (B, H, ctx_cap, hd)).astype(np.int8)
    vc = r.integers(-127, 128, (B, H, ctx_cap, hd)).astype(np.int8)
    ctx = np.array([1, 2, 63, 64, 65, 128, ctx_cap - 20, ctx_cap], np.uint32)
    table = np.array([round(2 ** 30 * np.exp(-i / 256)) for i in range(8192)], np.int32)
    score_m, out_m, out_s = 1_400_000_000, 1_300_000_000, 53
    want = O.attend_decode_ref(q, kc, vc, ctx, score_m, score_s, out_m, out_s, table, 30)
    bufs = [_dev_buf(dev, a) for a in (q, kc, vc, ctx, table)]
    out = np.zeros((B, H * hd), np.int8)
    dout = _dev_buf(dev, out)
    try:
        hip._check(hip.lib().hs_op_attend_decode_dev(
            dev.h, bufs[0], bufs[1], bufs[2], bufs[3], B, H, hd, ctx_cap, score_m, score_s,
            out_m, out_s, bufs[4], len(table), 30, dout, None))
        hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                out.nbytes))
    finally:
        for p in bufs + [dout]:
            hip.lib().hs_device_free(dev.h, p)
    assert np.array_equal(out, want)


@pytest.mark.parametrize("ctx_cap,hd", [(200, 64), (1024, 64), (512, 128), (320, 48)])
def test_attend_decode_table_without_zero_tail(dev, ctx_cap, hd):
    """A 300-entry table whose last entry is nonzero: every key past the table weighs the last
    entry (the index is min(M - score, len - 1), softmax.rs:78-104), through the wave-per-row-head,
    one-launch, split-key and row kernels."""
    import ctypes as C
    from taco_amd import hip
    r = np.random.default_rng(17 + hd)
    B, H = 8, 12
    q = r.integers(-127, 128, (B, H, hd)).astype(np.int8)
    kc = r.integers(-127, 128, (B, H, ctx_cap, hd)).astype(np.int8)
    vc = r.integers(-127, 128, (B, H, ctx_cap, hd)).astype(np.int8)
    ctx = np.array([1, 2, 63, 64, 65, 128, ctx_cap - 20, ctx_cap], np.uint32)
    table = np.array([round(2 ** 30 * np.exp(-i / 64)) for i in range(300)], np.int32)
    assert table[-1] > 0
    score_m, score_s, out_m, out_s = 1_400_000_000, 36, 1_300_000_000, 53
    want = O.attend_decode_ref(q, kc, vc, ctx, score_m, score_s, out_m, out_s, table, 30)
    bufs = [_dev_buf(dev, a) for a in (q, kc, vc, ctx, table)]
    out = np.zeros((B, H * hd), np.int8)
    dout = _dev_buf(dev, out)
    try:
        hip._check(hip.lib().hs_op_attend_decode_dev(
            dev.h, bufs[0], bufs[1], bufs[2], bufs[3], B, H, hd, ctx_cap, score_m, score_s,
            out_m, out_s, bufs[4], len(table), 30, dout, None))
        hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                out.nbytes))
    finally:
        for p in bufs + [dout]:
            hip.lib().hs_device_free(dev.h, p)
    assert np.array_equal(out, want)


def _coder_cases():
    r = np.random.default_rng(11)
    cases = []
    table = np.array([round(2 ** 40 * np.exp(-i / 256)) for i in range(8192)], np.uint64)
    for vocab in (300, 50257, 1000, 257, 1):
        rows = []
        for kind in range(6):
            l = r.integers(-3000, 3000, vocab).astype(np.int64)
            if kind == 1:  # ties at the maximum, far apart (different threads of the op)
                l[r.choice(vocab, size=min(vocab, 5), replace=False)] = 5000
            if kind == 2:  # every logit equal
                l[:] = 7
            if kind == 3:  # the maximum at the last id, a tie at the first
                l[-1] = 9000
                l[0] = 9000
            if kind == 4:  # extremes of the clamped range
                l = r.choice([-(1 << 40), 1 << 40, 0], vocab).astype(np.int64)
            rows.append(l)
        cases.append((vocab, np.array(rows), table))
    # a short table and a table with a flat start (ties among weights for different logits)
    t2 = np.array([1 << 40, 1 << 40, 1 << 39, 5, 1], np.uint64)
    cases.append((700, r.integers(-8, 8, (4, 700)).astype(np.int64), t2))
    # tables of 16,300 and 16,384 weighted entries: the packed histogram forms its bins' byte
    # addresses in 16 bits up to 16,320 weighted bins, and takes the per-symbol path above
    for L in (16300, 16384):
        t4 = np.array([round(2 ** 40 * np.exp(-i / 4096)) for i in range(L)], np.uint64)
        l4 = r.integers(-20000, 20000, (4, 50257)).astype(np.int64)
        l4[2, [7, 50000]] = 30000  # a tie at the maximum
        cases.append((50257, l4, t4))
    # the unpacked compact form (V >= 2^16) on a table without a zero tail
    t5 = np.array([round(2 ** 40 * np.exp(-i / 1024)) for i in range(4096)], np.uint64)
    cases.append((70000, r.integers(-9000, 9000, (3, 70000)).astype(np.int64), t5))
    # a table longer than the compact form allows (the i64 logits kernel)
    t3 = np.array([round(2 ** 40 * np.exp(-i / 2048)) for i in range(20000)], np.uint64)
    l3 = r.integers(-30000, 30000, (6, 3000)).astype(np.int64)
    l3[1, [5, 2999]] = 40000
    cases.append((3000, l3, t3))
    return cases


def test_coder_op_equals_from_weights(dev):
    from taco_amd import hip
    r = np.random.default_rng(12)
    for vocab, logits, table in _coder_cases():
        rows = len(logits)
        weights = []
        for l in logits:
            w = np.zeros(vocab, np.uint64)
            assert O.lib().or_logits_to_weights(O.ptr(l), vocab, O.ptr(table), len(table),
                                                O.ptr(w)) == 0
            weights.append(w)
        for bits in sorted({32, 24, max(1, (vocab - 1).bit_length())}):
            if vocab > 1 << bits:
                continue
            toks = r.integers(0, vocab, rows)
            enc = hip.coder(dev, logits, table, [(0, int(t)) for t in toks], bits)
            for i in range(rows):
                assert tuple(enc[i]) == (toks[i],) + O.freq_interval(weights[i], bits, int(toks[i])), \
                    (vocab, bits, i)
            targets = [0, (1 << bits) - 1] + [int(x) for x in r.integers(0, 1 << bits, rows - 2)]
            dec = hip.coder(dev, logits, table, [(1, t) for t in targets[:rows]], bits)
            for i in range(rows):
                assert tuple(dec[i]) == O.freq_find(weights[i], bits, targets[i]), (vocab, bits, i)


@pytest.mark.parametrize("overlap", [0, 32])
def test_head_dim_64_prefill_equals_the_reference(dev, overlap):
    """head_dim 64 takes the MFMA prefill attention (groups of up to 64 rows of one slot):
    windows shorter and longer than a group, and longer than n_ctx (context restarts)."""
    from taco_amd import fold, hip
    b = O.build_model((2, 2, 128, 256, 500, 160), 21, 16)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    lens = [1, 17, 64, 65, 130, 200, 333]
    blocks = [np.array(splitmix_tokens(40 + i, n, 499), np.uint32) for i, n in enumerate(lens)]
    batch = hip.HipBatch(hm, 4, 512)
    batch.set_overlap(overlap)
    from taco_amd import fold
    got = fold.fold_blocks(batch, blocks, overlap)
    for i, blk in enumerate(blocks):
        print(f"block {i} ({len(blk)} tokens, K {overlap})", flush=True)
        assert got[i] == O.encode_block(om, blk, overlap=overlap), i


@pytest.mark.parametrize("score_target,shift", [(768, 34), (1 << 22, 22), (1 << 23, 21)])
def test_head_dim_64_prefill_score_shifts(dev, score_target, shift):
    """The two prefill attention kernels for head_dim 64 and at most 256 keys: score shifts of 22
    or more (every score and distance an i32) take the short kernel, smaller ones the general
    kernel. Ragged groups (windows of 1 to 300 tokens, n_ctx 256)."""
    from taco_amd import fold, hip, synth
    from tests.test_oracle import read_hsm
    b = synth.build_model(synth.Dims(2, 4, 256, 512, 1000, 256), seed=0x5C0E, score_target=score_target)
    _, ts = read_hsm(b)
    assert ts["h.0.attn.score.rescale"][1] == shift
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    lens = [1, 40, 64, 100, 256, 300]
    blocks = [np.array(splitmix_tokens(90 + i, n, 999), np.uint32) for i, n in enumerate(lens)]
    batch = hip.HipBatch(hm, 4, 512)
    got = fold.fold_blocks(batch, blocks, 0)
    for i, blk in enumerate(blocks):
        print(f"score shift {shift}: block {i} ({len(blk)} tokens)", flush=True)
        assert got[i] == O.encode_block(om, blk, overlap=0), i


@pytest.mark.parametrize("score_mult", [-1_400_000_000, -(1 << 31)])
def test_head_dim_64_prefill_negative_score_multiplier(dev, score_mult):
    """A negative attention score multiplier: the short prefill kernel negates the Q bytes, so
    every score grows with its dot and the row max comes from the largest one; INT32_MIN, whose
    magnitude is not an i32, takes the general kernel. Ragged groups (windows of 1 to 300
    tokens, n_ctx 256)."""
    from taco_amd import fold, hip, synth
    from tests.test_oracle import read_hsm
    b = synth.build_model(synth.Dims(2, 4, 256, 512, 1000, 256), seed=0x5C0E, score_mult=score_mult)
    _, ts = read_hsm(b)
    assert int(ts["h.0.attn.score.rescale"][0][0]) == score_mult
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    lens = [1, 40, 64, 100, 256, 300]
    blocks = [np.array(splitmix_tokens(150 + i, n, 999), np.uint32) for i, n in enumerate(lens)]
    batch = hip.HipBatch(hm, 4, 512)
    got = fold.fold_blocks(batch, blocks, 0)
    for i, blk in enumerate(blocks):
        print(f"score multiplier {score_mult}: block {i} ({len(blk)} tokens)", flush=True)
        assert got[i] == O.encode_block(om, blk, overlap=0), i


@pytest.mark.parametrize("score_target", [768, 1 << 23])
def test_head_dim_64_prefill_up_to_512_keys(dev, score_target):
    """Groups of 257 to 512 keys: the 8-block form of the short prefill kernel (score shift 34)
    and the general kernel with its per-super-block recompute (score shift 21); n_ctx 512, a
    513-token window restarts."""
    from taco_amd import fold, hip, synth
    b = synth.build_model(synth.Dims(2, 4, 256, 512, 1000, 512), seed=0x5C0F, score_target=score_target)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    lens = [257, 300, 420, 512, 513]
    blocks = [np.array(splitmix_tokens(110 + i, n, 999), np.uint32) for i, n in enumerate(lens)]
    batch = hip.HipBatch(hm, 5, 4096)
    got = fold.fold_blocks(batch, blocks, 0)
    for i, blk in enumerate(blocks):
        print(f"score target {score_target}: block {i} ({len(blk)} tokens)", flush=True)
        assert got[i] == O.encode_block(om, blk, overlap=0), i


@pytest.mark.parametrize("overlap", [0, 100])
def test_head_dim_64_long_contexts_equal_the_reference(dev, overlap):
    """More than 256 keys per row (the MFMA prefill kernel recomputes Q K^T per pass for
    contexts past four key blocks), windows longer than n_ctx = 600 (restarts)."""
    from taco_amd import fold, hip
    b = O.build_model((1, 2, 128, 128, 400, 600), 33, 16)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    lens = [257, 320, 599, 600, 900]
    blocks = [np.array(splitmix_tokens(70 + i, n, 399), np.uint32) for i, n in enumerate(lens)]
    batch = hip.HipBatch(hm, 3, 1200)
    batch.set_overlap(overlap)
    got = fold.fold_blocks(batch, blocks, overlap)
    for i, blk in enumerate(blocks):
        print(f"block {i} ({len(blk)} tokens, K {overlap})", flush=True)
        assert got[i] == O.encode_block(om, blk, overlap=overlap), i


def test_read_bw_probe(dev):
    """hs_read_bw (read_gpu_ns, crates/hardshell-cuda/src/ops.rs:328-335): a streaming read of
    256 MiB runs at a plausible HBM rate, and a size that is not a multiple of 16 is refused."""
    import ctypes as C
    from taco_amd import hip
    gbs = hip.read_bw(dev, 256 << 20, 5) / 1e9
    print(f"stream read {gbs:.0f} GB/s", flush=True)
    assert 500 < gbs < 20000
    ns = C.c_uint64()
    assert hip.lib().hs_read_bw(dev.h, 1000, 1, C.byref(ns)) == hip.HS_UNSUPPORTED


def test_model_load_with_reuses_a_loaded_parse(dev, golden):
    """CudaModel::load_with (model.rs:259-349): the bytes of a loaded model give a model with the
    same hash and the same weights; other bytes get their own full load (their hash, their
    refusals)."""
    from taco_amd import hip
    b, hm, om = golden
    again = hip.HipModel.load_with(dev, b, hm)
    assert again.hash() == hm.hash()
    eot = hm.eot_token()
    inputs = [(0, eot), (0, 17), (0, 250)]
    want = hip.HipBatch(hm, 1, 8).run_weights(inputs)
    assert np.array_equal(hip.HipBatch(again, 1, 8).run_weights(inputs), want)
    other = O.build_model(O.tiny_dims(), 0x7AC0_0002, 64)
    m2 = hip.HipModel.load_with(dev, other, hm)
    assert m2.hash() == hashlib.sha256(other).digest()
    bad = bytearray(b)
    bad[0] ^= 1  # the magic
    with pytest.raises(hip.HipError):
        hip.HipModel.load_with(dev, bytes(bad), hm)


def test_run_without_readback_advances_like_run_weights(golden):
    """CudaBatch::run_without_readback (batch.rs:478-484): the same passes and positions as
    run_weights, nothing read back; the next weights equal those of a batch that read back."""
    from taco_amd import hip
    b, hm, om = golden
    eot = hm.eot_token()
    first = [(0, eot), (1, eot), (0, 5), (1, 77)]
    nxt = [(0, 11), (1, 12)]
    a, c = hip.HipBatch(hm, 2, 16), hip.HipBatch(hm, 2, 16)
    a.run_weights(first)
    c.run_without_readback(first)
    assert [c.position(s) for s in range(2)] == [a.position(s) for s in range(2)] == [2, 2]
    assert np.array_equal(c.run_weights(nxt), a.run_weights(nxt))


def test_probe_issue(dev):
    """hs_probe_issue times every op and refuses the ones it does not have."""
    from taco_amd import hip
    for op in range(7):
        assert hip.probe_issue(dev, op, 1, 64) > 0
    for op in (7, 8):  # the mixed forms run two waves per SIMD
        assert hip.probe_issue(dev, op, 2, 64) > 0
    with pytest.raises(hip.HipError):
        hip.probe_issue(dev, 9, 1, 64)
    with pytest.raises(hip.HipError):
        hip.probe_issue(dev, 7, 1, 64)
    with pytest.raises(hip.HipError):
        hip.probe_issue(dev, 0, 9, 64)


def test_kernel_resources(dev):
    """CudaDevice::kernel_resources (device.rs:65-74): every listed kernel has a name and
    registers; the main GEMM loop does not spill."""
    from taco_amd import hip
    res = hip.kernel_resources(dev)
    print(res, flush=True)
    assert len(res) >= 20 and all(name and regs > 0 for name, regs, _, _ in res)
    by = {name: (regs, priv) for name, regs, priv, _ in res}
    # the GEMM forms of the fold keep everything in registers (no private memory)
    for name in ("k_gemm<Act, narrow, 256x128>", "k_gemm<Residual, narrow, 256x128>",
                 "k_gemm<Residual, narrow, 256x256>", "k_gemm<Gelu, narrow, 256x256>",
                 "k_gemm<LogitsCompact, narrow, 256x128>", "k_gemm<Act, narrow, 128x192>",
                 "k_gemm<Residual, narrow, 128x192>"):
        assert by[name][1] == 0, name
