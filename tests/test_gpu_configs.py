"""The benchmark configurations at their full sizes on the GPU, and the LayerNorm forms each
pass size and width selects, against the oracle (the C++ restatement of the reference CPU path).

- GPT-2 medium shape (24 layers, d 1,024, 16 heads, d_ff 4,096): 256 windows of 256 Zipf(1.1)
  tokens folded in one call, 32 payloads spread over the slots equal to the CPU fast path's,
  and every block
  unfolded back to its tokens (crates/taco/src/gpu_fold.rs:205-306, gpu_unfold.rs:74-300).
- GPT-2 XL shape (48 layers, d 1,600, 25 heads, d_ff 6,400): 512 windows of 512 tokens, 16
  payloads spread over the slots equal to the CPU's.
- Decode attention at 64 streams x 12 heads x 64 over caches of 128, 512 and 1,024 positions.
- One- and two-layer models at d 1,024 and 1,600, version-2 ("wide") models and a model with
  |beta| > 256, each through a pass of fewer than 4,096 rows and one of at least 4,096 rows.
"""

import ctypes as C
import time

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import splitmix_tokens

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def dev():
    from taco_amd import hip
    return hip.HipDevice.open(0)


def _windows(tokens, n, sel):
    return [tokens[w * n:(w + 1) * n] for w in sel]


def _cpu_payloads(om, blocks, n):
    return O.fold_payloads(om, np.concatenate(blocks), len(blocks), n, chunk=32,
                           threads=min(16, len(blocks)))


def _spread(total, count, seed):
    """count window indices over 0..total-1: evenly spaced (the first and the last included)
    plus seeded random ones, so slot-, group-order- and offset-dependent errors show."""
    even = np.linspace(0, total - 1, count // 2).round().astype(int).tolist()
    rng = np.random.default_rng(seed)
    rest = [int(x) for x in rng.permutation(total) if int(x) not in even][:count - len(even)]
    return sorted(even + rest)


def test_gpt2_medium_fold_and_unfold_round_trip(dev):
    from taco_amd import fold, hip, synth
    t0 = time.time()
    mb = synth.build_model(synth.GPT2_MEDIUM)
    W, n = 256, 256
    tokens = synth.zipf_tokens(W * n)
    _log(f"medium: model {len(mb)} B and tokens built in {time.time() - t0:.1f}s")
    hm = hip.HipModel.load(dev, mb)
    batch = hip.HipBatch(hm, W, W * n)
    blocks = _windows(tokens, n, range(W))
    t0 = time.time()
    got = fold.fold_blocks(batch, blocks)
    _log(f"medium: fold of {W} x {n} in {time.time() - t0:.2f}s")
    sel = _spread(W, 32, 4)
    om = O.Model(mb)
    want = _cpu_payloads(om, _windows(tokens, n, sel), n)
    for i, w in enumerate(sel):
        assert got[w] == want[i], f"window {w}: the GPU payload differs from the CPU's"
    t0 = time.time()
    back = fold.unfold_blocks(batch, got, 0, cap=n)
    _log(f"medium: unfold of {W} blocks in {time.time() - t0:.2f}s")
    bad = [w for w in range(W) if not np.array_equal(back[w], blocks[w])]
    assert not bad, f"blocks {bad[:8]} did not round-trip"


def test_gpt2_xl_fold_equals_the_cpu(dev):
    from taco_amd import fold, hip, synth
    t0 = time.time()
    mb = synth.build_model(synth.GPT2_XL)
    W, n = 512, 512
    tokens = synth.zipf_tokens(W * n)
    _log(f"xl: model {len(mb)} B and tokens built in {time.time() - t0:.1f}s")
    hm = hip.HipModel.load(dev, mb)
    batch = hip.HipBatch(hm, W, W * n)
    t0 = time.time()
    got = fold.fold_blocks(batch, _windows(tokens, n, range(W)))
    _log(f"xl: fold of {W} x {n} in {time.time() - t0:.2f}s")
    del batch
    sel = _spread(W, 16, 5)
    om = O.Model(mb)
    want = _cpu_payloads(om, _windows(tokens, n, sel), n)
    for i, w in enumerate(sel):
        assert got[w] == want[i], f"window {w}: the GPU payload differs from the CPU's"


def _dev_buf(dev, arr):
    from taco_amd import hip
    p = C.c_void_p()
    hip._check(hip.lib().hs_device_alloc(dev.h, arr.nbytes, C.byref(p)))
    hip._check(hip.lib().hs_device_upload(dev.h, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes))
    return p


@pytest.mark.parametrize("ctx_len", [128, 512, 1024])
def test_attend_decode_at_the_benchmark_shape(dev, ctx_len):
    """64 streams x 12 heads x 64 with every stream at ctx_len positions (the decode attention
    workload), plus a second call with ragged lengths, against the oracle."""
    from taco_amd import hip
    r = np.random.default_rng(ctx_len)
    B, H, hd = 64, 12, 64
    q = r.integers(-127, 128, (B, H, hd)).astype(np.int8)
    kc = r.integers(-127, 128, (B, H, ctx_len, hd)).astype(np.int8)
    vc = r.integers(-127, 128, (B, H, ctx_len, hd)).astype(np.int8)
    table = np.array([round(2 ** 30 * np.exp(-i / 256)) for i in range(8192)], np.int32)
    score_m, score_s, out_m, out_s = 1_400_000_000, 33, 1_300_000_000, 53
    for ctx in (np.full(B, ctx_len, np.uint32),
                r.integers(1, ctx_len + 1, B).astype(np.uint32)):
        want = O.attend_decode_ref(q, kc, vc, ctx, score_m, score_s, out_m, out_s, table, 30)
        bufs = [_dev_buf(dev, a) for a in (q, kc, vc, ctx, table)]
        out = np.zeros((B, H * hd), np.int8)
        dout = _dev_buf(dev, out)
        try:
            hip._check(hip.lib().hs_op_attend_decode_dev(
                dev.h, bufs[0], bufs[1], bufs[2], bufs[3], B, H, hd, ctx_len, score_m, score_s,
                out_m, out_s, bufs[4], len(table), 30, dout, None))
            hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                    out.nbytes))
        finally:
            for p in bufs + [dout]:
                hip.lib().hs_device_free(dev.h, p)
        assert np.array_equal(out, want)


@pytest.mark.parametrize("ctx_len", [128, 1024])
def test_attend_decode_sets_timing(dev, ctx_len):
    """hs_op_attend_decode_sets_gpu_ns (the attend-decode bench's timing: one launch per cache set,
    back to back) launches on every set in turn: the output is the last set's attention, and a
    call with no sets is refused."""
    from taco_amd import hip
    r = np.random.default_rng(7 + ctx_len)
    B, H, hd, sets = 64, 12, 64, 3
    q = r.integers(-127, 128, (B, H, hd)).astype(np.int8)
    ctx = r.integers(1, ctx_len + 1, B).astype(np.uint32)
    table = np.array([round(2 ** 30 * np.exp(-i / 256)) for i in range(8192)], np.int32)
    score_m, score_s, out_m, out_s = 1_400_000_000, 34, 1_300_000_000, 53
    caches = [(r.integers(-127, 128, (B, H, ctx_len, hd)).astype(np.int8),
               r.integers(-127, 128, (B, H, ctx_len, hd)).astype(np.int8)) for _ in range(sets)]
    bufs = [_dev_buf(dev, a) for a in (q, ctx, table)]
    cbufs = [(_dev_buf(dev, k), _dev_buf(dev, v)) for k, v in caches]
    out = np.zeros((B, H * hd), np.int8)
    dout = _dev_buf(dev, out)
    dks = (C.c_void_p * sets)(*[k for k, _ in cbufs])
    dvs = (C.c_void_p * sets)(*[v for _, v in cbufs])
    ns = C.c_uint64()
    try:
        hip._check(hip.lib().hs_op_attend_decode_sets_gpu_ns(
            dev.h, bufs[0], dks, dvs, sets, bufs[1], B, H, hd, ctx_len, score_m, score_s, out_m,
            out_s, bufs[2], len(table), 30, dout, C.byref(ns)))
        hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                out.nbytes))
        st = hip.lib().hs_op_attend_decode_sets_gpu_ns(
            dev.h, bufs[0], dks, dvs, 0, bufs[1], B, H, hd, ctx_len, score_m, score_s, out_m,
            out_s, bufs[2], len(table), 30, dout, C.byref(ns))
    finally:
        for p in bufs + [dout] + [p for kv in cbufs for p in kv]:
            hip.lib().hs_device_free(dev.h, p)
    want = O.attend_decode_ref(q, caches[-1][0], caches[-1][1], ctx, score_m, score_s, out_m,
                               out_s, table, 30)
    assert np.array_equal(out, want)
    assert ns.value > 0
    assert st == hip.HS_INVALID_ARGUMENT


@pytest.mark.parametrize("B,H,ctx_len", [(256, 12, 200), (200, 16, 64), (171, 12, 256)])
def test_attend_decode_wave_per_head(dev, B, H, ctx_len):
    """Decode attention with at least 2,048 row-heads and at most 256 keys (a GPT-2-medium
    unfold pass: 256 slots x 16 heads) takes the wave-per-row-head kernel: full and ragged
    contexts against the oracle."""
    from taco_amd import hip
    r = np.random.default_rng(B * H + ctx_len)
    hd = 64
    q = r.integers(-127, 128, (B, H, hd)).astype(np.int8)
    kc = r.integers(-127, 128, (B, H, ctx_len, hd)).astype(np.int8)
    vc = r.integers(-127, 128, (B, H, ctx_len, hd)).astype(np.int8)
    table = np.array([round(2 ** 30 * np.exp(-i / 256)) for i in range(8192)], np.int32)
    score_m, score_s, out_m, out_s = 1_400_000_000, 33, 1_300_000_000, 53
    ragged = r.integers(1, ctx_len + 1, B).astype(np.uint32)
    ragged[:3] = [1, ctx_len, min(65, ctx_len)]
    for ctx in (np.full(B, ctx_len, np.uint32), ragged):
        want = O.attend_decode_ref(q, kc, vc, ctx, score_m, score_s, out_m, out_s, table, 30)
        bufs = [_dev_buf(dev, a) for a in (q, kc, vc, ctx, table)]
        out = np.zeros((B, H * hd), np.int8)
        dout = _dev_buf(dev, out)
        try:
            hip._check(hip.lib().hs_op_attend_decode_dev(
                dev.h, bufs[0], bufs[1], bufs[2], bufs[3], B, H, hd, ctx_len, score_m, score_s,
                out_m, out_s, bufs[4], len(table), 30, dout, None))
            hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                    out.nbytes))
        finally:
            for p in bufs + [dout]:
                hip.lib().hs_device_free(dev.h, p)
        assert np.array_equal(out, want)


# LayerNorm forms by pass size and width: fewer than 4,096 rows take a one-wave workgroup per
# row (4 or 8 column groups per lane); at least 4,096 rows take the 16-lanes-per-row form for
# d <= 1,024 (12 or 16 groups; single-precision element rule for 8-bit outputs with |beta| <=
# 256, the integer rule otherwise, two planes for a 16-bit ln_f) and the 4-rows-per-workgroup
# wave form for 1,024 < d <= 2,048.
LN_MODELS = {
    "d1024": dict(dims=(2, 16, 1024, 4096), kw={}),
    "d1600": dict(dims=(1, 25, 1600, 6400), kw={}),
    "d768_wide": dict(dims=(2, 12, 768, 3072), kw=dict(wide=True)),
    "d1024_wide": dict(dims=(1, 16, 1024, 4096), kw=dict(wide=True)),
    "d768_beta": dict(dims=(2, 12, 768, 3072), kw=dict(beta_max=1000)),
    "d1024_beta": dict(dims=(1, 16, 1024, 4096), kw=dict(beta_max=1000)),
}


@pytest.mark.parametrize("name", sorted(LN_MODELS))
@pytest.mark.parametrize("windows,n", [(8, 128), (32, 128), (33, 127)])
def test_layernorm_forms_equal_the_cpu(dev, name, windows, n):
    """`windows` x `n`-token windows in one pass: 1,024 rows (the decode-size form), 4,096 rows
    (the prefill forms) or 4,191 (their last workgroup partial), every interval against the CPU
    fast path's."""
    from taco_amd import hip, synth
    L, H, d, f = LN_MODELS[name]["dims"]
    V = 512
    mb = synth.build_model(synth.Dims(L, H, d, f, vocab=V, n_ctx=256), seed=0x1F00 + d,
                           **LN_MODELS[name]["kw"])
    hm, om = hip.HipModel.load(dev, mb), O.Model(mb)
    blocks = [np.array(splitmix_tokens(0x5EED + w, n, V - 1), np.uint32) for w in range(windows)]
    batch = hip.HipBatch(hm, windows, windows * n)
    inputs, queries = [], []
    for w, blk in enumerate(blocks):
        inputs += [(w, V - 1)] + [(w, int(t)) for t in blk[:-1]]
        queries += [(0, int(t)) for t in blk]
    raw = batch.run_coded_raw(inputs, queries, 32).reshape(windows, n, 3)
    for w in sorted({0, 3, windows - 1}):
        want = O.fast_window_intervals(om, blocks[w], chunk=32)
        bad = np.nonzero(np.any(raw[w] != want, axis=1))[0]
        assert len(bad) == 0, f"{name}, window {w}: {len(bad)} rows differ, first {bad[:8].tolist()}"


# Split-K products in decode-shaped passes: passes of at most 512 rows whose mlp.c_proj has
# K = d_ff > 4,096 run k_gemm<Raw> partials over K slices and the summing pass k_split_epi with
# the Residual rule (GPT-2 XL's mlp.c_proj, K 6,400, in every unfold pass).
SPLIT_MODELS = {"d256_f6400": (1, 4, 256, 6400), "d1600_f6400": (1, 25, 1600, 6400)}


@pytest.mark.parametrize("name", sorted(SPLIT_MODELS))
def test_split_k_residual_passes_equal_the_cpu(dev, name):
    """4 windows of 128 tokens: a first pass of 4 x 96 rows (384 rows, 12 or more K slices),
    then one row per slot per pass (4-row passes, 16 slices), every interval against the CPU
    fast path's."""
    from taco_amd import hip, synth
    L, H, d, f = SPLIT_MODELS[name]
    V, n, W, first = 512, 128, 4, 96
    mb = synth.build_model(synth.Dims(L, H, d, f, vocab=V, n_ctx=256), seed=0x5B11 + d)
    hm, om = hip.HipModel.load(dev, mb), O.Model(mb)
    blocks = [np.array(splitmix_tokens(0x7E57 + w, n, V - 1), np.uint32) for w in range(W)]
    feed = [[V - 1] + [int(t) for t in blk[:-1]] for blk in blocks]
    batch = hip.HipBatch(hm, W, 512)
    got = [[] for _ in range(W)]
    inputs, queries = [], []
    for w in range(W):
        inputs += [(w, t) for t in feed[w][:first]]
        queries += [(0, int(t)) for t in blocks[w][:first]]
    raw = batch.run_coded_raw(inputs, queries, 32).reshape(W, first, 3)
    for w in range(W):
        got[w].extend(raw[w])
    for pos in range(first, n):
        raw = batch.run_coded_raw([(w, feed[w][pos]) for w in range(W)],
                                  [(0, int(blocks[w][pos])) for w in range(W)], 32)
        for w in range(W):
            got[w].append(raw[w])
    for w in range(W):
        want = O.fast_window_intervals(om, blocks[w], chunk=32)
        g = np.array(got[w])
        bad = np.nonzero(np.any(g != want, axis=1))[0]
        assert len(bad) == 0, f"{name}, window {w}: {len(bad)} rows differ, first {bad[:8].tolist()}"


# Passes of more than 12,288 rows at d 768 (a last 64-row tile partly filled) through both forms
# of the residual epilogue and both LayerNorm element rules.
LARGE_PASS_MODELS = {
    "narrow": {},                                # shifts >= 31: the i32 rescale form
    "general": dict(residual_target=1 << 18),    # shifts below 31: the general rescale form
    "beta_1000": dict(beta_max=1000),            # |beta| > 256: the integer LayerNorm element rule
}


@pytest.mark.parametrize("name", sorted(LARGE_PASS_MODELS))
def test_large_pass_residual_forms_equal_the_cpu(dev, name):
    """97 windows of 127 tokens in one pass (12,319 rows), every interval of sampled windows
    against the CPU fast path's."""
    from taco_amd import hip, synth
    V, n, W = 512, 127, 97
    mb = synth.build_model(synth.Dims(2, 12, 768, 3072, vocab=V, n_ctx=256), seed=0xF05E,
                           **LARGE_PASS_MODELS[name])
    hm, om = hip.HipModel.load(dev, mb), O.Model(mb)
    blocks = [np.array(splitmix_tokens(0xAB00 + w, n, V - 1), np.uint32) for w in range(W)]
    batch = hip.HipBatch(hm, W, W * n)
    inputs, queries = [], []
    for w, blk in enumerate(blocks):
        inputs += [(w, V - 1)] + [(w, int(t)) for t in blk[:-1]]
        queries += [(0, int(t)) for t in blk]
    raw = batch.run_coded_raw(inputs, queries, 32).reshape(W, n, 3)
    for w in (0, 1, 48, 95, 96):
        want = O.fast_window_intervals(om, blocks[w], chunk=32)
        bad = np.nonzero(np.any(raw[w] != want, axis=1))[0]
        assert len(bad) == 0, f"{name}, window {w}: {len(bad)} rows differ, first {bad[:8].tolist()}"
