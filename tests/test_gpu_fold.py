"""GPU fold/unfold through the harness (libtaco_hip.so over the C ABI): payloads equal to the
oracle's encode_block, round trips, and the conformance containers rebuilt byte for byte."""

import hashlib
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import GOLDEN, splitmix_tokens
from tests.test_oracle import read_container, vocab_of

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from taco_amd import hip
    return hip.HipDevice.open(0)


def test_two_host_threads_fold_on_two_batches(dev):
    """Two batches of one model folded from two host threads at once (ctypes drops the GIL for
    the call), three rounds each: the kernels' launch-attribute and occupancy caches are shared
    across threads, and every payload must equal the single-threaded fold's."""
    import threading
    from taco_amd import fold, hip, synth
    mb = synth.build_model(synth.Dims(2, 12, 768, 3072, vocab=4096, n_ctx=256), seed=0x2720)
    hm = hip.HipModel.load(dev, mb)
    blocks = [np.array(splitmix_tokens(0x7A1 + w, 200, 4095), np.uint32) for w in range(32)]
    halves = (blocks[:16], blocks[16:])
    want = [fold.fold_blocks(hip.HipBatch(hm, 16, 16 * 200), h) for h in halves]
    batches = [hip.HipBatch(hm, 16, 16 * 200), hip.HipBatch(hm, 8, 1024)]
    got, errors = [[], []], []

    def run(i):
        try:
            for _ in range(3):
                got[i].append(fold.fold_blocks(batches[i], halves[i]))
        except Exception as e:  # surfaced below, on the test's thread
            errors.append((i, e))

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        for r in range(3):
            assert got[i][r] == want[i], f"thread {i}, round {r}: payloads differ"


@pytest.mark.parametrize("overlap", [0, 5, 32])
def test_fold_and_unfold_equal_the_reference(dev, overlap):
    from taco_amd import fold, hip
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    lens = [1, 40, 63, 64, 65, 150, 7]
    blocks = [np.array(splitmix_tokens(900 + i, n, 299), np.uint32) for i, n in enumerate(lens)]
    batch = hip.HipBatch(hm, 4, 300)  # more windows than slots: several waves
    batch.set_overlap(overlap)
    got = fold.fold_blocks(batch, blocks, overlap)
    for i, blk in enumerate(blocks):
        print(f"block {i} ({len(blk)} tokens, K {overlap})", flush=True)
        assert got[i] == O.encode_block(om, blk, overlap=overlap), i
    back = fold.unfold_blocks(batch, got, overlap)
    for i, blk in enumerate(blocks):
        assert np.array_equal(back[i], blk), i


def test_unfold_refills_slots_with_ragged_blocks(dev):
    """Blocks of very different lengths (empty ones among them) on fewer slots than blocks:
    each slot takes the next waiting block when its block ends (gpu_unfold.rs:74-196), with
    restarts inside the backend (lengths past n_ctx = 64), and every block decodes back."""
    from taco_amd import fold, hip
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    lens = [200, 1, 0, 3, 130, 2, 64, 65, 1, 17, 0, 90]
    blocks = [np.array(splitmix_tokens(1300 + i, n, 299), np.uint32) for i, n in enumerate(lens)]
    for overlap in (0, 9):
        payloads = [O.encode_block(om, blk, overlap=overlap) for blk in blocks]
        batch = hip.HipBatch(hm, 3, 64)
        back = fold.unfold_blocks(batch, payloads, overlap, cap=256)
        for i, blk in enumerate(blocks):
            assert np.array_equal(back[i], blk), (overlap, i)


def test_unfold_applies_its_overlap(dev):
    """The overlap argument is the batch's overlap for the decode (a batch left at another
    overlap still decodes the container's blocks), and one that does not fit is refused."""
    from taco_amd import fold, hip
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    blk = np.array(splitmix_tokens(4242, 150, 299), np.uint32)
    payload = O.encode_block(om, blk, overlap=32)
    batch = hip.HipBatch(hm, 2, 64)
    batch.set_overlap(0)
    assert np.array_equal(fold.unfold_blocks(batch, [payload], 32, cap=256)[0], blk)
    with pytest.raises(hip.HipError):
        fold.unfold_blocks(batch, [payload], 63, cap=256)


def test_stop_rule_equals_the_reference(dev):
    """codec.rs:105-112: the encoder stops when the varint plus the lower bound of the coder
    output reach `stop`; a payload of exactly `stop` bytes can still be made (it then loses to
    raw in the container)."""
    from taco_amd import fold, hip
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    blk = np.array(splitmix_tokens(77, 60, 299), np.uint32)
    full = O.encode_block(om, blk)
    stops = [1, 2, len(full) // 2, len(full) - 1, len(full), len(full) + 1, 10 ** 6]
    batch = hip.HipBatch(hm, 3, 128)
    got = fold.fold_blocks(batch, [blk] * len(stops), 0, stop=stops)
    for st, g in zip(stops, got):
        assert g == O.encode_block(om, blk, stop=st), st
    assert got[0] is None and got[-1] == full


@pytest.mark.parametrize("name,k", [("predicted_text_k0", 0), ("predicted_text_k32", 32)])
def test_conformance_container_rebuilt_on_the_gpu(dev, name, k):
    """Decode the golden container's tokens, fold them again on the GPU, and build the
    container: the bytes equal conformance/v2/<name>.taco."""
    from taco_amd import fold, hip
    hsm = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()
    om, hm = O.Model(hsm), hip.HipModel.load(dev, hsm)
    data = open(os.path.join(GOLDEN, name + ".taco"), "rb").read()
    original = open(os.path.join(GOLDEN, name + ".in"), "rb").read()
    c = read_container(data)
    assert c["overlap"] == k
    blocks = [np.array(O.decode_block(om, p, overlap=k), np.uint32) for kind, p in c["blocks"]]
    batch = hip.HipBatch(hm, 3, 512)
    batch.set_overlap(k)
    payloads = fold.fold_blocks(batch, blocks, k)
    out = fold.container(hm.hash(), original, c["block_size"], k, payloads)
    assert out == data
    back = fold.unfold_blocks(batch, payloads, k)
    vocab = vocab_of(hsm)
    assert b"".join(b"".join(vocab[t] for t in blk) for blk in back) == original


def test_gpt2_small_shape_windows_equal_the_cpu_fast_path(dev):
    """Four 256-token windows of the GPT-2-small-shape synthetic model (the bench workload):
    GPU payloads equal the oracle's fast path (itself equal to the reference session)."""
    from taco_amd import fold, hip, synth
    mb = synth.build_model(synth.GPT2_SMALL)
    tokens = synth.zipf_tokens(64 * 256)
    assert synth.sha256_tokens(tokens) == \
        "dd627cc10d96abd5e4f8649b46f3ac1ef238f0415636c7f33a3d51f15b6cc6ce"
    hm = hip.HipModel.load(dev, mb)
    om = O.Model(mb)
    sel = [0, 1, 37, 63]
    blocks = [tokens[w * 256:(w + 1) * 256] for w in sel]
    batch = hip.HipBatch(hm, 4, 1024)
    got = fold.fold_blocks(batch, blocks)
    want = O.fold_payloads(om, np.concatenate(blocks), 4, 256, chunk=32, threads=4)
    assert got == want
    # the intervals of one window, row by row, against the fast path's
    iv = O.fast_window_intervals(om, blocks[2], chunk=32)
    inputs = [(0, 50256)] + [(0, int(t)) for t in blocks[2][:-1]]
    b1 = hip.HipBatch(hm, 1, 256)
    raw = b1.run_coded_raw(inputs, [(0, int(t)) for t in blocks[2]], 32)
    assert np.array_equal(raw, iv)


@pytest.mark.parametrize("max_rows", [16384, 4096, 2688])
def test_bench_shape_intervals_equal_the_cpu_fast_path(dev, max_rows):
    """The benchmark's shape: 64 windows x 256 tokens in one run_coded call (one pass of 16,384
    rows, or passes of max_rows), against the CPU fast path's intervals for sampled windows."""
    from taco_amd import hip, synth
    mb = synth.build_model(synth.GPT2_SMALL)
    tokens = synth.zipf_tokens(64 * 256)
    hm, om = hip.HipModel.load(dev, mb), O.Model(mb)
    batch = hip.HipBatch(hm, 64, max_rows)
    inputs, queries = [], []
    for w in range(64):
        blk = tokens[w * 256:(w + 1) * 256]
        inputs += [(w, 50256)] + [(w, int(t)) for t in blk[:-1]]
        queries += [(0, int(t)) for t in blk]
    raw = batch.run_coded_raw(inputs, queries, 32).reshape(64, 256, 3)
    for w in (0, 1, 2, 11, 63):
        want = O.fast_window_intervals(om, tokens[w * 256:(w + 1) * 256], chunk=32)
        bad = np.nonzero(np.any(raw[w] != want, axis=1))[0]
        assert len(bad) == 0, f"window {w}: {len(bad)} rows differ, first {bad[:8].tolist()}"


def _payload_from_intervals(iv):
    ops = [[0, int(st), int(fr), 32] for _, st, fr in iv]
    n, head = len(iv), bytearray()
    v = n
    while True:
        lo = v & 0x7F
        v >>= 7
        head.append(lo | (0x80 if v else 0))
        if not v:
            break
    return bytes(head) + O.encode_script(ops)


def test_bench_fold_payloads_equal_the_cpu(dev):
    """The benchmark's fold step exactly (64 windows x 256 tokens through the harness): every
    window's payload against the threaded CPU baseline and, for any disagreement, a
    single-window CPU recomputation."""
    from taco_amd import fold, hip, synth
    mb = synth.build_model(synth.GPT2_SMALL)
    tokens = synth.zipf_tokens(64 * 256)
    hm, om = hip.HipModel.load(dev, mb), O.Model(mb)
    batch = hip.HipBatch(hm, 64, 64 * 256)
    blocks = [tokens[w * 256:(w + 1) * 256] for w in range(64)]
    gpu = fold.fold_blocks(batch, blocks)
    cpu = O.fold_payloads(om, tokens, 64, 256, chunk=32, threads=16)
    bad = [w for w in range(64) if gpu[w] != cpu[w]]
    detail = []
    for w in bad[:3]:
        one = _payload_from_intervals(O.fast_window_intervals(om, blocks[w], chunk=32))
        detail.append((w, len(gpu[w]), len(cpu[w]), len(one), one == gpu[w], one == cpu[w]))
    assert not bad, f"windows {bad} differ; (w, gpu, cpu16, cpu1, cpu1==gpu, cpu1==cpu16): {detail}"


@pytest.mark.parametrize("name,k", [("predicted_text_k0", 0), ("predicted_text_k32", 32)])
def test_byte_level_fold_rebuilds_the_conformance_container(dev, name, k):
    """The byte-level fold of the text profile (crates/taco/src/fold.rs:502-565): the .in bytes
    cut into 300-byte blocks, tokenized with tiny.hsm's vocabulary and merges, coded on the GPU
    and stored as the smaller of payload and bytes: the container equals the reference's byte
    for byte (every block of these containers is coded, so no zstd candidate would have won)."""
    from taco_amd import fold, hip
    hsm = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()
    original = open(os.path.join(GOLDEN, name + ".in"), "rb").read()
    want = open(os.path.join(GOLDEN, name + ".taco"), "rb").read()
    hm = hip.HipModel.load(dev, hsm)
    tok = fold.Tokenizer.for_model(hm)
    batch = hip.HipBatch(hm, 4, 512)
    batch.set_overlap(k)
    got = fold.fold_bytes(batch, tok, original, 300, k)
    assert got == want
