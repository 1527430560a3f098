"""Speculative decoding on the GPU against the oracle (the behaviour of
crates/hardshell-cuda/tests/speculative.rs and crates/hardshell/src/gpt2/stream.rs):
draft rows of several slots in one call, then a truncation of each slot after its first
wrong draft token, with context restarts (overlap K) and truncations back before a restart.
Every kept row must give the weights (or the coder interval) of the oracle session that never
ran a wrong token."""

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import splitmix_tokens

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from taco_amd import hip
    return hip.HipDevice.open(0)


def oracle_rows(om, toks, k):
    """Row i = the weights after input i of the stream (input 0 is the block start)."""
    s = O.Session(om, k)
    return [s.start_block()] + [s.step(int(t)) for t in toks]


def other_token(t, rng, vocab):
    return int((int(t) + 1 + rng.integers(0, vocab - 1)) % vocab)


def run_case(dev, dims, k, slots, max_rows, seed):
    from taco_amd import hip
    b = O.build_model(dims, seed, 64)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    vocab, n_ctx = dims[4], dims[5]
    n = n_ctx - 1 + 3 * (n_ctx - 1 - k) + 4
    seqs = [splitmix_tokens(seed ^ (j + 1), n + 3 * j, vocab) for j in range(slots)]
    want = [oracle_rows(om, s, k) for s in seqs]
    batch = hip.HipBatch(hm, slots, max_rows)
    batch.set_overlap(k)
    w = batch.run_weights([(s, om.eot) for s in range(slots)])
    for s in range(slots):
        assert np.array_equal(w[s], want[s][0])
        assert batch.stream_len(s) == 1
    rng = np.random.default_rng(seed ^ 0xD4AF)
    max_d = max(1, min(12, n_ctx - 1 - k))
    n_in = [1] * slots  # inputs run so far (the start included)
    call = cut_back = 0
    while any(n_in[s] <= len(seqs[s]) for s in range(slots)):
        inputs, drafts = [], []
        for s, seq in enumerate(seqs):
            if n_in[s] > len(seq) or rng.integers(0, 5) == 0:
                continue
            d = min(1 + int(rng.integers(0, max_d)), len(seq) + 1 - n_in[s])
            good = int(rng.integers(0, d))
            drafts.append((s, len(inputs), d, good))
            for j in range(d):
                t = seq[n_in[s] - 1 + j]
                inputs.append((s, t if j <= good else other_token(t, rng, vocab)))
        if not inputs:
            continue
        if call % 2 == 0:
            w = batch.run_weights(inputs)
            for s, at, d, good in drafts:
                for j in range(good + 1):
                    assert np.array_equal(w[at + j], want[s][n_in[s] + j]), \
                        f"K {k}, slot {s}, len {n_in[s]}, row {j}"
        else:
            queries = [(0, 0)] * len(inputs)
            for s, at, d, good in drafts:
                for j in range(good + 1):
                    nxt = n_in[s] + j
                    if nxt < len(seqs[s]):
                        queries[at + j] = (0, int(seqs[s][nxt]))
            iv = batch.run_coded_raw(inputs, queries, 32)
            for s, at, d, good in drafts:
                for j in range(good + 1):
                    tok = queries[at + j][1]
                    start, freq = O.freq_interval(want[s][n_in[s] + j], 32, tok)
                    assert tuple(int(x) for x in iv[at + j]) == (tok, start, freq), \
                        f"coder, K {k}, slot {s}"
        for s, at, d, good in drafts:
            assert batch.stream_len(s) == n_in[s] + d
            kept = good + 1
            if rng.integers(0, 4) == 0:  # sometimes fewer: back before a restart
                kept = 1 + int(rng.integers(0, good + 1))
            cut_back += kept < good + 1
            batch.truncate(s, n_in[s] + kept)
            n_in[s] += kept
        call += 1
    if max_d > 1:
        assert cut_back > 0


@pytest.mark.parametrize("k", [0, 1, 32, 62])
def test_draft_rows_and_truncations_equal_the_oracle(dev, k):
    run_case(dev, O.tiny_dims(), k, 5, 9, 0x5BEC ^ k)


def test_draft_rows_in_passes_of_two_rows(dev):
    run_case(dev, O.tiny_dims(), 20, 3, 2, 0x5BED)


@pytest.mark.parametrize("k", [0, 9, 18])
def test_odd_shapes_truncate_as_the_oracle(dev, k):
    run_case(dev, (1, 3, 60, 100, 300, 20), k, 4, 16, 0x5BEE ^ k)


def test_truncation_across_a_restart(dev):
    """n_ctx 64, K 32: 8 wrong rows from input 60 cross the restart; the truncation to 60
    inputs goes back before it, and the slot then continues as the oracle session."""
    from taco_amd import hip
    dims = O.tiny_dims()
    b = O.build_model(dims, 41, 64)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    toks = splitmix_tokens(42, 160, dims[4])
    want = oracle_rows(om, toks, 32)
    batch = hip.HipBatch(hm, 1, 64)
    batch.set_overlap(32)
    batch.run_weights([(0, om.eot)] + [(0, t) for t in toks[:59]])
    rng = np.random.default_rng(43)
    batch.run_weights([(0, other_token(t, rng, dims[4])) for t in toks[59:67]])
    assert batch.position(0) < 64
    with pytest.raises(hip.ModelError):
        batch.truncate(0, 69)
    batch.truncate(0, 60)
    assert (batch.position(0), batch.stream_len(0)) == (60, 60)
    w = batch.run_weights([(0, t) for t in toks[59:90]])
    for j in range(31):
        assert np.array_equal(w[j], want[60 + j]), j


def test_room_follows_the_stream_rule(dev):
    """stream.rs:119-121: n_ctx - pos inside a context, n_ctx - K - 1 at a full context."""
    from taco_amd import hip
    dims = O.tiny_dims()
    b = O.build_model(dims, 41, 64)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    batch = hip.HipBatch(hm, 2, 64)
    batch.set_overlap(10)
    assert batch.room(0) == 64 and batch.room(5) == 0
    batch.run_weights([(0, om.eot)] + [(0, 7)] * 63)
    assert batch.position(0) == 64 and batch.room(0) == 64 - 10 - 1
    batch.run_weights([(0, 8)])
    assert batch.position(0) == 12 and batch.room(0) == 52 and batch.stream_len(0) == 65
    batch.reset(0)
    assert batch.stream_len(0) == 0 and batch.position(0) == 0
