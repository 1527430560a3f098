"""The oracle's mixer rules of the logs profile (crates/taco-match/src/mixer.rs:256-292,491-516;
crates/hardshell-cuda/src/mixed.rs:36-90), pinned by what the rules fix in closed form: the
tie rule of the top token, rule 1 without a prediction, and for k = 0 the exact split of the
mass (the predicted token gets q R, the others m R), the one-hot row, and the bounds of rule 6
for weights above 2^48."""

import numpy as np
import pytest

from oracle import oracle as O


def test_stats_tie_rule_and_exact_total():
    assert O.mix_stats([0, 5, 5, 3], 3) == (13, 3, 1)  # the lowest id of a tie
    assert O.mix_stats([0, 0, 0], 1) == (0, 0, 0)       # every weight 0: token 0
    assert O.mix_stats([4, 9, 9, 1], O.MIX_NONE) == (23, 0, 1)
    big = [1 << 63] * 3 + [5]
    assert O.mix_stats(big, 3) == (3 * (1 << 63) + 5, 5, 0)  # the u128 sum


def test_rule_1_without_a_prediction():
    assert O.mix_apply([0, 1, 7, 0], O.MIX_NONE, 1234).tolist() == [1, 1, 7, 1]


@pytest.mark.parametrize("seed", range(6))
def test_k_zero_splits_the_mass_exactly(seed):
    # R < 2^46 gives k = 0: w'[i] = w[i] (2^16 - q) for i != p (all >= 1) and w'[p] = q R, so
    # the mass is 2^16 R and the predicted token holds exactly q / 2^16 of it.
    r = np.random.default_rng(seed)
    n = int(r.integers(2, 3000))
    w = r.integers(1, 1 << 30, n).astype(np.uint64)
    p = int(r.integers(0, n))
    for q in (1, 2, 1 << 15, 65534, 65535, int(r.integers(1, 65536))):
        got = O.mix_apply(w, p, q)
        R = int(w.sum()) - int(w[p])
        assert R < 1 << 46
        assert int(got[p]) == q * R
        assert sum(int(x) for x in got) == (1 << 16) * R
        others = np.delete(got, p)
        assert np.array_equal(others, np.delete(w, p) * np.uint64((1 << 16) - q))
        assert O.mix_record(int(w.sum()), int(w[p]), q) == (0, (1 << 16) - q, q * R)


def test_one_hot_row():
    # R = max(W - w[p], 1) = 1: the prediction gets q, every other token max(1, 0) = 1
    w = [0, 0, 1 << 40, 0, 0]
    assert O.mix_apply(w, 2, 777).tolist() == [1, 1, 777, 1, 1]
    # the prediction is not the one-hot token: R = 2^40, k = 0 (bitlen 41 + 16 < 62)
    got = O.mix_apply(w, 0, 1000)
    assert got.tolist() == [1000 << 40, 1, (1 << 40) * 64536, 1, 1]


@pytest.mark.parametrize("seed", range(4))
def test_large_weights_keep_the_bounds_of_rule_6(seed):
    # weights above 2^48 (the u128 loop of apply): k = bitlen(R) - 46, every w' < 2^62, the
    # predicted weight is floor(R q / 2^k), and the other weights lose less than one unit each
    # to the floor: m R / 2^k - (n - 1) < sum_{i != p} w' <= m R / 2^k + (number of max(1, 0)).
    r = np.random.default_rng(100 + seed)
    n = 500
    w = (r.integers(0, 1 << 62, n, dtype=np.uint64) >> np.uint64(int(r.integers(0, 14))))
    w[r.integers(0, n, 20)] = 0
    p = int(r.integers(0, n))
    q = int(r.integers(1, 65536))
    W, wp, _ = O.mix_stats(w, p)
    R = max(W - wp, 1)
    k, m, wpm = O.mix_record(W, wp, q)
    assert k == max(0, R.bit_length() + 16 - 62) and m == 65536 - q
    got = O.mix_apply(w, p, q)
    assert int(got[p]) == wpm == max(1, (R * q) >> k)
    assert all(int(x) < 1 << 62 for x in got)
    assert sum(int(x) for x in got) < 1 << 63
    rest = sum(int(x) for i, x in enumerate(got) if i != p)
    zeros = sum(1 for i, x in enumerate(w) if i != p and (int(x) * m) >> k == 0)
    assert m * R / 2 ** k - (n - 1) < rest <= m * R / 2 ** k + zeros


def test_record_refusals():
    with pytest.raises(ValueError):
        O.mix_record(100, 10, 0)
    with pytest.raises(ValueError):
        O.mix_record(100, 10, 1 << 16)
    with pytest.raises(ValueError):
        O.mix_record(100, 101, 5)  # w[p] above the sum: no weights give these statistics


def test_mixed_table_interval():
    # the mixed table is FreqTable::from_weights of the mixed weights (its own unit vectors pin
    # from_weights): with k = 0 the predicted symbol gets about q / 2^16 of the total
    w = np.array([3, 9, 0, 4, 4], np.uint64)
    mw = O.mix_apply(w, 3, 49152)  # q = 3/4
    start, freq = O.freq_interval(mw, 20, 3)
    assert abs(freq / (1 << 20) - 0.75) < 1e-4


# ---------------------------------------------------------------------------------------------
# The match model and the mixer of the logs profile, mixer rule version 1: the golden vectors of
# crates/taco-match (logistic tables, the synthetic log of tests/golden.rs) and the mixed blocks
# of the conformance/v2 containers.

import hashlib
import os

from tests.conftest import GOLDEN
from tests.test_oracle import read_container, vocab_of

M64 = (1 << 64) - 1


class SplitMix64:
    """crates/taco-match/tests/common/mod.rs:7-22."""

    def __init__(self, s):
        self.s = s & M64

    def next_u64(self):
        self.s = (self.s + 0x9E3779B97F4A7C15) & M64
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    def below(self, n):
        return self.next_u64() % n


def synthetic_log(seed, count, vocab=1000, newline=198):
    """tests/common/mod.rs:28-50: 8 templates with variable fields."""
    rng = SplitMix64(seed)
    templates = []
    for _ in range(8):
        n = 5 + rng.below(20)
        templates.append([rng.below(vocab) for _ in range(n)])
    out = []
    while len(out) < count:
        for tok in templates[rng.below(8)]:
            out.append(tok)
            if rng.below(4) == 0:
                for _ in range(1 + rng.below(3)):
                    out.append(rng.below(vocab))
        out.append(newline)
    return out[:count]


def test_logistic_tables_match_the_golden_hashes():
    # crates/taco-match/src/logistic.rs:147-156
    sq, st = O.logistic_tables()
    assert hashlib.sha256(sq.astype("<u2").tobytes()).hexdigest() == \
        "345a564594a6032f8b2f13850e4b38ce420a8c50c4953f2cffd244e9d29781bc"
    assert hashlib.sha256(st.astype("<i2").tobytes()).hexdigest() == \
        "c1ed057a2aed7ea9f38e6cce27eaee39ccee69719aba90c0bb39ba5d02aad142"
    assert sq[4095] == 32768 and sq[0] == 1 and sq[-1] == 65535


def test_match_model_and_mixer_golden_vectors():
    # crates/taco-match/tests/golden.rs:20-50: 4,000 tokens of the synthetic log, the weights of
    # tests/common/mod.rs:52-59, then predict / mix / update / observe at each position.
    seed = 20_261_018
    tokens = synthetic_log(seed, 4000)
    rng = SplitMix64(seed ^ 0xA5A5)
    st = O.MixState()
    hp, hw = hashlib.sha256(), hashlib.sha256()
    for t in tokens:
        p = st.predict()
        w = np.zeros(1000, np.uint64)
        for i in range(1000):
            v = rng.next_u64()
            w[i] = v >> (20 + rng.below(44))
        if rng.below(2) == 0:
            w[t] = 1 << 40
        out = st.mix(w)
        st.observe(t)
        tok, ln = p if p else (0xFFFFFFFF, 0)
        hp.update(tok.to_bytes(4, "little") + ln.to_bytes(4, "little"))
        hw.update(out.astype("<u8").tobytes())
    assert hp.hexdigest() == "a7ccc360407bc350f5444defc5dcb8b173ec6e7ee8c17b02998d70c20c73b23d"
    assert hw.hexdigest() == "31d87e9efc45a331b7019e4c8f6058cea247637a5a29a3b0016981407821d614"


MIXED_CONTAINERS = ["predicted_logs_k0", "predicted_logs_default_k", "all_kinds_logs"]


@pytest.mark.parametrize("name", MIXED_CONTAINERS)
def test_conformance_mixed_blocks_decode_and_reencode(name):
    # conformance/v2/vectors.tsv:14-15,19: the mixed blocks (kind 3) restore their bytes and
    # re-encode to the same payloads.
    hsm = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()
    m = O.Model(hsm)
    vocab = vocab_of(hsm)
    data = open(os.path.join(GOLDEN, name + ".taco"), "rb").read()
    original = open(os.path.join(GOLDEN, name + ".in"), "rb").read()
    c = read_container(data)
    assert c["checksum"] == hashlib.sha256(original).digest()
    mixed = 0
    for i, (kind, payload) in enumerate(c["blocks"]):
        if kind != 3:
            continue
        piece = original[i * c["block_size"]:(i + 1) * c["block_size"]]
        toks = O.decode_mixed_block(m, payload, overlap=c["overlap"])
        assert b"".join(vocab[t] for t in toks) == piece
        assert O.encode_mixed_block(m, toks, overlap=c["overlap"]) == payload
        mixed += 1
    assert mixed >= 1
