"""GPU parity of model-file version 2 ("wide") rules: i16 GELU outputs and a 16-bit ln_f as two
i8 planes with row sums, and the one-rounding LayerNorm with ln_beta_frac
(crates/hardshell/src/gpt2/ops.rs:178-206,246-277, crates/hardshell/src/layernorm.rs:153-175).
The golden v2 hashes of crates/hardshell/tests/wide.rs:259-277 pin the tiny model; larger and
odd shapes are compared with the oracle's reference session row by row, bit-exact."""

import hashlib

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import splitmix_tokens
from tests.test_oracle import GOLDEN_V2_MODEL, GOLDEN_V2_OUTPUT, weights_hash

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from taco_amd import hip
    return hip.HipDevice.open(0)


@pytest.fixture(scope="module")
def golden_v2(dev):
    from taco_amd import hip
    b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64, wide=True)
    assert hashlib.sha256(b).hexdigest() == GOLDEN_V2_MODEL
    hm = hip.HipModel.load(dev, b)
    assert hm.is_wide()
    return b, hm, O.Model(b)


def test_golden_v2_output_hash_on_gpu(golden_v2):
    # crates/hardshell/tests/wide.rs:259-277 through the GPU step path (150 tokens, 1 restart).
    from taco_amd import hip
    _, hm, _ = golden_v2
    s = hip.HipSession(hm)
    rows = [s.start_block()] + [s.step(t) for t in splitmix_tokens(0x7AC0_0002, 150, 300)]
    assert weights_hash(rows) == GOLDEN_V2_OUTPUT


@pytest.mark.parametrize("max_rows", [3, 64, 200])
def test_v2_prefill_passes_equal_the_reference(golden_v2, max_rows):
    from taco_amd import hip
    _, hm, om = golden_v2
    toks = splitmix_tokens(0x7AC0_0002, 150, 300)
    s = O.Session(om)
    want = np.array([s.start_block()] + [s.step(t) for t in toks])
    b = hip.HipBatch(hm, 1, max_rows)
    got = b.run_weights([(0, 299)] + [(0, t) for t in toks])
    assert np.array_equal(got, want)


def test_v2_overlap_equals_the_reference(golden_v2):
    # overlap 32 over 300 tokens (8 restarts), one row per call
    from taco_amd import hip
    _, hm, om = golden_v2
    toks = splitmix_tokens(0x7AC0_0002, 300, 300)
    s = O.Session(om, overlap=32)
    want = [s.start_block()] + [s.step(t) for t in toks]
    h = hip.HipSession(hm, overlap=32)
    got = [h.start_block()] + [h.step(t) for t in toks]
    assert np.array_equal(np.array(got), np.array(want))


def test_v2_batch_of_slots_equals_independent_sessions(golden_v2):
    from taco_amd import hip
    _, hm, om = golden_v2
    slots = 4
    seqs = [splitmix_tokens(200 + s, 30 + 9 * s, 299) for s in range(slots)]
    want = []
    for seq in seqs:
        s = O.Session(om)
        want.append([s.start_block()] + [s.step(t) for t in seq[:-1]])
    b = hip.HipBatch(hm, slots, 64)
    got = [[] for _ in range(slots)]
    done = [0] * slots
    while any(done[s] < len(seqs[s]) for s in range(slots)):
        inputs, owner = [], []
        for s in range(slots):
            take = min(len(seqs[s]) - done[s], 1 + 2 * s)
            for i in range(done[s], done[s] + take):
                inputs.append((s, 299 if i == 0 else seqs[s][i - 1]))
                owner.append(s)
            done[s] += take
        for o, row in zip(owner, b.run_weights(inputs)):
            got[o].append(row)
    for s in range(slots):
        assert np.array_equal(np.array(got[s]), np.array(want[s])), s


def test_v2_coded_intervals_equal_from_weights(golden_v2):
    from taco_amd import hip
    _, hm, om = golden_v2
    toks = splitmix_tokens(0x5EED, 63, 300)
    s = O.Session(om)
    weights = [s.start_block()] + [s.step(t) for t in toks[:-1]]
    b = hip.HipBatch(hm, 1, 64)
    inputs = [(0, 299)] + [(0, t) for t in toks[:-1]]
    enc = b.run_coded(inputs, [(0, t) for t in toks], 32)
    for i, (w, iv) in enumerate(zip(weights, enc)):
        st, fr = O.freq_interval(w, 32, toks[i])
        assert (iv.symbol, iv.start, iv.freq) == (toks[i], st, fr), i


# (n_layer, n_head, d_model, d_ff, vocab, n_ctx) of the synthetic wide models: head dims 32 and 64,
# a vocab that is not a multiple of 64, and exponent tables of 8,192 entries (compact logits) and
# 20,000 entries (i64 logits).
WIDE_SHAPES = [((2, 4, 128, 512, 1000, 256), 8192), ((2, 4, 128, 512, 1000, 256), 20000),
               ((1, 2, 128, 384, 777, 160), 8192)]


@pytest.mark.parametrize("dims,table_len", WIDE_SHAPES)
def test_v2_synthetic_models_equal_the_reference(dev, dims, table_len):
    from taco_amd import hip, synth
    print(f"wide model {dims} table {table_len}", flush=True)
    b = synth.build_model(synth.Dims(dims[0], dims[1], dims[2], dims[3], dims[4], dims[5]),
                          seed=0x51DE, wide=True, table_len=table_len)
    om, hm = O.Model(b), hip.HipModel.load(dev, b)
    assert om.wide and hm.is_wide()
    toks = splitmix_tokens(77, dims[5] + 40, dims[4] - 1)
    s = O.Session(om)
    want = np.array([s.start_block()] + [s.step(t) for t in toks])
    hb = hip.HipBatch(hm, 1, 97)
    got = hb.run_weights([(0, om.eot)] + [(0, t) for t in toks])
    assert np.array_equal(got, want)
