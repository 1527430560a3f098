"""GPU parity of the mixed coder op of the logs profile (crates/hardshell-cuda/src/mixed.rs,
src/batch/mixed.rs; the scenarios of crates/hardshell-cuda/tests/mixed.rs): every interval
equals FreqTable::from_weights of the oracle's Mixer::mix weights for the q that the host
mixer gave, and the statistics the mixer sees equal pass 1 of Mixer::mix. The mixer here is a
deterministic function of its inputs; the op's contract holds for any q in 1..=65535."""

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import splitmix_tokens

pytestmark = pytest.mark.gpu

EDGE_Q = [1, 2, 1 << 15, 65534, 65535]


@pytest.fixture(scope="module")
def dev():
    from taco_amd import hip
    return hip.HipDevice.open(0)


def test_mixer_q(i, stats):
    """A deterministic mixer: the edge values of q, then a hash of the statistics."""
    if i < len(EDGE_Q):
        return EDGE_Q[i]
    h = (int(stats.total) * 0x9E3779B1 ^ int(stats.predicted) * 0x85EBCA77 ^ int(stats.top) ^ i)
    return 1 + h % 65535


test_mixer_q.__test__ = False  # a helper, not a test


def want_interval(w, table, q, bits, query):
    """The interval of query (kind, value) in the table named by `table`."""
    from taco_amd import hip
    if table == hip.HS_MIX_PLAIN:
        mw = np.asarray(w, np.uint64)
    else:
        mw = O.mix_apply(w, table, q)
    kind, value = query
    if kind == 0:
        s, f = O.freq_interval(mw, bits, value)
        return (value, s, f)
    return O.freq_find(mw, bits, value)


def weight_row(r, vocab, shape):
    if shape == 0:
        return r.integers(0, 1 << 40, vocab, dtype=np.uint64)
    if shape == 1:  # zeros among small weights
        w = r.integers(0, 50, vocab, dtype=np.uint64)
        w[r.random(vocab) < 0.5] = 0
        return w
    if shape == 2:
        return np.zeros(vocab, np.uint64)
    if shape == 3:  # one-hot (R = 1 when p is the hot token)
        w = np.zeros(vocab, np.uint64)
        w[int(r.integers(0, vocab))] = 1 << 40
        return w
    if shape == 4:  # above 2^48 where the row sum allows it: the u128 loop of apply
        return r.integers(0, min(1 << 52, (1 << 63) // vocab), vocab, dtype=np.uint64)
    w = r.integers(0, 4, vocab, dtype=np.uint64) * np.uint64(1 << 30)  # ties
    return w


@pytest.mark.parametrize("vocab,bits", [(300, 9), (300, 16), (1000, 32), (50257, 16), (50257, 32)])
def test_mixed_op_on_given_weights_equals_the_cpu_table(dev, vocab, bits):
    from taco_amd import hip
    print(f"mixed op vocab {vocab} bits {bits}", flush=True)
    r = np.random.default_rng(vocab + bits)
    rows = 24
    w = np.stack([weight_row(r, vocab, i % 6) for i in range(rows)])
    preds, queries = [], []
    for i in range(rows):
        if i % 7 == 6:
            preds.append(hip.HS_MIX_NONE)
        elif i % 6 == 3 and i % 2:  # the hot token of a one-hot row
            preds.append(int(np.argmax(w[i])))
        else:
            preds.append(int(r.integers(0, vocab)))
        if i % 3 == 2:
            queries.append((1, int(r.integers(0, 1 << bits))))
        else:
            queries.append((0, int(r.integers(0, vocab))))
    seen = []

    def mixer(i, st):
        seen.append((i, int(st.total), int(st.predicted), int(st.top)))
        return test_mixer_q(i, st)

    stats, got = hip.mixed_intervals_of_weights(dev, w, queries, preds, bits, mixer)
    assert [s[0] for s in seen] == [i for i in range(rows) if preds[i] != hip.HS_MIX_NONE]
    for i in range(rows):
        p = preds[i]
        total, wp, top = O.mix_stats(w[i], p)
        assert tuple(int(x) for x in stats[i]) == (total, wp, top), i
        q = test_mixer_q(i, hip.MixStats(total, wp, top)) if p != hip.HS_MIX_NONE else 0
        assert tuple(int(x) for x in got[i]) == want_interval(w[i], p, q, bits, queries[i]), i


def test_mixed_op_refuses_bad_arguments(dev):
    from taco_amd import hip
    w = np.ones((2, 10), np.uint64)
    q = [(0, 1), (0, 2)]
    with pytest.raises(hip.Unsupported):  # a q outside 1..=65535
        hip.mixed_intervals_of_weights(dev, w, q, [3, 4], 16, lambda i, s: 0)
    with pytest.raises(hip.Unsupported):
        hip.mixed_intervals_of_weights(dev, w, q, [3, 4], 16, lambda i, s: 1 << 16)
    with pytest.raises(hip.Unsupported):  # a predicted token out of range
        hip.mixed_intervals_of_weights(dev, w, q, [3, 10], 16, lambda i, s: 5)
    big = np.full((1, 4), 1 << 62, np.uint64)
    with pytest.raises(hip.Unsupported):  # a weight sum of 2^64
        hip.mixed_intervals_of_weights(dev, big, [(0, 1)], [2], 16, lambda i, s: 5)


def _model(dev, kind):
    from taco_amd import hip, synth
    if kind == "tiny":
        b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64)
    elif kind == "tiny-v2":
        b = O.build_model(O.tiny_dims(), 0x7AC0_0001, 64, wide=True)
    else:  # i64 logits: an exponent table longer than the compact form allows
        b = synth.build_model(synth.Dims(2, 4, 128, 512, 1000, 256), seed=0x51DE, table_len=20000)
    return O.Model(b), hip.HipModel.load(dev, b)


def _streams(slots, vocab, seed):
    return [splitmix_tokens(seed + s, 40 + 23 * s, vocab - 1) for s in range(slots)]


@pytest.mark.parametrize("kind,max_rows,overlap", [("tiny", 64, 0), ("tiny", 7, 9), ("long", 40, 0),
                                                   ("tiny-v2", 33, 0)])
def test_mixed_batch_equals_the_cpu_mixer(dev, kind, max_rows, overlap):
    from taco_amd import hip
    print(f"mixed batch {kind} rows {max_rows} overlap {overlap}", flush=True)
    om, hm = _model(dev, kind)
    V = om.vocab
    slots = 4
    seqs = _streams(slots, V, 31)
    # the oracle's weights of every row of every slot (row 0: input EOT)
    want_w = []
    for seq in seqs:
        s = O.Session(om, overlap=overlap)
        want_w.append([s.start_block()] + [s.step(t) for t in seq[:-1]])
    r = np.random.default_rng(5)
    b = hip.HipBatch(hm, slots, max_rows)
    b.set_overlap(overlap)
    done = [0] * slots
    calls = 0
    while any(done[s] < len(seqs[s]) for s in range(slots)):
        inputs, queries, tables, keys = [], [], [], []
        for s in range(slots):
            take = min(len(seqs[s]) - done[s], [1, 5, 17, 2][(s + calls) % 4])
            for i in range(done[s], done[s] + take):
                inputs.append((s, om.eot if i == 0 else seqs[s][i - 1]))
                tok = seqs[s][i]
                kind_t = (s + i) % 5
                if kind_t == 0:
                    tables.append(hip.HS_MIX_PLAIN)
                elif kind_t == 1:
                    tables.append(hip.HS_MIX_NONE)
                elif kind_t == 2:
                    tables.append(tok)  # a right prediction
                else:
                    tables.append(int(r.integers(0, V)))
                queries.append((0, tok) if i % 3 else (1, int(r.integers(0, 1 << 32))))
                keys.append((s, i))
            done[s] += take
        seen = []

        def mixer(i, st):
            seen.append(i)
            return test_mixer_q(i + calls, st)

        got = b.run_coded_mixed(inputs, queries, tables, 32, mixer)
        assert seen == [i for i, t in enumerate(tables) if t not in (hip.HS_MIX_PLAIN, hip.HS_MIX_NONE)]
        for i, (s, j) in enumerate(keys):
            w = want_w[s][j]
            p = tables[i]
            q = 0
            if p not in (hip.HS_MIX_PLAIN, hip.HS_MIX_NONE):
                total, wp, top = O.mix_stats(w, p)
                q = test_mixer_q(i + calls, hip.MixStats(total, wp, top))
            assert tuple(int(x) for x in got[i]) == want_interval(w, p, q, 32, queries[i]), (s, j)
        calls += 1


@pytest.mark.parametrize("kind", ["tiny", "long"])
def test_dual_intervals_equal_the_cpu_tables(dev, kind):
    from taco_amd import hip
    om, hm = _model(dev, kind)
    V = om.vocab
    slots = 3
    seqs = _streams(slots, V, 77)
    r = np.random.default_rng(9)
    inputs, tokens, preds, keys = [], [], [], []
    for s, seq in enumerate(seqs):
        for i, tok in enumerate(seq):
            inputs.append((s, om.eot if i == 0 else seq[i - 1]))
            tokens.append(tok)
            preds.append(hip.HS_MIX_NONE if i % 4 == 0 else (tok if i % 4 == 1 else int(r.integers(0, V))))
            keys.append((s, i))
    want_w = []
    for seq in seqs:
        ss = O.Session(om)
        want_w.append([ss.start_block()] + [ss.step(t) for t in seq[:-1]])
    b = hip.HipBatch(hm, slots, 64)
    plain, mixed = b.run_coded_dual(inputs, tokens, preds, 32, test_mixer_q)
    for i, (s, j) in enumerate(keys):
        w = want_w[s][j]
        st, fr = O.freq_interval(w, 32, tokens[i])
        assert tuple(int(x) for x in plain[i]) == (tokens[i], st, fr), i
        p = preds[i]
        q = 0
        if p != hip.HS_MIX_NONE:
            total, wp, top = O.mix_stats(w, p)
            q = test_mixer_q(i, hip.MixStats(total, wp, top))
        assert tuple(int(x) for x in mixed[i]) == want_interval(w, p, q, 32, (0, tokens[i])), i


def test_mixed_refusals_keep_positions(dev):
    from taco_amd import hip
    om, hm = _model(dev, "tiny")
    b = hip.HipBatch(hm, 2, 16)
    b.run_coded_mixed([(0, 299), (1, 299)], [(0, 5), (0, 6)], [hip.HS_MIX_NONE, 7], 32, lambda i, s: 9)
    before = (b.position(0), b.position(1))
    with pytest.raises(hip.Unsupported):
        b.run_coded_mixed([(0, 5), (1, 6)], [(0, 1), (0, 2)], [3, 4], 32, lambda i, s: 0)
    with pytest.raises(hip.Unsupported):
        b.run_coded_mixed([(0, 5), (1, 6)], [(0, 1), (0, 2)], [3, 300], 32, lambda i, s: 7)
    with pytest.raises(hip.Unsupported):  # HS_MIX_PLAIN is not a prediction of a dual call
        b.run_coded_dual([(0, 5)], [1], [hip.HS_MIX_PLAIN], 32, lambda i, s: 7)
    assert (b.position(0), b.position(1)) == before


def _table(kind):
    if kind == "flat":  # a flat start (d0 = 4), then a decay to zeros
        t = [1 << 40] * 5 + [round(2 ** 40 * np.exp(-i / 64)) for i in range(1, 3000)]
    elif kind == "short":  # 40 entries, the last ones 0 (zcut < len)
        t = [max(0, (1 << 36) - i * (1 << 31)) for i in range(40)]
    elif kind == "notail":  # no zero tail: every d >= len - 1 weighs the last entry
        t = [round(2 ** 40 * np.exp(-i / 1024)) for i in range(4096)]
    elif kind == "long":  # longer than the compact form: the i64 kernels
        t = [round(2 ** 40 * np.exp(-i / 256)) for i in range(20000)]
    else:
        t = [round(2 ** 40 * np.exp(-i / 256)) for i in range(8192)]
    return np.array(t, np.uint64)


@pytest.mark.parametrize("vocab,kind", [(300, "exp"), (50257, "exp"), (1000, "flat"), (257, "short"),
                                        (1000, "long"), (70000, "exp"), (1000, "notail"),
                                        (50257, "notail"), (70000, "notail")])
def test_mixed_op_on_logits_equals_the_cpu_table(dev, vocab, kind):
    # The compact (d16) and i64 sources of the statistics and mixed kernels on rows built to
    # reach their corners: the prediction as the unique argmax (the best other weight then comes
    # from a later bin), w'[p] equal to the best other weight (the lower id wins), predictions
    # among zero weights (d >= zcut, counted as weight 1), rows where every other weight is 0,
    # ties at the maximum, plain rows and rows without a prediction.
    from taco_amd import hip
    print(f"mixed op on logits vocab {vocab} table {kind}", flush=True)
    table = _table(kind)
    L = len(table)
    r = np.random.default_rng(vocab * 7 + L)
    rows, preds, qs, queries = [], [], [], []

    def add(l, p, q, query=None):
        rows.append(np.asarray(l, np.int64))
        preds.append(p)
        qs.append(q)
        queries.append(query if query is not None else (0, int(r.integers(0, vocab))))

    for rep in range(2):
        base = r.integers(-3 * L, 50, vocab).astype(np.int64)
        a = int(np.argmax(base))
        add(base, a, EDGE_Q[rep])                                # p = argmax
        add(base, int(r.integers(0, vocab)), 40000 + rep)        # a random p
        far = int(np.argmin(base))
        add(base, far, 65535, (1, int(r.integers(0, 1 << 32))))  # p among the smallest
        add(base, hip.HS_MIX_NONE, 0)
        add(base, hip.HS_MIX_PLAIN, 0, (1, int(r.integers(0, 1 << 32))))
        # every other weight 0 but one: R = table[0], q = 2^15 makes w'[p] = the best other
        lone = np.full(vocab, -(1 << 40), np.int64)
        x, y = sorted(r.choice(vocab, 2, replace=False).tolist())
        lone[x] = 0
        add(lone, y, 1 << 15, (0, y))   # tie, the other (x < y) wins
        lone2 = np.full(vocab, -(1 << 40), np.int64)
        lone2[y] = 0
        add(lone2, x, 1 << 15, (0, x))  # tie, p (x < y) wins
        add(lone, x, 3)                 # p is the only weight: R = 1
        flat = np.full(vocab, 7, np.int64)
        add(flat, int(r.integers(0, vocab)), 12345, (1, int(r.integers(0, 1 << 32))))
        ext = r.choice([-(1 << 40), 1 << 40, 0], vocab).astype(np.int64)
        add(ext, int(r.integers(0, vocab)), 999)
    logits = np.stack(rows)
    qmap = {i: q for i, q in enumerate(qs)}
    seen = []

    def mixer(i, st):
        seen.append(i)
        return qmap[i]

    stats, got = hip.mixed_coder_logits(dev, logits, table, queries, preds, 32, mixer)
    assert seen == [i for i, p in enumerate(preds) if p not in (hip.HS_MIX_NONE, hip.HS_MIX_PLAIN)]
    for i in range(len(rows)):
        w = O.logits_to_weights(logits[i], table)
        p = preds[i]
        total, wp, top = O.mix_stats(w, p)
        assert tuple(int(x) for x in stats[i]) == (total, wp, top), i
        assert tuple(int(x) for x in got[i]) == want_interval(w, p, qs[i], 32, queries[i]), i


def _leb(n):
    head = bytearray()
    while True:
        lo = n & 0x7F
        n >>= 7
        head.append(lo | (0x80 if n else 0))
        if not n:
            return bytes(head)


@pytest.mark.parametrize("name", ["predicted_logs_k0", "predicted_logs_default_k", "all_kinds_logs"])
def test_conformance_mixed_blocks_through_the_gpu(dev, name):
    """The mixed blocks (kind 3) of the conformance/v2 logs containers, decoded on the GPU with
    the mixed coder op (Decode queries, one row per block per call, as gpu_unfold.rs with
    MIXED-INTEGRATION.md section 5; the host mixer is the oracle's match model and mixer of
    crates/taco/src/mix.rs), restore their bytes; fold's dual op on the decoded tokens (all
    rows of a block in one call, section 4) re-encodes the same payloads, and its plain
    intervals are the coded block's."""
    import os
    from taco_amd import hip
    from tests.conftest import GOLDEN
    from tests.test_oracle import read_container, vocab_of
    hsm = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()
    om, hm = O.Model(hsm), hip.HipModel.load(dev, hsm)
    vocab = vocab_of(hsm)
    data = open(os.path.join(GOLDEN, name + ".taco"), "rb").read()
    original = open(os.path.join(GOLDEN, name + ".in"), "rb").read()
    c = read_container(data)
    blocks = [(i, p) for i, (k, p) in enumerate(c["blocks"]) if k == 3]
    assert blocks
    n_b = len(blocks)
    b = hip.HipBatch(hm, n_b, 64)
    b.set_overlap(c["overlap"])
    decs, counts, toks, states = [], [], [], []
    for _, payload in blocks:
        n, used, shift = 0, 0, 0
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
        states.append(O.MixState())
    nxt = [om.eot] * n_b
    while any(len(toks[s]) < counts[s] for s in range(n_b)):
        live = [s for s in range(n_b) if len(toks[s]) < counts[s]]
        preds = [states[s].predict() for s in live]
        tables = [p[0] if p else hip.HS_MIX_NONE for p in preds]

        def mixer(i, st):  # the host step of unfold: mix_stats only (the token is not known)
            return states[live[i]].mix_stats(int(st.total), int(st.predicted), int(st.top))

        got = b.run_coded_mixed([(s, nxt[s]) for s in live], [(1, decs[s].target(32)) for s in live],
                                tables, 32, mixer)
        for s, (sym, start, freq) in zip(live, got):
            decs[s].decode_interval(int(start), int(freq), 32)
            states[s].observe(int(sym))
            toks[s].append(int(sym))
            nxt[s] = int(sym)
    for s, (i, payload) in enumerate(blocks):
        piece = original[i * c["block_size"]:(i + 1) * c["block_size"]]
        assert b"".join(vocab[t] for t in toks[s]) == piece, s
    # fold: every row of every block in one dual call; the match model runs ahead (it depends
    # only on the tokens), the mixer steps in input order inside the host step
    b2 = hip.HipBatch(hm, n_b, 512)
    b2.set_overlap(c["overlap"])
    inputs, tokens, predictions, owner = [], [], [], []
    for s in range(n_b):
        ahead = O.MixState()
        for j, t in enumerate(toks[s]):
            p = ahead.predict()
            inputs.append((s, om.eot if j == 0 else toks[s][j - 1]))
            tokens.append(t)
            predictions.append(p[0] if p else hip.HS_MIX_NONE)
            owner.append((s, j))
            ahead.observe(t)
    mixers = [O.MixState() for _ in range(n_b)]
    done = [0] * n_b  # tokens each block's mixer has observed

    def dual_mixer(i, st):
        s, j = owner[i]
        while done[s] < j:  # rows without a prediction had no call: observe them now
            mixers[s].observe(toks[s][done[s]])
            done[s] += 1
        q = mixers[s].mix_stats(int(st.total), int(st.predicted), int(st.top))
        mixers[s].observe(toks[s][j])
        done[s] = j + 1
        return q

    plain, mixed = b2.run_coded_dual(inputs, tokens, predictions, 32, dual_mixer)
    for s, (i, payload) in enumerate(blocks):
        rows = [r for r, (ss, _) in enumerate(owner) if ss == s]
        ops = [[0, int(mixed[r][1]), int(mixed[r][2]), 32] for r in rows]
        assert _leb(len(rows)) + O.encode_script(ops) == payload, s
        ops = [[0, int(plain[r][1]), int(plain[r][2]), 32] for r in rows]
        assert _leb(len(rows)) + O.encode_script(ops) == O.encode_block(om, toks[s], overlap=c["overlap"])
