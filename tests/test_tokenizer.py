"""The tokenizer of the byte-level fold (libtaco_hip.so, tc_tokenize; crates/taco/src/tokenizer):
the reference's own unit cases, the pre-tokenizer against the published GPT-2 pattern run by the
`regex` module, the BPE merge rounds against the quadratic algorithm of tools/baseline/bpe.py on
random merge lists, and the conformance/v2 blocks: encoding each coded block's bytes with
tiny.hsm's vocabulary and merges gives the token ids that its payload decodes to. Host code
only; no GPU."""

import hashlib
import json
import os
import random

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import GOLDEN
from tests.test_oracle import read_container, vocab_of

BYTES = [bytes([b]) for b in range(256)]


def fold():
    from taco_amd import fold as F
    return F


def tok(vocab, eot, merges):
    return fold().Tokenizer.from_parts(vocab, eot, merges)


def merges_of(hsm: bytes):
    hl = int.from_bytes(hsm[12:16], "little")
    h = json.loads(hsm[16:16 + hl])
    off, ln = h["merges"]["offset"], h["merges"]["length"]
    return [(int.from_bytes(hsm[off + 8 * i:off + 8 * i + 4], "little"),
             int.from_bytes(hsm[off + 8 * i + 4:off + 8 * i + 8], "little")) for i in range(ln // 8)]


# ---- the reference's unit cases (tokenizer/mod.rs:215-268, pretokenize.rs:171-213) ------------

def test_merges_join_pieces():
    v = BYTES + [b"th", b"the", b" the", b"<|endoftext|>"]
    t = tok(v, 259, [(116, 104), (256, 101), (32, 257)])
    assert t.encode(b"the  the").tolist() == [257, 32, 258]


@pytest.mark.parametrize("merges,why", [
    ([(97, 99)], "no token has the joined bytes"),
    ([(97, 1000)], "not in the vocabulary"),
    ([(97, 257)], "<|endoftext|>"),
    ([(97, 98), (97, 98)], "two times"),
])
def test_refuses_bad_merges(merges, why):
    from taco_amd import hip
    v = BYTES + [b"ab", b"<|endoftext|>"]
    with pytest.raises(hip.HipError, match=why):
        tok(v, 257, merges)


def test_refuses_ambiguous_and_missing_byte_tokens():
    from taco_amd import hip
    with pytest.raises(hip.HipError, match="two or more tokens"):
        tok(BYTES + [b"ab", b"ab"], None, [(97, 98)])
    v = list(BYTES)
    v[7] = b"xx"
    with pytest.raises(hip.HipError, match="byte 7"):
        tok(v, None, [])


def test_invalid_utf8_uses_single_byte_tokens():
    t = tok(BYTES, None, [])
    data = bytes([0xE0, 0x41, 0xFF, 0xC3, 0xA9])
    assert t.encode(data).tolist() == list(data)


@pytest.mark.parametrize("text,want", [
    ("Hello world", ["Hello", " world"]),
    ("  two  spaces", [" ", " two", " ", " spaces"]),
    ("don't we'll", ["don", "'t", " we", "'ll"]),
    ("\"'s", ["\"'", "s"]),
    ("'S", ["'", "S"]),
    ("a\n\n b", ["a", "\n\n", " b"]),
    ("a\tb", ["a", "\t", "b"]),
    ("a   ", ["a", "   "]),
    (" ", [" "]),
    ("x \n", ["x", " \n"]),
    ("abc123!?", ["abc", "123", "!?"]),
    (" 42 ++", [" 42", " ++"]),
    ("हि", ["ह", "ि"]),
])
def test_pieces_of_the_reference_cases(text, want):
    assert fold().pieces(text.encode()) == [w.encode() for w in want]


# ---- the pre-tokenizer against the published pattern -------------------------------------------

GPT2_PATTERN = r"""'s|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+"""


def test_pieces_equal_the_published_pattern():
    """openai/gpt-2 encoder.py's pattern (tools/baseline/bpe.py) run by the regex module on random
    texts over letters, numbers, white space, apostrophes and other characters of several
    scripts."""
    regex = pytest.importorskip("regex")
    pat = regex.compile(GPT2_PATTERN)
    alphabet = list("abzAZ019 '\t\n\r.,!?-_\"") + ["s", "t", "re", "ve", "ll", "d", "m", "'s", "'ll",
                                                  "é", "ß", "ह", "ि", "中",
                                                  "٣", "½", "Ⅳ", " ", "　",
                                                  " ", "​", "€", "\U0001f600", "́"]
    rng = random.Random(7)
    for _ in range(3000):
        text = "".join(rng.choice(alphabet) for _ in range(rng.randint(0, 24)))
        want = [m.encode() for m in pat.findall(text)]
        assert fold().pieces(text.encode()) == want, repr(text)


# ---- the merge rounds against the quadratic algorithm -----------------------------------------

def bpe_quadratic(symbols, merges):
    """_bpe of tools/baseline/bpe.py on ids: join every occurrence of the lowest-ranked pair,
    left to right, until no pair has a merge."""
    word = list(symbols)
    while len(word) > 1:
        best = None
        for i in range(len(word) - 1):
            m = merges.get((word[i], word[i + 1]))
            if m is not None and (best is None or m[0] < best[0]):
                best = (m[0], i)
        if best is None:
            break
        first, second = word[best[1]], word[best[1] + 1]
        merged = merges[(first, second)][1]
        out, i = [], 0
        while i < len(word):
            if i + 1 < len(word) and word[i] == first and word[i + 1] == second:
                out.append(merged)
                i += 2
            else:
                out.append(word[i])
                i += 1
        word = out
    return word


def test_merge_rounds_equal_the_quadratic_algorithm():
    """Random merge lists over a 4-letter alphabet with shuffled ranks (later tokens may rank
    lower, so a join can make a pair of a rank below the current one), random words of one
    piece (letters only)."""
    rng = random.Random(0x1234)
    letters = [ord(c) for c in "abcd"]
    for case in range(400):
        vocab = list(BYTES)
        by_bytes = {bytes([b]): b for b in range(256)}
        ids = list(letters)
        pairs = []
        for _ in range(rng.randint(0, 14)):
            a, b = rng.choice(ids), rng.choice(ids)
            joined = vocab[a] + vocab[b]
            if (a, b) in [p for p, _ in pairs]:
                continue
            if joined in by_bytes:
                if by_bytes[joined] in ids and by_bytes[joined] >= 256:
                    pairs.append(((a, b), by_bytes[joined]))
                continue
            by_bytes[joined] = len(vocab)
            vocab.append(joined)
            ids.append(len(vocab) - 1)
            pairs.append(((a, b), len(vocab) - 1))
        rng.shuffle(pairs)
        merges = {p: (rank, m) for rank, (p, m) in enumerate(pairs)}
        t = tok(vocab, None, [p for p, _ in pairs])
        for _ in range(5):
            word = [rng.choice(letters) for _ in range(rng.randint(0, 24))]
            want = bpe_quadratic(word, merges)
            assert t.encode(bytes(word)).tolist() == want, (case, pairs, word)


def test_long_pieces_equal_the_quadratic_algorithm():
    """Pieces of 200-3,000 letters over two letters (runs of one letter, where the pair (a, a)
    overlaps itself, and mixed runs), with merge lists that build up to 8-letter tokens in
    shuffled order."""
    rng = random.Random(0x5EED)
    a, b = ord("a"), ord("b")
    for case in range(12):
        vocab = list(BYTES)
        by_bytes = {bytes([x]): x for x in range(256)}
        ids = [a, b]
        pairs = []
        while len(pairs) < 20:
            x, y = rng.choice(ids), rng.choice(ids)
            joined = vocab[x] + vocab[y]
            if len(joined) > 8 or joined in by_bytes or (x, y) in [p for p, _ in pairs]:
                continue
            by_bytes[joined] = len(vocab)
            vocab.append(joined)
            ids.append(len(vocab) - 1)
            pairs.append(((x, y), len(vocab) - 1))
        if case % 2:
            rng.shuffle(pairs)
        merges = {p: (rank, m) for rank, (p, m) in enumerate(pairs)}
        t = tok(vocab, None, [p for p, _ in pairs])
        n = rng.randint(200, 3000)
        if case % 3 == 0:
            word = [a] * n
        else:
            word = [rng.choice((a, a, b)) for _ in range(n)]
        assert t.encode(bytes(word)).tolist() == bpe_quadratic(word, merges), case


# ---- the conformance blocks -------------------------------------------------------------------

@pytest.mark.parametrize("name", ["predicted_text_k0", "predicted_text_k32", "all_kinds_text"])
def test_conformance_blocks_tokenize_to_their_decoded_ids(name):
    """Each coded block of a conformance/v2 container decodes (with tiny.hsm) to token ids; the
    tokenizer of tiny.hsm's vocabulary and merges gives exactly those ids for the block's bytes
    (crates/taco/src/fold.rs:517-530: the reference tokenized these blocks to code them)."""
    hsm = open(os.path.join(GOLDEN, "tiny.hsm"), "rb").read()
    m = O.Model(hsm)
    vocab = vocab_of(hsm)
    t = tok(vocab, 299, merges_of(hsm))
    data = open(os.path.join(GOLDEN, name + ".taco"), "rb").read()
    original = open(os.path.join(GOLDEN, name + ".in"), "rb").read()
    c = read_container(data)
    coded = 0
    for i, (kind, payload) in enumerate(c["blocks"]):
        if kind != 1:
            continue
        piece = original[i * c["block_size"]:(i + 1) * c["block_size"]]
        want = O.decode_block(m, payload, overlap=c["overlap"])
        assert t.encode(piece).tolist() == list(want), (name, i)
        coded += 1
    assert coded >= 2
