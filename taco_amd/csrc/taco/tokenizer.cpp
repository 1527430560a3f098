// The encoder side of taco's tokenizer (crates/taco/src/tokenizer/{mod,pretokenize,bpe}.rs):
// GPT-2 byte-level BPE over maximal runs of well-formed UTF-8, with every byte outside such a
// run as its single-byte token, so the bytes of the tokens are the input for every input.
// Host code of the harness (libtaco_hip.so), as the tokenizer is in the reference's taco crate.

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "common.h"
#include "taco_hip.h"

namespace {

#include "unicode_classes.inc"

// ---- character classes of the pre-tokenizer pattern (pretokenize.rs:31-84) ------------------

enum Class { LETTER, NUMBER, SPACE, OTHER };

template <size_t N>
bool in_ranges(uint32_t c, const uint32_t (&r)[N][2]) {
    size_t lo = 0, hi = N;  // the first range whose last code point is >= c
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (r[mid][1] < c) lo = mid + 1; else hi = mid;
    }
    return lo < N && r[lo][0] <= c;
}

Class class_of(uint32_t c) {
    if (c < 128) {
        if ((c | 32) >= 'a' && (c | 32) <= 'z') return LETTER;
        if (c >= '0' && c <= '9') return NUMBER;
        if (c == ' ' || (c >= 9 && c <= 13)) return SPACE;  // \t \n \v \f \r
        return OTHER;
    }
    if (in_ranges(c, k_letter)) return LETTER;
    if (in_ranges(c, k_number)) return NUMBER;
    if (in_ranges(c, k_space)) return SPACE;
    return OTHER;
}

// ---- UTF-8 ---------------------------------------------------------------------------------

// The length of the well-formed UTF-8 character at s[0 .. n) (Unicode table 3-7), or 0.
size_t utf8_char(const uint8_t *s, size_t n, uint32_t *cp) {
    const uint8_t b0 = s[0];
    if (b0 < 0x80) {
        *cp = b0;
        return 1;
    }
    auto cont = [&](size_t i, uint8_t lo, uint8_t hi) { return i < n && s[i] >= lo && s[i] <= hi; };
    if (b0 >= 0xC2 && b0 <= 0xDF) {
        if (!cont(1, 0x80, 0xBF)) return 0;
        *cp = ((uint32_t)(b0 & 0x1F) << 6) | (s[1] & 0x3F);
        return 2;
    }
    if (b0 >= 0xE0 && b0 <= 0xEF) {
        const uint8_t lo = b0 == 0xE0 ? 0xA0 : 0x80, hi = b0 == 0xED ? 0x9F : 0xBF;
        if (!cont(1, lo, hi) || !cont(2, 0x80, 0xBF)) return 0;
        *cp = ((uint32_t)(b0 & 0x0F) << 12) | ((uint32_t)(s[1] & 0x3F) << 6) | (s[2] & 0x3F);
        return 3;
    }
    if (b0 >= 0xF0 && b0 <= 0xF4) {
        const uint8_t lo = b0 == 0xF0 ? 0x90 : 0x80, hi = b0 == 0xF4 ? 0x8F : 0xBF;
        if (!cont(1, lo, hi) || !cont(2, 0x80, 0xBF) || !cont(3, 0x80, 0xBF)) return 0;
        *cp = ((uint32_t)(b0 & 0x07) << 18) | ((uint32_t)(s[1] & 0x3F) << 12) | ((uint32_t)(s[2] & 0x3F) << 6) |
              (s[3] & 0x3F);
        return 4;
    }
    return 0;
}

// The characters of a well-formed run: byte offset and code point of each, plus the end.
struct Chars {
    std::vector<uint32_t> off, cp;
};

// ---- the pre-tokenizer (pretokenize.rs:86-160) ------------------------------------------------
// 's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+ reduced to rules on
// the four classes, applied at the start of the rest of the text:
//  1. an apostrophe and s, t, re, ve, m, ll or d is a piece;
//  2. a letter, number or other character starts a run of its class;
//  3. a space (U+0020) before a letter, number or other character starts a run of that class;
//  4. else n white-space characters: one piece if they reach the end or n = 1, else the first
//     n - 1 (the last one may start a rule-3 piece).
// Returns the number of characters of the first piece of chars [i .. n).
size_t first_piece(const Chars &t, size_t i) {
    const size_t n = t.cp.size();
    const uint32_t c0 = t.cp[i];
    if (c0 == '\'' && i + 1 < n) {
        static const char *const sfx[] = {"s", "t", "re", "ve", "m", "ll", "d"};
        for (const char *s : sfx) {
            const size_t k = std::strlen(s);
            bool ok = i + k < n;  // k more characters exist
            for (size_t q = 0; ok && q < k; q++) ok = t.cp[i + 1 + q] == (uint32_t)(uint8_t)s[q];
            if (ok) return 1 + k;
        }
    }
    const Class k0 = class_of(c0);
    size_t start = i;
    Class run = k0;
    bool have_run = k0 != SPACE;
    if (k0 == SPACE && c0 == ' ' && i + 1 < n && class_of(t.cp[i + 1]) != SPACE) {
        have_run = true;
        run = class_of(t.cp[i + 1]);
        start = i + 1;
    }
    if (have_run) {
        size_t j = start;
        while (j < n && class_of(t.cp[j]) == run) j++;
        return j - i;
    }
    size_t j = i;
    while (j < n && class_of(t.cp[j]) == SPACE) j++;
    const size_t count = j - i;
    if (j == n || count == 1) return count;
    return count - 1;
}

// ---- BPE merges of one piece (the semantics of bpe.rs:41-116) ---------------------------------
// The rule: the adjacent pair that comes first in the merge list is joined at each of its
// occurrences, scanning left to right and leaving out an occurrence that overlaps one just
// joined; this repeats until no adjacent pair is in the list.
//
// A piece of n symbols is a row of n slots. A live slot holds a symbol and, when it has a live
// right neighbour, the list order of the pair it starts (NO_RULE otherwise). A min-tournament
// over the slots' orders names the round's pair at its root. The round then asks the tournament
// for the leftmost slot at or after a cursor whose order is at most the round's, joins there and
// moves the cursor one slot past the join. A join changes only the orders of its own slot and of
// its live left neighbour, both left of the cursor, and at the round's start no slot holds a
// smaller order, so the search meets exactly the occurrences of the round's pair, in order.
// Each join retires a slot, so a piece costs O(n log n) tournament steps.

struct PairRule {
    uint32_t order;   // position of the pair in the merge list
    uint32_t result;  // the token of the joined bytes
};

using PairRules = std::unordered_map<uint64_t, PairRule>;

inline uint64_t pair_code(uint32_t left, uint32_t right) { return ((uint64_t)left << 32) | right; }

class PieceJoiner {
  public:
    explicit PieceJoiner(const PairRules &rules) : rules_(rules) {}

    // Appends the tokens of `piece` after every join to `out`.
    void run(const std::vector<uint32_t> &piece, std::vector<uint32_t> &out) {
        const size_t n = piece.size();
        if (n < 2) {
            out.insert(out.end(), piece.begin(), piece.end());
            return;
        }
        tok_ = piece;
        made_.assign(n, 0);
        right_.resize(n);
        left_.resize(n);
        for (size_t i = 0; i < n; i++) {
            right_[i] = i + 1;  // n: no right neighbour
            left_[i] = i;       // i: no left neighbour (only slot 0)
            if (i) left_[i] = i - 1;
        }
        leaves_ = 1;
        while (leaves_ < n) leaves_ <<= 1;
        min_.assign(2 * leaves_, NO_RULE);
        for (size_t i = 0; i + 1 < n; i++) min_[leaves_ + i] = order_of(i);
        for (size_t k = leaves_ - 1; k >= 1; k--) min_[k] = std::min(min_[2 * k], min_[2 * k + 1]);

        while (min_[1] != NO_RULE) {
            const uint32_t round = min_[1];
            for (size_t at = 0;;) {
                const size_t p = leftmost_at_most(at, round);
                if (p == NONE) break;
                join(p);
                at = p + 1;
            }
        }
        for (size_t i = 0; i < n; i = right_[i]) out.push_back(tok_[i]);
    }

  private:
    static constexpr uint32_t NO_RULE = UINT32_MAX;
    static constexpr size_t NONE = SIZE_MAX;

    // The order of the pair that slot i starts (its result kept in made_[i]).
    uint32_t order_of(size_t i) {
        const size_t r = right_[i];
        if (r >= tok_.size()) return NO_RULE;
        const auto it = rules_.find(pair_code(tok_[i], tok_[r]));
        if (it == rules_.end()) return NO_RULE;
        made_[i] = it->second.result;
        return it->second.order;
    }

    void set(size_t i, uint32_t v) {
        size_t k = leaves_ + i;
        min_[k] = v;
        for (k >>= 1; k; k >>= 1) min_[k] = std::min(min_[2 * k], min_[2 * k + 1]);
    }

    // The leftmost slot >= lo whose order is <= bound, or NONE: test the subtrees right of lo in
    // order (climb while the node is a right child, then step to its right sibling) and descend
    // into the first whose minimum qualifies.
    size_t leftmost_at_most(size_t lo, uint32_t bound) const {
        if (lo >= leaves_) return NONE;
        size_t k = leaves_ + lo;
        for (;;) {
            if (min_[k] <= bound) {
                while (k < leaves_) {
                    k = 2 * k;
                    if (min_[k] > bound) k++;
                }
                return k - leaves_;
            }
            while (k & 1) k >>= 1;
            if (k == 0) return NONE;
            k++;
        }
    }

    // Joins slot p with its right neighbour: p takes the result, the neighbour retires, and the
    // orders of p and of p's left neighbour are taken again.
    void join(size_t p) {
        const size_t n = tok_.size();
        const size_t gone = right_[p];
        tok_[p] = made_[p];
        const size_t after = right_[gone];
        right_[p] = after;
        if (after < n) left_[after] = p;
        set(gone, NO_RULE);
        set(p, order_of(p));
        if (left_[p] != p) set(left_[p], order_of(left_[p]));
    }

    const PairRules &rules_;
    std::vector<uint32_t> tok_, made_, min_;
    std::vector<size_t> right_, left_;
    size_t leaves_ = 0;
};

}  // namespace

struct tc_tokenizer {
    uint32_t byte_tokens[256];
    PairRules rules;
    size_t vocab_size = 0;
};

namespace {

// Tokenizer::new (mod.rs:87-147): tokens in id order (EOT and empty tokens never in the output),
// the merges in rank order.
hs_status make_tokenizer(size_t count, const std::function<std::pair<const uint8_t *, size_t>(size_t)> &tok,
                         uint32_t eot, const uint32_t *merges, size_t n_merges, tc_tokenizer **out) {
    if (count > UINT32_MAX) return hs::fail(HS_MODEL_ERROR, HS_MODEL_VOCABULARY, "the vocabulary has more than u32::MAX tokens");
    auto t = std::make_unique<tc_tokenizer>();
    t->vocab_size = count;
    std::unordered_map<std::string, int64_t> owners;  // -1: two or more tokens
    std::vector<char> usable(count, 0);
    for (size_t id = 0; id < count; id++) {
        const auto b = tok(id);
        usable[id] = b.second > 0 && id != eot;
        if (!usable[id]) continue;
        const std::string key((const char *)b.first, b.second);
        auto it = owners.find(key);
        if (it == owners.end()) owners.emplace(key, (int64_t)id);
        else it->second = -1;
    }
    for (int c = 0; c < 256; c++) {
        const auto it = owners.find(std::string(1, (char)c));
        if (it == owners.end() || it->second < 0)
            return hs::fail(HS_MODEL_ERROR, HS_MODEL_VOCABULARY,
                            "byte " + std::to_string(c) + " has no single-byte token, or two");
        t->byte_tokens[c] = (uint32_t)it->second;
    }
    t->rules.reserve(n_merges);
    for (size_t r = 0; r < n_merges; r++) {
        const uint32_t l = merges[2 * r], rr = merges[2 * r + 1];
        auto fault = [&](const char *why) {
            return hs::fail(HS_MODEL_ERROR, HS_MODEL_VOCABULARY, "merge " + std::to_string(r) + ": " + why);
        };
        if (l >= count || rr >= count) return fault("a part is not in the vocabulary");
        if (!usable[l] || !usable[rr]) return fault("a part is <|endoftext|> or has no bytes");
        const auto a = tok(l), b = tok(rr);
        std::string joined((const char *)a.first, a.second);
        joined.append((const char *)b.first, b.second);
        const auto it = owners.find(joined);
        if (it == owners.end()) return fault("no token has the joined bytes");
        if (it->second < 0) return fault("two or more tokens have the joined bytes");
        if (!t->rules.emplace(pair_code(l, rr), PairRule{(uint32_t)r, (uint32_t)it->second}).second)
            return fault("the pair occurs two times");
    }
    *out = t.release();
    return HS_OK;
}

// Tokenizer::encode_into (mod.rs:183-201).
void encode(const tc_tokenizer &t, const uint8_t *data, size_t len, std::vector<uint32_t> &ids) {
    Chars run;
    std::vector<uint32_t> symbols;
    PieceJoiner joiner(t.rules);
    size_t i = 0;
    while (i < len) {
        // the maximal well-formed run at i
        run.off.clear();
        run.cp.clear();
        size_t j = i;
        uint32_t cp;
        size_t k;
        while (j < len && (k = utf8_char(data + j, len - j, &cp)) != 0) {
            run.off.push_back((uint32_t)(j - i));
            run.cp.push_back(cp);
            j += k;
        }
        run.off.push_back((uint32_t)(j - i));
        for (size_t c = 0; c < run.cp.size();) {
            const size_t nc = first_piece(run, c);
            symbols.clear();
            for (size_t b = run.off[c]; b < run.off[c + nc]; b++) symbols.push_back(t.byte_tokens[data[i + b]]);
            joiner.run(symbols, ids);
            c += nc;
        }
        if (j < len) {  // a byte outside well-formed UTF-8 is its single-byte token
            ids.push_back(t.byte_tokens[data[j]]);
            j++;
        }
        i = j;
    }
}

}  // namespace

extern "C" hs_status tc_tokenizer_new(const uint8_t *token_bytes, const size_t *token_offsets, size_t count,
                                      uint32_t eot, const uint32_t *merges, size_t n_merges,
                                      tc_tokenizer **out) {
    hs::clear_error();
    if (!out || (count && (!token_bytes || !token_offsets)) || (n_merges && !merges))
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    *out = nullptr;
    return make_tokenizer(count, [&](size_t id) {
        return std::make_pair(token_bytes + token_offsets[id], token_offsets[id + 1] - token_offsets[id]);
    }, eot, merges, n_merges, out);
}

extern "C" hs_status tc_tokenizer_for_model(const hs_model *model, tc_tokenizer **out) {
    hs::clear_error();
    if (!model || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    *out = nullptr;
    const uint32_t *pairs = nullptr;
    const size_t nm = hs_model_merges(model, &pairs);
    return make_tokenizer(hs_model_vocab(model), [&](size_t id) {
        const uint8_t *p = nullptr;
        size_t n = 0;
        if (hs_model_token(model, (uint32_t)id, &p, &n) != HS_OK) return std::make_pair((const uint8_t *)nullptr, (size_t)0);
        return std::make_pair(p, n);
    }, hs_model_eot(model), pairs, nm, out);
}

extern "C" void tc_tokenizer_free(tc_tokenizer *t) { delete t; }

extern "C" hs_status tc_tokenize(const tc_tokenizer *t, const uint8_t *data, size_t len, uint32_t *ids,
                                 size_t cap, size_t *count) {
    hs::clear_error();
    if (!t || !count || (len && !data) || (cap && !ids)) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    std::vector<uint32_t> out;
    encode(*t, data, len, out);
    *count = out.size();
    if (out.size() > cap) return hs::fail(HS_LENGTH_MISMATCH, 0, "the output holds " + std::to_string(cap) + " ids, " + std::to_string(out.size()) + " are needed");
    std::memcpy(ids, out.data(), out.size() * sizeof(uint32_t));
    return HS_OK;
}

extern "C" size_t tc_pretokenize(const uint8_t *text, size_t len, size_t *ends, size_t cap) {
    Chars run;
    size_t j = 0, k;
    uint32_t cp;
    while (j < len && (k = utf8_char(text + j, len - j, &cp)) != 0) {
        run.off.push_back((uint32_t)j);
        run.cp.push_back(cp);
        j += k;
    }
    if (j != len) return SIZE_MAX;  // not well-formed UTF-8
    run.off.push_back((uint32_t)j);
    size_t n = 0;
    for (size_t c = 0; c < run.cp.size();) {
        c += first_piece(run, c);
        if (n < cap) ends[n] = run.off[c];
        n++;
    }
    return n;
}
