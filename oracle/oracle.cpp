// The oracle: a CPU restatement of the reference HardShell engine, coder, block payload and
// seeded test builder. TEST INFRASTRUCTURE ONLY: the tests, the smoke check and the CPU
// baseline of the benchmark load it as the checker; the product never does.
//
// Build: see oracle/build.sh (g++ -O2 -mavx2 -ffp-contract=off; no fast-math, so the f64
// builder follows IEEE 754 exactly as the Rust reference does).
//
// Every section cites the reference file:line it restates. Where a rule must be alike (an
// integer rule, a table, a byte layout), the code states the same rule in its own form.

#include "oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <limits>
#include <memory>
#include <string>
#include <thread>
#include <vector>

typedef __int128 i128;
typedef unsigned __int128 u128;

namespace {

// ============================================================================================
// 1. Integer rules — crates/hardshell/src/int.rs
// ============================================================================================

// shift_round (int.rs:110-124): floor((p + 2^(s-1)) / 2^s); s = 0 gives p; s > max gives 0.
inline i128 shift_round(i128 p, unsigned s, unsigned max_shift) {
    if (s == 0) return p;
    if (s > max_shift) return 0;
    u128 half = (u128)1 << (s - 1);
    i128 q = (i128)((u128)p + half);  // wrapping add, as the reference
    return q >> s;                    // arithmetic shift (gcc), a floor division
}

// rescale (int.rs:63-67): the exact product in i128, max shift 95.
inline i128 rescale(int64_t x, int32_t m, uint8_t s) {
    return shift_round((i128)x * (i128)m, s, 95);
}

// rescale_wide (int.rs:85-90): wrapping i128 product, max shift 126.
inline i128 rescale_wide(i128 x, int32_t m, uint8_t s) {
    i128 p = (i128)((u128)x * (u128)(i128)m);
    return shift_round(p, s, 126);
}

// rescale_wide_offset (int.rs:102-106).
inline i128 rescale_wide_offset(i128 x, int32_t m, i128 c, uint8_t s) {
    i128 p = (i128)((u128)x * (u128)(i128)m + (u128)c);
    return shift_round(p, s, 126);
}

// clamp (int.rs:131-134): max(lo, min(x, hi)); lo wins when the bounds cross.
inline int64_t clamp64(int64_t x, int64_t lo, int64_t hi) {
    int64_t u = x < hi ? x : hi;
    return u > lo ? u : lo;
}

// clamp_wide (int.rs:138-147).
inline int64_t clamp_wide(i128 x, int64_t lo, int64_t hi) {
    i128 u = x < (i128)hi ? x : (i128)hi;
    return (int64_t)(u > (i128)lo ? u : (i128)lo);
}

inline int8_t clamp_act_i8(i128 x) { return (int8_t)clamp_wide(x, -127, 127); }
inline int16_t clamp_act_i16(i128 x) { return (int16_t)clamp_wide(x, -32767, 32767); }
inline int32_t clamp_i32(i128 x, int32_t lo, int32_t hi) { return (int32_t)clamp_wide(x, lo, hi); }

// floor_div (int.rs:41-44) for b > 0.
inline int64_t floor_div(int64_t a, int64_t b) {
    int64_t q = a / b, r = a % b;
    return (r != 0 && r < 0) ? q - 1 : q;
}

// isqrt_u128 (int.rs:213-233): the exact floor square root. This form is the bitwise
// (digit-by-digit, base 4) method.
inline u128 isqrt_u128(u128 x) {
    u128 bit = (u128)1 << 126;
    while (bit > x) bit >>= 2;
    u128 rem = x, res = 0;
    while (bit != 0) {
        if (rem >= res + bit) {
            rem -= res + bit;
            res = (res >> 1) + bit;
        } else {
            res >>= 1;
        }
        bit >>= 2;
    }
    return res;
}

// rescale_clamp (kernels/fast.rs:242-253): the same value as clamp_wide(rescale(..)).
inline int64_t rescale_clamp(int64_t x, int32_t m, uint8_t s, int64_t lo, int64_t hi) {
    return clamp_wide(rescale(x, m, s), lo, hi);
}

// Table::lookup (int.rs:262-274): the index is clamped to the table.
template <typename T>
inline T table_lookup(const std::vector<T> &t, int64_t index) {
    int64_t i = clamp64(index, 0, (int64_t)t.size() - 1);
    return t[(size_t)i];
}

constexpr int32_t RES = (1 << 30) - 1;          // gpt2/mod.rs:116
constexpr int64_t SCORE_LIMIT = (int64_t)1 << 40;  // gpt2/mod.rs:119

// ============================================================================================
// 2. LayerNorm, softmax, logits — layernorm.rs:201-256, softmax.rs:78-104, logits.rs:62-72
// ============================================================================================

struct LayerNorm {
    std::vector<int16_t> g;
    std::vector<int32_t> b;
    int32_t m = 0;
    uint8_t s = 0;
};

struct LnConst {
    uint8_t k = 0, j = 0;
    uint64_t eps = 1;
};

// Writes narrow(y) for each element; bits 8 gives i8, 16 gives i16.
template <typename OutT>
void layernorm_apply(const LayerNorm &ln, LnConst c, uint8_t beta_frac, const int32_t *x,
                     OutT *out) {
    const size_t n = ln.g.size();
    int64_t sum = 0;
    for (size_t i = 0; i < n; i++) sum += x[i];
    const int64_t mean = floor_div(sum, (int64_t)n);
    u128 sq = 0;
    for (size_t i = 0; i < n; i++) {
        int64_t d = (int64_t)x[i] - mean;
        uint64_t a = d < 0 ? (uint64_t)(-d) : (uint64_t)d;
        sq += (u128)a * a;
    }
    const u128 var = sq / (u128)n;
    const u128 root = isqrt_u128((var << (2 * (unsigned)c.j)) + (u128)c.eps);
    const u128 inv_u = ((u128)1 << c.k) / (root > 0 ? root : 1);
    const i128 inv = (i128)inv_u;
    for (size_t i = 0; i < n; i++) {
        const i128 centred = (i128)((int64_t)x[i] - mean);
        const i128 t = centred * inv * (i128)ln.g[i];
        i128 y;
        if (beta_frac == 0) {
            y = rescale_wide(t, ln.m, ln.s) + (i128)ln.b[i];
        } else {
            const i128 cc = (i128)ln.b[i] << (ln.s - beta_frac);
            y = rescale_wide_offset(t, ln.m, cc, ln.s);
        }
        if (sizeof(OutT) == 1)
            out[i] = (OutT)clamp_act_i8(y);
        else
            out[i] = (OutT)clamp_act_i16(y);
    }
}

// softmax: d = max - s; e = table[clamp(d)]; p = floor_div(e << P, sum e).
void softmax_row(const int64_t *scores, size_t n, const std::vector<int32_t> &table, uint8_t p,
                 int64_t *out) {
    int64_t mx = scores[0];
    for (size_t j = 1; j < n; j++) mx = std::max(mx, scores[j]);
    int64_t sum = 0;
    for (size_t j = 0; j < n; j++) {
        int64_t d = clamp_wide((i128)mx - (i128)scores[j], 0, INT64_MAX);
        int64_t e = table_lookup(table, d);
        out[j] = e;
        sum += e;
    }
    for (size_t j = 0; j < n; j++) out[j] = floor_div(out[j] << p, sum);
}

void logits_to_weights(const int64_t *logits, size_t n, const std::vector<uint64_t> &table,
                       uint64_t *out) {
    int64_t mx = logits[0];
    for (size_t v = 1; v < n; v++) mx = std::max(mx, logits[v]);
    for (size_t v = 0; v < n; v++) {
        int64_t d = clamp_wide((i128)mx - (i128)logits[v], 0, INT64_MAX);
        out[v] = table_lookup(table, d);
    }
}

// ============================================================================================
// 3. A small JSON reader for the .hsm header (hsm/header.rs). Well-formed input only.
// ============================================================================================

struct JV {
    enum Kind { OBJ, ARR, STR, NUM } kind = NUM;
    std::vector<std::pair<std::string, JV>> obj;
    std::vector<JV> arr;
    std::string str;
    uint64_t num = 0;
    const JV *get(const char *k) const {
        for (auto &p : obj)
            if (p.first == k) return &p.second;
        return nullptr;
    }
};

struct JsonReader {
    const char *p, *e;
    bool ok = true;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    JV value() {
        ws();
        JV v;
        if (p >= e) { ok = false; return v; }
        if (*p == '{') {
            v.kind = JV::OBJ;
            p++;
            ws();
            if (p < e && *p == '}') { p++; return v; }
            while (ok) {
                ws();
                JV k = value();
                if (k.kind != JV::STR) { ok = false; break; }
                ws();
                if (p >= e || *p != ':') { ok = false; break; }
                p++;
                JV val = value();
                v.obj.emplace_back(k.str, std::move(val));
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == '}') { p++; break; }
                ok = false;
            }
        } else if (*p == '[') {
            v.kind = JV::ARR;
            p++;
            ws();
            if (p < e && *p == ']') { p++; return v; }
            while (ok) {
                v.arr.push_back(value());
                ws();
                if (p < e && *p == ',') { p++; continue; }
                if (p < e && *p == ']') { p++; break; }
                ok = false;
            }
        } else if (*p == '"') {
            v.kind = JV::STR;
            p++;
            while (p < e && *p != '"') v.str.push_back(*p++);
            if (p >= e) ok = false; else p++;
        } else if (*p >= '0' && *p <= '9') {
            v.kind = JV::NUM;
            while (p < e && *p >= '0' && *p <= '9') v.num = v.num * 10 + (uint64_t)(*p++ - '0');
        } else {
            ok = false;
        }
        return v;
    }
};

// ============================================================================================
// 4. The model — gpt2/model.rs:292-343 (tensor names: gpt2/mod.rs:39-76)
// ============================================================================================

struct RowRescale {
    std::vector<int32_t> m;
    uint8_t s = 0;
};

struct Linear {
    size_t rows = 0, cols = 0;
    std::vector<int8_t> w;  // [rows, cols]
    std::vector<int32_t> b;
    RowRescale r;
};

struct Gelu {
    bool wide = false;
    std::vector<int8_t> t8;
    std::vector<int16_t> t16;
    int64_t off = 0;
    int64_t lo() const { return -off; }
    int64_t hi() const { return off - 1; }
    // GeluTable::apply (gelu.rs:58-62)
    int64_t apply(int64_t x) const {
        int64_t c = clamp64(x, -off, off - 1);
        return wide ? (int64_t)table_lookup(t16, c + off) : (int64_t)table_lookup(t8, c + off);
    }
};

struct Block {
    LayerNorm ln1, ln2;
    Linear c_attn, c_proj, c_fc, mlp_proj;
    int32_t score_m = 0, out_m = 0;
    uint8_t score_s = 0, out_s = 0;
    Gelu gelu;
};

}  // namespace

struct or_model {
    uint32_t n_layer = 0, n_head = 0, d = 0, f = 0, vocab = 0, n_ctx = 0, eot = 0, hd = 0;
    LnConst lnc;
    uint8_t softmax_p = 0, ln_f_bits = 8, ln_beta_frac = 0;
    std::vector<int8_t> wte, wpe;
    RowRescale embed, logit, pos;
    std::vector<Block> blocks;
    LayerNorm ln_f;
    std::vector<int32_t> attn_exp;
    std::vector<uint64_t> logits_exp;
    std::vector<std::vector<uint8_t>> vocab_bytes;
    bool wide() const {
        if (ln_f_bits == 16 || ln_beta_frac > 0) return true;
        for (auto &b : blocks)
            if (b.gelu.wide) return true;
        return false;
    }
};

namespace {

struct RawTensor {
    std::string dtype;
    std::vector<uint64_t> shape;
    const uint8_t *data = nullptr;
    uint64_t length = 0;
    int shift = -1;
};

template <typename T>
std::vector<T> take_vec(const std::map<std::string, RawTensor> &ts, const std::string &name,
                        bool &ok) {
    auto it = ts.find(name);
    if (it == ts.end()) { ok = false; return {}; }
    std::vector<T> v(it->second.length / sizeof(T));
    std::memcpy(v.data(), it->second.data, v.size() * sizeof(T));
    return v;
}

int shift_of(const std::map<std::string, RawTensor> &ts, const std::string &name, bool &ok) {
    auto it = ts.find(name);
    if (it == ts.end() || it->second.shift < 0) { ok = false; return 0; }
    return it->second.shift;
}

}  // namespace

extern "C" or_model *or_model_load(const uint8_t *bytes, size_t len) {
    if (len < 16 || std::memcmp(bytes, "HSHLMDL\0", 8) != 0) return nullptr;
    uint32_t header_len;
    std::memcpy(&header_len, bytes + 12, 4);
    if (16 + (size_t)header_len > len) return nullptr;
    JsonReader jr{(const char *)bytes + 16, (const char *)bytes + 16 + header_len};
    JV h = jr.value();
    if (!jr.ok || h.kind != JV::OBJ) return nullptr;
    const JV *model = h.get("model"), *vocab = h.get("vocabulary"), *tensors = h.get("tensors");
    if (!model || !vocab || !tensors) return nullptr;
    auto num = [](const JV *o, const char *k) -> uint64_t {
        const JV *v = o ? o->get(k) : nullptr;
        return v ? v->num : 0;
    };
    auto m = std::make_unique<or_model>();
    m->n_layer = (uint32_t)num(model, "n_layer");
    m->n_head = (uint32_t)num(model, "n_head");
    m->d = (uint32_t)num(model, "d_model");
    m->f = (uint32_t)num(model, "d_ff");
    m->vocab = (uint32_t)num(model, "vocab_size");
    m->n_ctx = (uint32_t)num(model, "n_ctx");
    m->eot = (uint32_t)num(model, "eot_token");
    if (m->n_head == 0 || m->d % m->n_head != 0) return nullptr;
    m->hd = m->d / m->n_head;
    const JV *c = model->get("constants");
    m->lnc.k = (uint8_t)num(c, "ln_k");
    m->lnc.j = (uint8_t)num(c, "ln_j");
    m->lnc.eps = num(c, "ln_eps");
    m->softmax_p = (uint8_t)num(c, "softmax_p");
    if (c && c->get("ln_f_bits")) m->ln_f_bits = (uint8_t)num(c, "ln_f_bits");
    if (c && c->get("ln_beta_frac")) m->ln_beta_frac = (uint8_t)num(c, "ln_beta_frac");
    // Vocabulary: u16 length + bytes per token (hsm/reader.rs:156-180).
    uint64_t voff = num(vocab, "offset"), vlen = num(vocab, "length");
    if (voff + vlen > len) return nullptr;
    size_t pos = 0;
    for (uint32_t t = 0; t < m->vocab; t++) {
        if (pos + 2 > vlen) return nullptr;
        uint16_t l;
        std::memcpy(&l, bytes + voff + pos, 2);
        pos += 2;
        if (pos + l > vlen) return nullptr;
        m->vocab_bytes.emplace_back(bytes + voff + pos, bytes + voff + pos + l);
        pos += l;
    }
    std::map<std::string, RawTensor> ts;
    for (auto &e : tensors->arr) {
        RawTensor r;
        const JV *name = e.get("name"), *dtype = e.get("dtype"), *shape = e.get("shape");
        if (!name || !dtype || !shape) return nullptr;
        r.dtype = dtype->str;
        for (auto &d : shape->arr) r.shape.push_back(d.num);
        uint64_t off = num(&e, "offset");
        r.length = num(&e, "length");
        if (off + r.length > len) return nullptr;
        r.data = bytes + off;
        if (e.get("shift")) r.shift = (int)num(&e, "shift");
        ts[name->str] = r;
    }
    bool ok = true;
    auto rows = [&](const std::string &n) {
        RowRescale r;
        r.m = take_vec<int32_t>(ts, n, ok);
        r.s = (uint8_t)shift_of(ts, n, ok);
        return r;
    };
    auto lin = [&](const std::string &p, size_t rws, size_t cols) {
        Linear l;
        l.rows = rws;
        l.cols = cols;
        l.w = take_vec<int8_t>(ts, p + ".w", ok);
        l.b = take_vec<int32_t>(ts, p + ".b", ok);
        l.r = rows(p + ".rescale");
        if (l.w.size() != rws * cols || l.b.size() != rws || l.r.m.size() != rws) ok = false;
        return l;
    };
    auto lnorm = [&](const std::string &p) {
        LayerNorm n;
        n.g = take_vec<int16_t>(ts, p + ".g", ok);
        n.b = take_vec<int32_t>(ts, p + ".b", ok);
        RowRescale r = rows(p + ".rescale");
        n.m = r.m.empty() ? 0 : r.m[0];
        n.s = r.s;
        return n;
    };
    const size_t d = m->d, f = m->f;
    m->wte = take_vec<int8_t>(ts, "wte", ok);
    m->embed = rows("wte.rescale_embed");
    m->logit = rows("wte.rescale_logits");
    m->wpe = take_vec<int8_t>(ts, "wpe", ok);
    m->pos = rows("wpe.rescale");
    for (uint32_t l = 0; l < m->n_layer; l++) {
        std::string p = "h." + std::to_string(l);
        Block b;
        b.ln1 = lnorm(p + ".ln_1");
        b.c_attn = lin(p + ".attn.c_attn", 3 * d, d);
        RowRescale sc = rows(p + ".attn.score.rescale");
        RowRescale ao = rows(p + ".attn.out.rescale");
        b.score_m = sc.m.empty() ? 0 : sc.m[0];
        b.score_s = sc.s;
        b.out_m = ao.m.empty() ? 0 : ao.m[0];
        b.out_s = ao.s;
        b.c_proj = lin(p + ".attn.c_proj", d, d);
        b.ln2 = lnorm(p + ".ln_2");
        b.c_fc = lin(p + ".mlp.c_fc", f, d);
        auto gt = ts.find(p + ".mlp.gelu");
        if (gt == ts.end()) return nullptr;
        if (gt->second.dtype == "i16") {
            b.gelu.wide = true;
            b.gelu.t16 = take_vec<int16_t>(ts, p + ".mlp.gelu", ok);
            b.gelu.off = (int64_t)b.gelu.t16.size() / 2;
        } else {
            b.gelu.t8 = take_vec<int8_t>(ts, p + ".mlp.gelu", ok);
            b.gelu.off = (int64_t)b.gelu.t8.size() / 2;
        }
        b.mlp_proj = lin(p + ".mlp.c_proj", d, f);
        m->blocks.push_back(std::move(b));
    }
    m->ln_f = lnorm("ln_f");
    m->attn_exp = take_vec<int32_t>(ts, "attn_exp", ok);
    m->logits_exp = take_vec<uint64_t>(ts, "logits_exp", ok);
    if (!ok || m->wte.size() != (size_t)m->vocab * d || m->wpe.size() != (size_t)m->n_ctx * d)
        return nullptr;
    return m.release();
}

extern "C" void or_model_free(or_model *m) { delete m; }

extern "C" void or_model_dims(const or_model *m, uint32_t *dims) {
    dims[0] = m->n_layer;
    dims[1] = m->n_head;
    dims[2] = m->d;
    dims[3] = m->f;
    dims[4] = m->vocab;
    dims[5] = m->n_ctx;
    dims[6] = m->eot;
    dims[7] = m->wide() ? 1 : 0;
}

// ============================================================================================
// 5. The reference session — gpt2/reference.rs:144-329 (context rule: gpt2/context.rs:133-155)
// ============================================================================================

namespace {

inline int32_t dot_i8(const int8_t *a, const int8_t *b, size_t n) {
    int32_t s = 0;
    for (size_t i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

void matvec_i8(const Linear &l, const int8_t *x, int32_t *out) {
    for (size_t r = 0; r < l.rows; r++) out[r] = dot_i8(&l.w[r * l.cols], x, l.cols);
}

}  // namespace

struct or_session {
    const or_model *m;
    uint32_t k;  // overlap
    size_t pos = 0;
    std::vector<uint32_t> toks;
    std::vector<int8_t> kc, vc;  // [L][n_ctx][d]
    std::vector<int32_t> x, acc;
    std::vector<int8_t> a, qkv, att, g;
    std::vector<int16_t> g16, a16;
    std::vector<int64_t> acc64, scores, probs, head, logits;
    std::vector<uint64_t> weights;
    // probes of the last forward row
    bool probing = false;
    std::vector<int32_t> p_embed, p_block0;
    std::vector<int8_t> p_ln1, p_qkv, p_att;

    or_session(const or_model *mm, uint32_t kk) : m(mm), k(kk) {
        const size_t d = m->d, L = m->n_layer, C = m->n_ctx;
        toks.assign(C, 0);
        kc.assign(L * C * d, 0);
        vc.assign(L * C * d, 0);
        x.assign(d, 0);
        a.assign(d, 0);
        acc.assign(std::max<size_t>({3 * d, (size_t)m->f, (size_t)m->vocab}), 0);
        qkv.assign(3 * d, 0);
        att.assign(d, 0);
        g.assign(m->f, 0);
        g16.assign(m->f, 0);
        a16.assign(d, 0);
        acc64.assign(std::max<size_t>(d, m->vocab), 0);
        scores.assign(C, 0);
        probs.assign(C, 0);
        head.assign(m->hd, 0);
        logits.assign(m->vocab, 0);
        weights.assign(m->vocab, 0);
    }

    void embed(uint32_t tok, size_t t) {
        const size_t d = m->d;
        const int32_t tm = m->embed.m[tok], pm = m->pos.m[t];
        for (size_t j = 0; j < d; j++) {
            i128 v = rescale(m->wte[tok * d + j], tm, m->embed.s) +
                     rescale(m->wpe[t * d + j], pm, m->pos.s);
            x[j] = clamp_i32(v, -RES, RES);
        }
    }

    // reference.rs:224-231
    void add_to_residual(const Linear &l, const int8_t *in) {
        matvec_i8(l, in, acc.data());
        for (size_t r = 0; r < l.rows; r++) {
            i128 delta = rescale((int64_t)acc[r] + l.b[r], l.r.m[r], l.r.s);
            x[r] = clamp_i32((i128)x[r] + delta, -RES, RES);
        }
    }

    // reference.rs:234-286
    void attention(const Block &b, size_t layer, size_t t) {
        const size_t d = m->d, hd = m->hd, C = m->n_ctx;
        layernorm_apply(b.ln1, m->lnc, m->ln_beta_frac, x.data(), a.data());
        if (probing && layer == 0) p_ln1 = a;
        matvec_i8(b.c_attn, a.data(), acc.data());
        for (size_t r = 0; r < 3 * d; r++)
            qkv[r] = clamp_act_i8(rescale((int64_t)acc[r] + b.c_attn.b[r], b.c_attn.r.m[r],
                                          b.c_attn.r.s));
        if (probing && layer == 0) p_qkv = qkv;
        const size_t base = layer * C * d;
        std::memcpy(&kc[base + t * d], &qkv[d], d);
        std::memcpy(&vc[base + t * d], &qkv[2 * d], d);
        const size_t n = t + 1;
        for (size_t h = 0; h < m->n_head; h++) {
            const size_t off = h * hd;
            for (size_t j = 0; j < n; j++) {
                int32_t dt = dot_i8(&qkv[off], &kc[base + j * d + off], hd);
                scores[j] = clamp_wide(rescale(dt, b.score_m, b.score_s), -SCORE_LIMIT,
                                       SCORE_LIMIT);
            }
            softmax_row(scores.data(), n, m->attn_exp, m->softmax_p, probs.data());
            std::fill(head.begin(), head.end(), 0);
            for (size_t j = 0; j < n; j++)
                for (size_t c = 0; c < hd; c++)
                    head[c] += probs[j] * (int64_t)vc[base + j * d + off + c];
            for (size_t c = 0; c < hd; c++)
                att[off + c] = clamp_act_i8(rescale(head[c], b.out_m, b.out_s));
        }
        if (probing && layer == 0) p_att = att;
        add_to_residual(b.c_proj, att.data());
    }

    // reference.rs:289-329
    void mlp(const Block &b) {
        const size_t d = m->d, f = m->f;
        layernorm_apply(b.ln2, m->lnc, m->ln_beta_frac, x.data(), a.data());
        matvec_i8(b.c_fc, a.data(), acc.data());
        const int64_t lo = b.gelu.lo(), hi = b.gelu.hi();
        if (!b.gelu.wide) {
            for (size_t r = 0; r < f; r++) {
                int64_t in = clamp_wide(
                    rescale((int64_t)acc[r] + b.c_fc.b[r], b.c_fc.r.m[r], b.c_fc.r.s), lo, hi);
                g[r] = (int8_t)b.gelu.apply(in);
            }
            add_to_residual(b.mlp_proj, g.data());
        } else {
            for (size_t r = 0; r < f; r++) {
                int64_t in = clamp_wide(
                    rescale((int64_t)acc[r] + b.c_fc.b[r], b.c_fc.r.m[r], b.c_fc.r.s), lo, hi);
                g16[r] = (int16_t)b.gelu.apply(in);
            }
            const Linear &l = b.mlp_proj;
            for (size_t r = 0; r < d; r++) {
                int64_t s = 0;
                for (size_t c = 0; c < f; c++) s += (int64_t)l.w[r * f + c] * g16[c];
                i128 delta = rescale(s + l.b[r], l.r.m[r], l.r.s);
                x[r] = clamp_i32((i128)x[r] + delta, -RES, RES);
            }
        }
    }

    // reference.rs:170-205
    void forward(uint32_t tok, bool want_logits) {
        const size_t t = pos, d = m->d, V = m->vocab;
        toks[t] = tok;
        embed(tok, t);
        if (probing) p_embed = x;
        for (size_t l = 0; l < m->n_layer; l++) {
            attention(m->blocks[l], l, t);
            mlp(m->blocks[l]);
            if (probing && l == 0) p_block0 = x;
        }
        if (!want_logits) {
            pos = t + 1;
            return;
        }
        if (m->ln_f_bits == 16) {
            layernorm_apply(m->ln_f, m->lnc, m->ln_beta_frac, x.data(), a16.data());
            for (size_t v = 0; v < V; v++) {
                int64_t s = 0;
                for (size_t c = 0; c < d; c++) s += (int64_t)m->wte[v * d + c] * a16[c];
                logits[v] = clamp_wide(rescale(s, m->logit.m[v], m->logit.s), -SCORE_LIMIT,
                                       SCORE_LIMIT);
            }
        } else {
            layernorm_apply(m->ln_f, m->lnc, m->ln_beta_frac, x.data(), a.data());
            for (size_t v = 0; v < V; v++) {
                int32_t s = dot_i8(&m->wte[v * d], a.data(), d);
                logits[v] = clamp_wide(rescale(s, m->logit.m[v], m->logit.s), -SCORE_LIMIT,
                                       SCORE_LIMIT);
            }
        }
        logits_to_weights(logits.data(), V, m->logits_exp, weights.data());
        pos = t + 1;
    }

    // reference.rs:144-162
    int step(uint32_t token) {
        const size_t C = m->n_ctx;
        if ((size_t)k + 2 > C) return -1;
        if (token >= m->vocab) return -1;
        if (pos >= C) {
            std::vector<uint32_t> kept(toks.begin() + (C - k), toks.begin() + C);
            pos = 0;
            forward(m->eot, false);
            for (uint32_t t : kept) forward(t, false);
        }
        forward(token, true);
        return 0;
    }
};

extern "C" or_session *or_session_new(const or_model *m, uint32_t overlap) {
    return new or_session(m, overlap);
}
extern "C" void or_session_free(or_session *s) { delete s; }
extern "C" int or_session_start_block(or_session *s, uint64_t *weights) {
    s->pos = 0;
    int r = s->step(s->m->eot);
    if (r == 0 && weights) std::memcpy(weights, s->weights.data(), 8 * s->weights.size());
    return r;
}
extern "C" int or_session_step(or_session *s, uint32_t token, uint64_t *weights) {
    int r = s->step(token);
    if (r == 0 && weights) std::memcpy(weights, s->weights.data(), 8 * s->weights.size());
    return r;
}
extern "C" uint32_t or_session_position(const or_session *s) { return (uint32_t)s->pos; }
extern "C" int or_session_probe(or_session *s, uint32_t token, int32_t *x_after_embed,
                                int8_t *ln1_out, int8_t *qkv_out, int8_t *att_out,
                                int32_t *x_after_block0) {
    s->probing = true;
    int r = s->step(token);
    s->probing = false;
    if (r != 0) return r;
    const size_t d = s->m->d;
    std::memcpy(x_after_embed, s->p_embed.data(), 4 * d);
    std::memcpy(ln1_out, s->p_ln1.data(), d);
    std::memcpy(qkv_out, s->p_qkv.data(), 3 * d);
    std::memcpy(att_out, s->p_att.data(), d);
    std::memcpy(x_after_block0, s->p_block0.data(), 4 * d);
    return 0;
}

// ============================================================================================
// 6. Integer rule exports (for the tests)
// ============================================================================================

extern "C" void or_rescale(int64_t x, int32_t m, uint8_t s, int64_t *hi, uint64_t *lo) {
    i128 r = rescale(x, m, s);
    *hi = (int64_t)(r >> 64);
    *lo = (uint64_t)r;
}
extern "C" void or_rescale_wide(int64_t xhi, uint64_t xlo, int32_t m, uint8_t s, int64_t *hi,
                                uint64_t *lo) {
    i128 x = (i128)(((u128)(uint64_t)xhi << 64) | xlo);
    i128 r = rescale_wide(x, m, s);
    *hi = (int64_t)(r >> 64);
    *lo = (uint64_t)r;
}
extern "C" int64_t or_rescale_clamp(int64_t x, int32_t m, uint8_t s, int64_t lo, int64_t hi) {
    return rescale_clamp(x, m, s, lo, hi);
}
extern "C" int64_t or_floor_div(int64_t a, int64_t b) { return floor_div(a, b); }
extern "C" uint64_t or_isqrt_u128(uint64_t xhi, uint64_t xlo) {
    return (uint64_t)isqrt_u128(((u128)xhi << 64) | xlo);
}
extern "C" int or_layernorm(const int32_t *x, size_t n, const int16_t *gamma, const int32_t *beta,
                            int32_t m, uint8_t s, uint8_t beta_frac, uint8_t k, uint8_t j,
                            uint64_t eps, int bits, void *out) {
    LayerNorm ln;
    ln.g.assign(gamma, gamma + n);
    ln.b.assign(beta, beta + n);
    ln.m = m;
    ln.s = s;
    LnConst c;
    c.k = k;
    c.j = j;
    c.eps = eps;
    if (bits == 16)
        layernorm_apply(ln, c, beta_frac, x, (int16_t *)out);
    else
        layernorm_apply(ln, c, beta_frac, x, (int8_t *)out);
    return 0;
}
extern "C" int or_softmax(const int64_t *scores, size_t n, const int32_t *table, size_t len,
                          uint8_t p, int64_t *out) {
    if (n == 0 || len == 0 || p > 30) return -1;
    std::vector<int32_t> t(table, table + len);
    softmax_row(scores, n, t, p, out);
    return 0;
}
extern "C" int or_logits_to_weights(const int64_t *logits, size_t n, const uint64_t *table,
                                    size_t len, uint64_t *out) {
    if (n == 0 || len == 0) return -1;
    std::vector<uint64_t> t(table, table + len);
    logits_to_weights(logits, n, t, out);
    return 0;
}

// ============================================================================================
// 7. Frequency tables and the range coder — taco-coder/src/{freq,encoder,decoder}.rs
// ============================================================================================

namespace {

// FreqTable::from_weights (freq.rs:103-149). starts[i] = sum of f_j for j < i (u32).
bool from_weights(const uint64_t *w, size_t n, uint32_t bits, std::vector<uint32_t> &starts) {
    const uint64_t total = (uint64_t)1 << bits;
    if (n == 0 || (uint64_t)n > total) return false;
    u128 W = 0;
    size_t largest = 0;
    uint64_t best = 0;
    for (size_t i = 0; i < n; i++) {
        W += w[i];
        if (w[i] > best) {
            best = w[i];
            largest = i;
        }
    }
    const bool all_zero = (W == 0);
    if (all_zero) W = n;
    const u128 spare = total - (uint64_t)n;
    starts.resize(n);
    uint64_t acc = 0;
    for (size_t i = 0; i < n; i++) {
        const u128 wi = all_zero ? 1 : w[i];
        const uint64_t q = (uint64_t)(wi * spare / W);
        starts[i] = (uint32_t)acc;
        acc += 1 + q;
    }
    const uint32_t rem = (uint32_t)(total - acc);
    if (rem > 0)
        for (size_t i = largest + 1; i < n; i++) starts[i] += rem;
    return true;
}

inline void interval_of(const std::vector<uint32_t> &st, uint32_t bits, size_t i, uint64_t &start,
                        uint64_t &freq) {
    start = st[i];
    const uint64_t end = (i + 1 < st.size()) ? (uint64_t)st[i + 1] : ((uint64_t)1 << bits);
    freq = end - start;
}

inline size_t find_symbol(const std::vector<uint32_t> &st, uint64_t target) {
    // the largest i with starts[i] <= target (partition point minus one)
    size_t lo = 0, hi = st.size();
    while (lo < hi) {
        size_t mid = (lo + hi) / 2;
        if ((uint64_t)st[mid] <= target) lo = mid + 1; else hi = mid;
    }
    return lo - 1;
}

constexpr uint64_t TOP = (uint64_t)1 << 56;  // taco-coder/src/lib.rs:110-114

// Encoder (encoder.rs:13-212): low is 65 bits wide, a carry rule of LZMA with a 64-bit window.
struct Encoder {
    u128 low = 0;
    uint64_t range = UINT64_MAX;
    uint8_t cache = 0;
    size_t pending = 0;
    std::vector<uint8_t> out;
    size_t nonzero_len = 0;

    void shift_low() {
        const uint8_t carry = (uint8_t)((low >> 64) & 1);
        const uint64_t window = (uint64_t)low;
        if (pending == 0 || window < 0xFF00000000000000ull || carry != 0) {
            if (pending > 0) {
                const uint8_t first = (uint8_t)(cache + carry);
                out.push_back(first);
                if (first != 0) nonzero_len = out.size();
                const uint8_t fill = (uint8_t)(0xFF + carry);
                for (size_t i = 1; i < pending; i++) out.push_back(fill);
                if (fill != 0 && pending > 1) nonzero_len = out.size();
            }
            cache = (uint8_t)(window >> 56);
            pending = 0;
        }
        pending += 1;
        low = (u128)(window << 8);
    }
    void renormalise() {
        while (range < TOP) {
            range <<= 8;
            shift_low();
        }
    }
    void encode_parts(uint64_t start, uint64_t freq, bool is_last, uint32_t bits) {
        const uint64_t r = range >> bits;
        const uint64_t offset = r * start;
        low += offset;
        range = is_last ? range - offset : r * freq;
        renormalise();
    }
    void encode_bit(uint32_t p1, bool bit) {
        const uint64_t bound = (range >> 12) * p1;
        if (bit) {
            range = bound;
        } else {
            low += bound;
            range -= bound;
        }
        renormalise();
    }
    std::vector<uint8_t> finish() {
        const u128 end = low + range;
        for (unsigned k : {64u, 56u}) {
            const u128 mask = ((u128)1 << k) - 1;
            const u128 v = (low + mask) & ~mask;
            if (v < end) {
                low = v;
                break;
            }
        }
        shift_low();
        shift_low();
        while (!out.empty() && out.back() == 0) out.pop_back();
        return out;
    }
};

}  // namespace

struct or_decoder {
    std::vector<uint8_t> in;
    size_t pos = 0;
    uint64_t code = 0, range = UINT64_MAX;
    uint8_t next() { return pos < in.size() ? in[pos++] : (pos++, 0); }
    void renormalise() {
        while (range < TOP) {
            range <<= 8;
            code = (code << 8) | next();
        }
    }
    uint64_t target(uint32_t bits) const {
        const uint64_t r = range >> bits;
        const uint64_t t = code / r;
        const uint64_t last = ((uint64_t)1 << bits) - 1;
        return t < last ? t : last;
    }
    bool decode_interval(uint64_t start, uint64_t freq, uint32_t bits) {
        const uint64_t t = target(bits);
        if (!(t >= start && t - start < freq)) return false;
        const uint64_t r = range >> bits;
        const uint64_t offset = r * start;
        code -= offset;
        const bool is_last = start + freq == ((uint64_t)1 << bits);
        range = is_last ? range - offset : r * freq;
        renormalise();
        return true;
    }
    bool decode_bit(uint32_t p1) {
        const uint64_t bound = (range >> 12) * p1;
        const bool bit = code < bound;
        if (bit) {
            range = bound;
        } else {
            code -= bound;
            range -= bound;
        }
        renormalise();
        return bit;
    }
};

extern "C" int or_freq_from_weights(const uint64_t *w, size_t n, uint32_t bits, uint64_t *freqs) {
    std::vector<uint32_t> st;
    if (bits > 32 || !from_weights(w, n, bits, st)) return -1;
    for (size_t i = 0; i < n; i++) {
        uint64_t s, f;
        interval_of(st, bits, i, s, f);
        freqs[i] = f;
    }
    return 0;
}

extern "C" int or_freq_interval(const uint64_t *w, size_t n, uint32_t bits, uint32_t symbol,
                                uint64_t *start, uint64_t *freq) {
    std::vector<uint32_t> st;
    if (bits > 32 || !from_weights(w, n, bits, st) || symbol >= n) return -1;
    interval_of(st, bits, symbol, *start, *freq);
    return 0;
}

extern "C" int or_freq_find(const uint64_t *w, size_t n, uint32_t bits, uint64_t target,
                            uint32_t *symbol, uint64_t *start, uint64_t *freq) {
    std::vector<uint32_t> st;
    if (bits > 32 || !from_weights(w, n, bits, st) || target >= ((uint64_t)1 << bits)) return -1;
    size_t i = find_symbol(st, target);
    *symbol = (uint32_t)i;
    interval_of(st, bits, i, *start, *freq);
    return 0;
}

extern "C" size_t or_encode_script(const uint64_t *ops, size_t nops, uint8_t *out, size_t cap) {
    Encoder e;
    for (size_t i = 0; i < nops; i++) {
        const uint64_t *o = &ops[4 * i];
        if (o[0] == 0) {
            const uint32_t bits = (uint32_t)o[3];
            e.encode_parts(o[1], o[2], o[1] + o[2] == ((uint64_t)1 << bits), bits);
        } else {
            e.encode_bit((uint32_t)o[1], o[2] != 0);
        }
    }
    std::vector<uint8_t> b = e.finish();
    if (b.size() <= cap) std::memcpy(out, b.data(), b.size());
    return b.size();
}

extern "C" or_decoder *or_decoder_new(const uint8_t *bytes, size_t len) {
    or_decoder *d = new or_decoder;
    d->in.assign(bytes, bytes + len);
    for (int i = 0; i < 8; i++) d->code = (d->code << 8) | d->next();
    return d;
}
extern "C" void or_decoder_free(or_decoder *d) { delete d; }
extern "C" uint64_t or_decoder_target(const or_decoder *d, uint32_t bits) { return d->target(bits); }
extern "C" int or_decoder_decode_interval(or_decoder *d, uint64_t start, uint64_t freq,
                                          uint32_t bits) {
    return d->decode_interval(start, freq, bits) ? 0 : -1;
}
extern "C" int or_decoder_decode_bit(or_decoder *d, uint32_t p1) { return d->decode_bit(p1) ? 1 : 0; }

// ============================================================================================
// 8. The block payload — crates/taco/src/codec.rs:72-126,279-310; payload.rs:20-31
// ============================================================================================

namespace {

void write_varint(uint64_t v, std::vector<uint8_t> &out) {
    for (;;) {
        uint8_t low = (uint8_t)(v & 0x7F);
        v >>= 7;
        if (v == 0) {
            out.push_back(low);
            return;
        }
        out.push_back(low | 0x80);
    }
}

size_t varint_len(uint64_t v) {
    size_t n = 1;
    while (v > 0x7F) {
        v >>= 7;
        n++;
    }
    return n;
}

// read_varint (payload.rs:40-60): minimal LEB128, at most 10 bytes.
bool read_varint(const uint8_t *b, size_t len, uint64_t &value, size_t &used) {
    value = 0;
    unsigned shift = 0;
    for (size_t i = 0; i < len && i < 10; i++) {
        const uint64_t group = b[i] & 0x7F;
        if (i == 9 && group > 1) return false;
        value |= group << shift;
        shift += 7;
        if ((b[i] & 0x80) == 0) {
            if (b[i] == 0 && i > 0) return false;
            used = i + 1;
            return true;
        }
    }
    return false;
}

}  // namespace

// ============================================================================================
// 8b. The logs profile: the match model and the mixer of one block, mixer rule version 1
//     (crates/taco-match/src/{logistic,matcher,mixer,skip}.rs; crates/taco/src/mix.rs).
// ============================================================================================

namespace {

// logistic.rs:25-75: squash over x in -4095..=4095 (units of 1/256 nat) from E[j] = 2^62
// exp(-j/256) by a rounded recurrence, and stretch(p) = the smallest x with squash(x) >= p.
struct Logistic {
    static constexpr int XM = 4095;
    std::vector<uint16_t> sq;
    std::vector<int16_t> st;
    Logistic() {
        const u128 C = (u128)4593706758521714574ull;
        std::vector<u128> e(XM + 1);
        e[0] = (u128)1 << 62;
        for (int j = 0; j < XM; j++) e[j + 1] = (e[j] * C + ((u128)1 << 61)) >> 62;
        sq.assign(2 * XM + 1, 0);
        auto clampp = [](int64_t v) { return (uint16_t)(v < 1 ? 1 : (v > 65535 ? 65535 : v)); };
        for (int x = 0; x <= XM; x++) {
            const u128 d = ((u128)1 << 62) + e[x];
            const int64_t v = (int64_t)((((u128)1 << 78) + d / 2) / d);
            sq[XM + x] = clampp(v);
            sq[XM - x] = clampp(65536 - v);
        }
        st.assign(1 << 16, 0);
        size_t x = 0;
        for (uint32_t q = 0; q < (1u << 16); q++) {
            while (x < sq.size() && sq[x] < q) x++;
            st[q] = (int16_t)((int)std::min<size_t>(x, 2 * XM) - XM);
        }
    }
    uint32_t squash(int64_t x) const { return sq[(size_t)(std::min<int64_t>(std::max<int64_t>(x, -XM), XM) + XM)]; }
    int32_t stretch(uint32_t q) const { return st[std::min<uint32_t>(q, 65535)]; }
};

const Logistic &logistic() {
    static const Logistic t;
    return t;
}

// skip.rs:44-62: a 22-bit hit probability moving to y 2^22 by floor(2 d / (2n + 3)).
struct Adaptive {
    uint32_t hit = 1u << 21;
    uint16_t count = 0;
    void update(bool y, uint16_t limit) {
        const uint32_t n = count, h = hit, den = 2 * n + 3;
        hit = y ? h + (((1u << 22) - h) * 2) / den : h - (h * 2) / den;
        count = (uint16_t)std::min<uint32_t>(n + 1, limit);
    }
};

// mixer.rs:470-480: L - 1 below 16, then one bucket per octave, at most 20.
int mix_bucket(uint32_t len) {
    if (len < 16) return (int)len - 1;
    const int bits = 32 - __builtin_clz(len);
    return std::min(15 + bits - 5, 20);
}

// The mixer of rule version 1 (mixer.rs:49-86 constants, :399-470 update and probability).
struct MixerV1 {
    static constexpr int SETS = 42;
    Adaptive buckets[21];
    int32_t w[SETS][3];
    uint32_t updates[SETS];
    bool pending = false;
    uint32_t p_token = 0, p_q = 0;
    int p_bucket = 0, p_set = 0;
    int32_t p_xs[3] = {0, 0, 0};
    MixerV1() {
        for (int c = 0; c < SETS; c++) {
            w[c][0] = 1 << 16;
            w[c][1] = 1 << 16;
            w[c][2] = 0;
            updates[c] = 0;
        }
    }
    static int64_t rate(uint32_t n) {  // max(16, floor(160 * 64 / (n + 64)))
        const uint32_t r = 160u * 64u / (n + 64u);
        return (int64_t)std::max<uint32_t>(r, 16);
    }
    // rules 2 to 5 and the pending state (mixer.rs:302-315, :452-467)
    uint32_t mix_stats(u128 total, uint64_t wp, bool agree, uint32_t token, uint32_t len) {
        const Logistic &t = logistic();
        uint64_t pg = total ? (uint64_t)(((u128)wp << 16) / total) : 1;
        pg = std::min<uint64_t>(std::max<uint64_t>(pg, 1), 65535);
        const int b = mix_bucket(len);
        const int32_t xs[3] = {t.stretch((uint32_t)pg), t.stretch(buckets[b].hit >> 6), 256};
        const int set = 2 * b + (agree ? 1 : 0);
        int64_t dot = 0;
        for (int i = 0; i < 3; i++) dot += (int64_t)w[set][i] * xs[i];
        int64_t x = (dot + (1 << 15)) >> 16;
        x = std::min<int64_t>(std::max<int64_t>(x, -4095), 4095);
        const uint32_t q = t.squash(x);
        pending = true;
        p_token = token;
        p_q = q;
        p_bucket = b;
        p_set = set;
        for (int i = 0; i < 3; i++) p_xs[i] = xs[i];
        return q;
    }
    void clear() { pending = false; }
    // rule 7 (mixer.rs:399-432)
    void update(uint32_t actual) {
        if (!pending) return;
        pending = false;
        const bool y = actual == p_token;
        const int64_t err = (y ? 65536 : 0) - (int64_t)p_q;
        const uint32_t n = updates[p_set];
        const int64_t lr = rate(n);
        updates[p_set] = std::min<uint32_t>(n + 1, 1u << 20);
        for (int i = 0; i < 3; i++) {
            const int64_t d = ((int64_t)p_xs[i] * err * lr + (1 << 19)) >> 20;
            const int64_t v = std::min<int64_t>(std::max<int64_t>((int64_t)w[p_set][i] + d, -(1 << 22)), 1 << 22);
            w[p_set][i] = (int32_t)v;
        }
        buckets[p_bucket].update(y, 255);
    }
};

// The match model of rule version 1 (matcher.rs:40-90 constants, :318-415 rules).
struct MatchV1 {
    static constexpr int ORDERS = 6, HASH_BITS = 20, VERIFY = 64;
    static constexpr uint32_t MAX_LEN = 65535;
    static constexpr int order_of[ORDERS] = {32, 16, 8, 4, 2, 1};
    std::vector<uint32_t> tables, hist;
    size_t ptr = 0;
    uint32_t len = 0;
    MatchV1() : tables((size_t)ORDERS << HASH_BITS, 0) {}
    bool predict(uint32_t &token, uint32_t &length) const {
        if (len == 0 || ptr >= hist.size()) return false;
        token = hist[ptr];
        length = len;
        return true;
    }
    void observe(uint32_t t) {
        if (len > 0) {
            if (ptr < hist.size() && hist[ptr] == t) {
                ptr++;
                len = std::min(len + 1, MAX_LEN);
            } else {
                len = 0;
            }
        }
        hist.push_back(t);
        const size_t i = hist.size();
        // the slot of each order at position i (rule 1)
        int64_t slots[ORDERS];
        for (int o = 0; o < ORDERS; o++) slots[o] = -1;
        uint64_t acc = 0, bk = 1;
        int next = ORDERS;
        for (size_t k = 1; k <= (size_t)order_of[0] && k <= i; k++) {
            acc += ((uint64_t)hist[i - k] + 1) * bk;
            bk *= 0x9E3779B97F4A7C15ull;
            while (next > 0 && (size_t)order_of[next - 1] == k) {
                const uint64_t x = (acc ^ (acc >> 32)) * 0xD6E8FEB86659FD93ull;
                slots[next - 1] = (int64_t)(x >> (64 - HASH_BITS));
                next--;
            }
        }
        // rule 3.3: the longest verified match, longest order first
        if (len < (uint32_t)order_of[0]) {
            for (int o = 0; o < ORDERS; o++) {
                if ((uint32_t)order_of[o] <= len) break;
                if (slots[o] < 0) continue;
                const uint32_t e = tables[((size_t)o << HASH_BITS) + (size_t)slots[o]];
                if (e == 0) continue;
                const size_t c = e - 1;
                const size_t limit = std::min<size_t>(VERIFY, c);
                uint32_t v = 0;
                while (v < limit && hist[c - v - 1] == hist[i - v - 1]) v++;
                if (v >= (uint32_t)order_of[o]) {
                    ptr = c;
                    len = v;
                    break;
                }
            }
        }
        for (int o = 0; o < ORDERS; o++)
            if (slots[o] >= 0) tables[((size_t)o << HASH_BITS) + (size_t)slots[o]] = (uint32_t)(i + 1);
    }
};

// Rule 6 of Mixer::mix (mixer.rs:491-516) for the statistics total and w[p] = w_p and the
// probability q: w'[i] = max(1, (w[i] m) >> k), then w'[p] = max(1, (R q) >> k).
int mix_apply_q(uint64_t *w, size_t n, uint32_t p, u128 total, uint32_t q) {
    if (p >= n) return 4;
    if (q == 0 || q >= (1u << 16)) return 1;
    const uint64_t wp = w[p];
    if ((u128)wp > total) return 2;
    u128 r = total - wp;
    if (r < 1) r = 1;
    unsigned bits = 0;
    for (u128 t = r; t; t >>= 1) bits++;
    const unsigned k = bits + 16 > 62 ? bits + 16 - 62 : 0;
    const u128 vp = (r * (u128)q) >> k;
    if (vp >> 64) return 3;
    const uint32_t m = (1u << 16) - q;
    for (size_t i = 0; i < n; i++) {
        const u128 v = ((u128)w[i] * m) >> k;
        w[i] = v > 1 ? (uint64_t)v : 1;  // below 2^62 for i != p (w[i] <= R)
    }
    w[p] = vp > 1 ? (uint64_t)vp : 1;
    return 0;
}

// Pass 1 of Mixer::mix (mixer.rs:278-288): the u128 sum, w[p] and the first index of the
// largest weight (0 when every weight is 0).
void mix_pass1(const uint64_t *w, size_t n, uint32_t p, u128 &total, uint64_t &wp, size_t &top) {
    total = 0;
    top = 0;
    uint64_t top_w = 0;
    for (size_t i = 0; i < n; i++) {
        total += w[i];
        if (w[i] > top_w) {
            top = i;
            top_w = w[i];
        }
    }
    wp = p < n ? w[p] : 0;
}

}  // namespace

// The match model and the mixer of one block (crates/taco/src/mix.rs:30-111).
struct or_mix_state {
    MatchV1 model;
    MixerV1 mixer;
};

extern "C" or_mix_state *or_mix_state_new() { return new or_mix_state(); }
extern "C" void or_mix_state_free(or_mix_state *s) { delete s; }
// MatchModel::predict: 1 and (token, length), or 0 without a prediction.
extern "C" int or_mix_state_predict(const or_mix_state *s, uint32_t *token, uint32_t *length) {
    return s->model.predict(*token, *length) ? 1 : 0;
}
// MixState::mix_stats (mix.rs:90-100): q from the statistics of the GPT-2 weights, 0 without a
// prediction (the pending state is cleared then).
extern "C" uint32_t or_mix_state_mix_stats(or_mix_state *s, uint64_t total, uint64_t predicted,
                                           uint32_t top) {
    uint32_t tok, len;
    s->mixer.clear();
    if (!s->model.predict(tok, len)) return 0;
    return s->mixer.mix_stats(total, predicted, tok == top, tok, len);
}
// Mixer::mix (mixer.rs:256-292): the weights in place, with the model's prediction.
extern "C" int or_mix_state_mix(or_mix_state *s, uint64_t *w, size_t n) {
    uint32_t tok, len;
    s->mixer.clear();
    if (!s->model.predict(tok, len)) {
        for (size_t i = 0; i < n; i++) w[i] = w[i] > 1 ? w[i] : 1;
        return 0;
    }
    if (tok >= n) return -1;
    u128 total;
    uint64_t wp;
    size_t top;
    mix_pass1(w, n, tok, total, wp, top);
    const uint32_t q = s->mixer.mix_stats(total, wp, top == tok, tok, len);
    return mix_apply_q(w, n, tok, total, q);
}
// MixState::observe (mix.rs:71-74): Mixer::update, then MatchModel::observe.
extern "C" void or_mix_state_observe(or_mix_state *s, uint32_t token) {
    s->mixer.update(token);
    s->model.observe(token);
}
// The synthetic-log vectors of crates/taco-match/tests/golden.rs:20-44 with custom match
// parameters are not needed: rule version 1 fixes them.
extern "C" void or_logistic_tables(uint16_t *squash, int16_t *stretch) {
    const Logistic &t = logistic();
    std::memcpy(squash, t.sq.data(), t.sq.size() * 2);
    std::memcpy(stretch, t.st.data(), t.st.size() * 2);
}

extern "C" size_t or_encode_block(const or_model *m, uint32_t overlap, const uint32_t *tokens,
                                  size_t n, size_t stop, uint8_t *out, size_t cap) {
    const size_t prefix = varint_len(n);
    if (prefix >= stop) return (size_t)-1;
    or_session s(m, overlap);
    Encoder e;
    std::vector<uint32_t> st;
    s.pos = 0;
    if (n > 0) {
        if (s.step(m->eot) != 0) return (size_t)-1;
        for (size_t i = 0; i < n; i++) {
            if (tokens[i] >= m->vocab) return (size_t)-1;
            from_weights(s.weights.data(), m->vocab, 32, st);
            uint64_t start, freq;
            interval_of(st, 32, tokens[i], start, freq);
            e.encode_parts(start, freq, start + freq == ((uint64_t)1 << 32), 32);
            if (prefix + e.nonzero_len >= stop) return (size_t)-1;
            if (i + 1 < n && s.step(tokens[i]) != 0) return (size_t)-1;
        }
    }
    std::vector<uint8_t> payload;
    write_varint(n, payload);
    std::vector<uint8_t> coded = e.finish();
    payload.insert(payload.end(), coded.begin(), coded.end());
    if (payload.size() <= cap) std::memcpy(out, payload.data(), payload.size());
    return payload.size();
}

extern "C" long or_decode_block(const or_model *m, uint32_t overlap, const uint8_t *payload,
                                size_t len, uint32_t *tokens, size_t cap) {
    uint64_t count;
    size_t used;
    if (!read_varint(payload, len, count, used) || count == 0 || count > cap) return -1;
    or_decoder d;
    d.in.assign(payload + used, payload + len);
    for (int i = 0; i < 8; i++) d.code = (d.code << 8) | d.next();
    or_session s(m, overlap);
    if (s.step(m->eot) != 0) return -1;
    std::vector<uint32_t> st;
    for (uint64_t i = 0; i < count; i++) {
        from_weights(s.weights.data(), m->vocab, 32, st);
        const uint64_t t = d.target(32);
        const size_t sym = find_symbol(st, t);
        uint64_t start, freq;
        interval_of(st, 32, sym, start, freq);
        if (!d.decode_interval(start, freq, 32)) return -1;
        tokens[i] = (uint32_t)sym;
        if (i + 1 < count && s.step((uint32_t)sym) != 0) return -1;
    }
    return (long)count;
}

// A mixed block (codec.rs:19-22, 354-370): the calls of a coded block, with the weights of the
// match model and the mixer between the session and the table, and MixState::observe after
// each token.
extern "C" size_t or_encode_mixed_block(const or_model *m, uint32_t overlap, const uint32_t *tokens,
                                        size_t n, uint8_t *out, size_t cap) {
    or_session s(m, overlap);
    or_mix_state ms;
    Encoder e;
    std::vector<uint32_t> st;
    std::vector<uint64_t> w(m->vocab);
    if (n > 0) {
        if (s.step(m->eot) != 0) return (size_t)-1;
        for (size_t i = 0; i < n; i++) {
            if (tokens[i] >= m->vocab) return (size_t)-1;
            std::copy(s.weights.begin(), s.weights.end(), w.begin());
            if (or_mix_state_mix(&ms, w.data(), w.size()) != 0) return (size_t)-1;
            from_weights(w.data(), m->vocab, 32, st);
            uint64_t start, freq;
            interval_of(st, 32, tokens[i], start, freq);
            e.encode_parts(start, freq, start + freq == ((uint64_t)1 << 32), 32);
            or_mix_state_observe(&ms, tokens[i]);
            if (i + 1 < n && s.step(tokens[i]) != 0) return (size_t)-1;
        }
    }
    std::vector<uint8_t> payload;
    write_varint(n, payload);
    std::vector<uint8_t> coded = e.finish();
    payload.insert(payload.end(), coded.begin(), coded.end());
    if (payload.size() <= cap) std::memcpy(out, payload.data(), payload.size());
    return payload.size();
}

extern "C" long or_decode_mixed_block(const or_model *m, uint32_t overlap, const uint8_t *payload,
                                      size_t len, uint32_t *tokens, size_t cap) {
    uint64_t count;
    size_t used;
    if (!read_varint(payload, len, count, used) || count == 0 || count > cap) return -1;
    or_decoder d;
    d.in.assign(payload + used, payload + len);
    for (int i = 0; i < 8; i++) d.code = (d.code << 8) | d.next();
    or_session s(m, overlap);
    or_mix_state ms;
    if (s.step(m->eot) != 0) return -1;
    std::vector<uint32_t> st;
    std::vector<uint64_t> w(m->vocab);
    for (uint64_t i = 0; i < count; i++) {
        std::copy(s.weights.begin(), s.weights.end(), w.begin());
        if (or_mix_state_mix(&ms, w.data(), w.size()) != 0) return -1;
        from_weights(w.data(), m->vocab, 32, st);
        const uint64_t t = d.target(32);
        const size_t sym = find_symbol(st, t);
        uint64_t start, freq;
        interval_of(st, 32, sym, start, freq);
        if (!d.decode_interval(start, freq, 32)) return -1;
        tokens[i] = (uint32_t)sym;
        or_mix_state_observe(&ms, (uint32_t)sym);
        if (i + 1 < count && s.step((uint32_t)sym) != 0) return -1;
    }
    return (long)count;
}

// ============================================================================================
// 9. The fast engine: the timed CPU baseline. A batched forward over a run of rows with AVX2
//    products (crates/hardshell/src/kernels/avx2.rs:110-199: vpmovsxbw + vpmaddwd, 4 weight
//    rows x 2 input rows) and chunked prefill (crates/taco/src/fold.rs:24, FOLD_CHUNK = 32).
//    It gives the reference session's weights bit for bit (tests/test_oracle.py).
// ============================================================================================

namespace {

inline int32_t hsum8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

inline __m256i widen16(const int8_t *p) {
    return _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)p));
}

// out[r * rows + o] = w[o * cols ..] . x[r * cols ..]
void matmul_avx2(const int8_t *w, size_t rows, const int8_t *x, size_t n, size_t cols,
                 int32_t *out) {
    const size_t kv = cols / 16 * 16;
    size_t o = 0;
    for (; o + 4 <= rows; o += 4) {
        const int8_t *w0 = w + o * cols, *w1 = w0 + cols, *w2 = w1 + cols, *w3 = w2 + cols;
        size_t r = 0;
        for (; r + 2 <= n; r += 2) {
            const int8_t *x0 = x + r * cols, *x1 = x0 + cols;
            __m256i a00 = _mm256_setzero_si256(), a01 = a00, a10 = a00, a11 = a00, a20 = a00,
                    a21 = a00, a30 = a00, a31 = a00;
            for (size_t k = 0; k < kv; k += 16) {
                __m256i v0 = widen16(x0 + k), v1 = widen16(x1 + k);
                __m256i u0 = widen16(w0 + k), u1 = widen16(w1 + k), u2 = widen16(w2 + k),
                        u3 = widen16(w3 + k);
                a00 = _mm256_add_epi32(a00, _mm256_madd_epi16(u0, v0));
                a01 = _mm256_add_epi32(a01, _mm256_madd_epi16(u0, v1));
                a10 = _mm256_add_epi32(a10, _mm256_madd_epi16(u1, v0));
                a11 = _mm256_add_epi32(a11, _mm256_madd_epi16(u1, v1));
                a20 = _mm256_add_epi32(a20, _mm256_madd_epi16(u2, v0));
                a21 = _mm256_add_epi32(a21, _mm256_madd_epi16(u2, v1));
                a30 = _mm256_add_epi32(a30, _mm256_madd_epi16(u3, v0));
                a31 = _mm256_add_epi32(a31, _mm256_madd_epi16(u3, v1));
            }
            int32_t s[8] = {hsum8(a00), hsum8(a01), hsum8(a10), hsum8(a11),
                            hsum8(a20), hsum8(a21), hsum8(a30), hsum8(a31)};
            for (size_t k = kv; k < cols; k++) {
                s[0] += w0[k] * x0[k]; s[1] += w0[k] * x1[k];
                s[2] += w1[k] * x0[k]; s[3] += w1[k] * x1[k];
                s[4] += w2[k] * x0[k]; s[5] += w2[k] * x1[k];
                s[6] += w3[k] * x0[k]; s[7] += w3[k] * x1[k];
            }
            for (int q = 0; q < 4; q++) {
                out[r * rows + o + q] = s[2 * q];
                out[(r + 1) * rows + o + q] = s[2 * q + 1];
            }
        }
        for (; r < n; r++) {
            const int8_t *x0 = x + r * cols;
            for (int q = 0; q < 4; q++) {
                const int8_t *wq = w + (o + q) * cols;
                __m256i a = _mm256_setzero_si256();
                for (size_t k = 0; k < kv; k += 16)
                    a = _mm256_add_epi32(a, _mm256_madd_epi16(widen16(wq + k), widen16(x0 + k)));
                int32_t s = hsum8(a);
                for (size_t k = kv; k < cols; k++) s += wq[k] * x0[k];
                out[r * rows + o + q] = s;
            }
        }
    }
    for (; o < rows; o++) {
        const int8_t *wq = w + o * cols;
        for (size_t r = 0; r < n; r++) {
            const int8_t *x0 = x + r * cols;
            __m256i a = _mm256_setzero_si256();
            for (size_t k = 0; k < kv; k += 16)
                a = _mm256_add_epi32(a, _mm256_madd_epi16(widen16(wq + k), widen16(x0 + k)));
            int32_t s = hsum8(a);
            for (size_t k = kv; k < cols; k++) s += wq[k] * x0[k];
            out[r * rows + o] = s;
        }
    }
}

inline int32_t dot_avx2(const int8_t *a, const int8_t *b, size_t n) {
    const size_t kv = n / 16 * 16;
    __m256i acc = _mm256_setzero_si256();
    for (size_t k = 0; k < kv; k += 16)
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(widen16(a + k), widen16(b + k)));
    int32_t s = hsum8(acc);
    for (size_t k = kv; k < n; k++) s += a[k] * b[k];
    return s;
}

// One session of the fast path: a KV cache and the work buffers of up to `cap` rows.
// Rows of one call are at consecutive positions of this session (engine.rs:112-197).
struct FastSession {
    const or_model *m;
    size_t cap;
    size_t pos = 0;
    std::vector<int8_t> kc, vc;  // [L][n_ctx][d]
    std::vector<int32_t> x, acc;
    std::vector<int8_t> a, qkv, att, g;
    std::vector<int16_t> g16, a16;
    std::vector<int64_t> scores, probs, head, logits;

    FastSession(const or_model *mm, size_t cp) : m(mm), cap(cp) {
        const size_t d = m->d, L = m->n_layer, C = m->n_ctx;
        kc.assign(L * C * d, 0);
        vc.assign(L * C * d, 0);
        x.assign(cap * d, 0);
        a.assign(cap * d, 0);
        qkv.assign(cap * 3 * d, 0);
        att.assign(cap * d, 0);
        g.assign(cap * m->f, 0);
        g16.assign(cap * m->f, 0);
        a16.assign(d, 0);
        acc.assign(cap * std::max<size_t>({3 * d, (size_t)m->f, (size_t)m->vocab}), 0);
        scores.assign(C, 0);
        probs.assign(C, 0);
        head.assign(m->hd, 0);
        logits.assign(m->vocab, 0);
    }

    void linear_residual(const Linear &l, const int8_t *in, size_t n) {
        matmul_avx2(l.w.data(), l.rows, in, n, l.cols, acc.data());
        const int64_t lim = SCORE_LIMIT;
        for (size_t r = 0; r < n; r++)
            for (size_t o = 0; o < l.rows; o++) {
                int64_t delta = rescale_clamp((int64_t)acc[r * l.rows + o] + l.b[o], l.r.m[o],
                                              l.r.s, -lim, lim);
                int32_t &xv = x[r * m->d + o];
                xv = (int32_t)clamp64((int64_t)xv + delta, -RES, RES);
            }
    }

    // Forward of n rows at positions pos0 .. pos0+n-1 with tokens toks; `want[i]` marks the
    // rows whose weights are written (packed, in row order) into `weights`.
    void forward(const uint32_t *toks, size_t n, size_t pos0, const bool *want, uint64_t *weights) {
        const size_t d = m->d, f = m->f, hd = m->hd, C = m->n_ctx, V = m->vocab;
        for (size_t r = 0; r < n; r++) {
            const uint32_t tok = toks[r];
            const size_t p = pos0 + r;
            for (size_t j = 0; j < d; j++) {
                i128 v = rescale(m->wte[tok * d + j], m->embed.m[tok], m->embed.s) +
                         rescale(m->wpe[p * d + j], m->pos.m[p], m->pos.s);
                x[r * d + j] = clamp_i32(v, -RES, RES);
            }
        }
        for (size_t l = 0; l < m->n_layer; l++) {
            const Block &b = m->blocks[l];
            for (size_t r = 0; r < n; r++)
                layernorm_apply(b.ln1, m->lnc, m->ln_beta_frac, &x[r * d], &a[r * d]);
            matmul_avx2(b.c_attn.w.data(), 3 * d, a.data(), n, d, acc.data());
            for (size_t r = 0; r < n; r++)
                for (size_t o = 0; o < 3 * d; o++)
                    qkv[r * 3 * d + o] = (int8_t)rescale_clamp(
                        (int64_t)acc[r * 3 * d + o] + b.c_attn.b[o], b.c_attn.r.m[o],
                        b.c_attn.r.s, -127, 127);
            const size_t base = l * C * d;
            for (size_t r = 0; r < n; r++) {
                std::memcpy(&kc[base + (pos0 + r) * d], &qkv[r * 3 * d + d], d);
                std::memcpy(&vc[base + (pos0 + r) * d], &qkv[r * 3 * d + 2 * d], d);
            }
            for (size_t r = 0; r < n; r++) {
                const size_t keys = pos0 + r + 1;
                for (size_t h = 0; h < m->n_head; h++) {
                    const size_t off = h * hd;
                    const int8_t *q = &qkv[r * 3 * d + off];
                    for (size_t j = 0; j < keys; j++)
                        scores[j] = rescale_clamp(dot_avx2(q, &kc[base + j * d + off], hd),
                                                  b.score_m, b.score_s, -SCORE_LIMIT, SCORE_LIMIT);
                    softmax_row(scores.data(), keys, m->attn_exp, m->softmax_p, probs.data());
                    std::fill(head.begin(), head.end(), 0);
                    for (size_t j = 0; j < keys; j++) {
                        const int64_t pj = probs[j];
                        const int8_t *v = &vc[base + j * d + off];
                        for (size_t c = 0; c < hd; c++) head[c] += pj * v[c];
                    }
                    for (size_t c = 0; c < hd; c++)
                        att[r * d + off + c] = clamp_act_i8(rescale(head[c], b.out_m, b.out_s));
                }
            }
            linear_residual(b.c_proj, att.data(), n);
            for (size_t r = 0; r < n; r++)
                layernorm_apply(b.ln2, m->lnc, m->ln_beta_frac, &x[r * d], &a[r * d]);
            matmul_avx2(b.c_fc.w.data(), f, a.data(), n, d, acc.data());
            const int64_t lo = b.gelu.lo(), hi = b.gelu.hi();
            if (!b.gelu.wide) {
                for (size_t r = 0; r < n; r++)
                    for (size_t o = 0; o < f; o++)
                        g[r * f + o] = (int8_t)b.gelu.apply(
                            rescale_clamp((int64_t)acc[r * f + o] + b.c_fc.b[o], b.c_fc.r.m[o],
                                          b.c_fc.r.s, lo, hi));
                linear_residual(b.mlp_proj, g.data(), n);
            } else {
                for (size_t r = 0; r < n; r++)
                    for (size_t o = 0; o < f; o++)
                        g16[r * f + o] = (int16_t)b.gelu.apply(
                            rescale_clamp((int64_t)acc[r * f + o] + b.c_fc.b[o], b.c_fc.r.m[o],
                                          b.c_fc.r.s, lo, hi));
                const Linear &pl = b.mlp_proj;
                for (size_t r = 0; r < n; r++)
                    for (size_t o = 0; o < d; o++) {
                        int64_t s = 0;
                        for (size_t c = 0; c < f; c++) s += (int64_t)pl.w[o * f + c] * g16[r * f + c];
                        int64_t delta = rescale_clamp(s + pl.b[o], pl.r.m[o], pl.r.s, -SCORE_LIMIT,
                                                      SCORE_LIMIT);
                        int32_t &xv = x[r * d + o];
                        xv = (int32_t)clamp64((int64_t)xv + delta, -RES, RES);
                    }
            }
        }
        // Final LayerNorm and logits only for the rows with an output (engine.rs:180-195).
        size_t packed = 0;
        for (size_t r = 0; r < n; r++) {
            if (!want[r]) continue;
            uint64_t *w = weights + packed * V;
            if (m->ln_f_bits == 16) {
                layernorm_apply(m->ln_f, m->lnc, m->ln_beta_frac, &x[r * d], a16.data());
                for (size_t v = 0; v < V; v++) {
                    int64_t s = 0;
                    for (size_t c = 0; c < d; c++) s += (int64_t)m->wte[v * d + c] * a16[c];
                    logits[v] = rescale_clamp(s, m->logit.m[v], m->logit.s, -SCORE_LIMIT,
                                              SCORE_LIMIT);
                }
                logits_to_weights(logits.data(), V, m->logits_exp, w);
            } else {
                layernorm_apply(m->ln_f, m->lnc, m->ln_beta_frac, &x[r * d], &a[packed * d]);
            }
            packed++;
        }
        if (m->ln_f_bits != 16 && packed > 0) {
            // One product with wte for all packed rows (each weight read once).
            std::vector<int32_t> lacc(packed * V);
            matmul_avx2(m->wte.data(), V, a.data(), packed, d, lacc.data());
            for (size_t i = 0; i < packed; i++) {
                for (size_t v = 0; v < V; v++)
                    logits[v] = rescale_clamp(lacc[i * V + v], m->logit.m[v], m->logit.s,
                                              -SCORE_LIMIT, SCORE_LIMIT);
                logits_to_weights(logits.data(), V, m->logits_exp, weights + i * V);
            }
        }
    }
};

// The rows of one window (EOT, t0 .. t_{n-2}) run in chunks; for each row the callback gets
// its weights and the index of the token they code.
template <typename F>
void run_window(const or_model *m, const uint32_t *tokens, size_t n, size_t chunk, F &&on_row) {
    chunk = std::max<size_t>(1, std::min<size_t>(chunk, m->n_ctx));
    FastSession s(m, chunk);
    std::vector<uint32_t> in(n);
    in[0] = m->eot;
    for (size_t i = 1; i < n; i++) in[i] = tokens[i - 1];
    std::vector<uint64_t> w(chunk * m->vocab);
    std::vector<char> want(chunk, 1);
    for (size_t r0 = 0; r0 < n; r0 += chunk) {
        const size_t c = std::min(chunk, n - r0);
        s.forward(&in[r0], c, r0, (const bool *)want.data(), w.data());
        for (size_t i = 0; i < c; i++) on_row(r0 + i, &w[i * m->vocab]);
    }
}

}  // namespace

extern "C" void or_matmul_i8(const int8_t *w, size_t rows, const int8_t *x, size_t n, size_t cols,
                             int32_t *out) {
    matmul_avx2(w, rows, x, n, cols, out);
}

extern "C" int or_fast_window_weights(const or_model *m, const uint32_t *tokens, size_t n,
                                      size_t chunk, uint64_t *weights) {
    if (n == 0 || n > m->n_ctx) return -1;
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= m->vocab) return -1;
    run_window(m, tokens, n, chunk, [&](size_t row, const uint64_t *w) {
        std::memcpy(weights + row * m->vocab, w, 8 * (size_t)m->vocab);
    });
    return 0;
}

extern "C" int or_fast_window_intervals(const or_model *m, const uint32_t *tokens, size_t n,
                                        size_t chunk, uint64_t *intervals) {
    if (n == 0 || n > m->n_ctx) return -1;
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= m->vocab) return -1;
    std::vector<uint32_t> st;
    run_window(m, tokens, n, chunk, [&](size_t row, const uint64_t *w) {
        from_weights(w, m->vocab, 32, st);
        uint64_t start, freq;
        interval_of(st, 32, tokens[row], start, freq);
        intervals[3 * row] = tokens[row];
        intervals[3 * row + 1] = start;
        intervals[3 * row + 2] = freq;
    });
    return 0;
}

extern "C" int or_fold_payloads(const or_model *m, const uint32_t *tokens, size_t count, size_t n,
                                size_t chunk, int threads, uint8_t *out, size_t cap,
                                size_t *lens) {
    if (n == 0 || n > m->n_ctx) return -1;
    for (size_t i = 0; i < count * n; i++)
        if (tokens[i] >= m->vocab) return -1;
    threads = std::max(1, threads);
    auto work = [&](int t) {
        std::vector<uint32_t> st;
        for (size_t w = (size_t)t; w < count; w += (size_t)threads) {
            const uint32_t *tk = tokens + w * n;
            Encoder e;
            run_window(m, tk, n, chunk, [&](size_t row, const uint64_t *wts) {
                from_weights(wts, m->vocab, 32, st);
                uint64_t start, freq;
                interval_of(st, 32, tk[row], start, freq);
                e.encode_parts(start, freq, start + freq == ((uint64_t)1 << 32), 32);
            });
            std::vector<uint8_t> p;
            write_varint(n, p);
            std::vector<uint8_t> coded = e.finish();
            p.insert(p.end(), coded.begin(), coded.end());
            lens[w] = p.size();
            if (p.size() <= cap) std::memcpy(out + w * cap, p.data(), p.size());
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; t++) pool.emplace_back(work, t);
    work(0);
    for (auto &th : pool) th.join();
    return 0;
}

// ============================================================================================
// 10. The seeded test builder — crates/hardshell/tests/common/{mod,builder,reference}.rs
//     f64 with basic operations only, in the reference's evaluation order.
// ============================================================================================

namespace {

struct Rng {  // splitmix64 (common/mod.rs:16-50)
    uint64_t s;
    uint64_t next() {
        s += 0x9E3779B97F4A7C15ull;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
    double normal() {
        double s = 0.0;
        for (int i = 0; i < 12; i++) s += uniform();
        return s - 6.0;
    }
    uint64_t below(uint64_t n) { return next() % n; }
};

double pow2(int k) {
    uint64_t bits = (uint64_t)(1023 + k) << 52;
    double d;
    std::memcpy(&d, &bits, 8);
    return d;
}

const double LN2 = 0.6931471805599453094172321214581766;

double det_exp(double x) {  // common/mod.rs:61-78
    if (x < -700.0) return 0.0;
    if (x > 700.0) return INFINITY;
    double k = std::round(x / LN2);
    double r = x - k * LN2;
    double term = 1.0, sum = 1.0;
    for (int i = 1; i < 22; i++) {
        term = term * r / (double)i;
        sum += term;
    }
    return sum * pow2((int)k);
}

double det_tanh(double x) {
    if (x > 20.0) return 1.0;
    if (x < -20.0) return -1.0;
    double e = det_exp(2.0 * x);
    return (e - 1.0) / (e + 1.0);
}

double gelu(double x) {
    const double C = 0.7978845608028654;
    return 0.5 * x * (1.0 + det_tanh(C * (x + 0.044715 * x * x * x)));
}

// Rust's saturating float-to-int casts (NaN gives 0).
template <typename T>
T sat_cast(double v) {
    if (std::isnan(v)) return 0;
    const double lo = (double)std::numeric_limits<T>::min(), hi = (double)std::numeric_limits<T>::max();
    if (v <= lo) return std::numeric_limits<T>::min();
    if (v >= hi) return std::numeric_limits<T>::max();
    return (T)v;
}

double fmax_rs(double a, double b) {  // f64::max: a NaN operand gives the other
    if (std::isnan(a)) return b;
    if (std::isnan(b)) return a;
    return a > b ? a : b;
}

double clamp_rs(double v, double lo, double hi) {
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

void quant_mult_rows(const std::vector<double> &rs, std::vector<int32_t> &m, uint8_t &s_out) {
    double mx = 0.0;
    for (double r : rs) mx = fmax_rs(mx, r);
    int s = 0;
    while (s < 126 && mx * pow2(s + 1) < 2147483647.0) s++;
    m.clear();
    for (double r : rs) m.push_back(sat_cast<int32_t>(std::round(r * pow2(s))));
    s_out = (uint8_t)s;
}

void quant_mult(double r, int32_t &m, uint8_t &s) {
    std::vector<int32_t> mv;
    quant_mult_rows({r}, mv, s);
    m = mv[0];
}

struct QMat {
    std::vector<int8_t> q;
    std::vector<double> scale;
    size_t rows = 0, cols = 0;
    std::vector<double> row(size_t r) const {
        std::vector<double> o(cols);
        for (size_t c = 0; c < cols; c++) o[c] = (double)q[r * cols + c] * scale[r];
        return o;
    }
    std::vector<double> matvec(const std::vector<double> &x) const {
        std::vector<double> o(rows);
        for (size_t r = 0; r < rows; r++) {
            double sum = 0.0;
            for (size_t c = 0; c < cols; c++) sum += (double)q[r * cols + c] * x[c];
            o[r] = sum * scale[r];
        }
        return o;
    }
};

struct FLin {
    QMat w;
    std::vector<double> b;
    std::vector<double> apply(const std::vector<double> &x) const {
        std::vector<double> o = w.matvec(x);
        for (size_t i = 0; i < o.size(); i++) o[i] = o[i] + b[i];
        return o;
    }
};

struct FBlock {
    std::vector<double> ln1_g, ln1_b, ln2_g, ln2_b;
    FLin c_attn, c_proj, fc, proj;
};

struct Dims {
    size_t n_layer, n_head, d_model, d_ff, vocab, n_ctx;
};

QMat quantise_rows(Rng &rng, size_t rows, size_t cols, double stdv) {
    QMat m;
    m.rows = rows;
    m.cols = cols;
    std::vector<double> row(cols);
    for (size_t r = 0; r < rows; r++) {
        for (auto &v : row) v = stdv * rng.normal();
        double mx = 0.0;
        for (double v : row) mx = fmax_rs(mx, std::fabs(v));
        double s = mx > 0.0 ? mx / 127.0 : 1.0;
        for (double v : row) m.q.push_back(sat_cast<int8_t>(clamp_rs(std::round(v / s), -127.0, 127.0)));
        m.scale.push_back(s);
    }
    return m;
}

std::vector<double> floats(Rng &rng, size_t n, double mean, double stdv) {
    std::vector<double> o(n);
    for (auto &v : o) v = mean + stdv * rng.normal();
    return o;
}

FLin flin(Rng &rng, size_t out, size_t inp, double stdv) {
    FLin l;
    l.w = quantise_rows(rng, out, inp, stdv);
    l.b = floats(rng, out, 0.0, 0.02);
    return l;
}

struct FloatModel {
    Dims d;
    QMat wte, wpe;
    std::vector<FBlock> blocks;
    std::vector<double> lnf_g, lnf_b;
};

struct Calib {
    double res = 0, lnf = 0;
    std::vector<double> ln1, q, k, v, att, ln2, fc, gelu;
};

double amax(const std::vector<double> &x, size_t off = 0, size_t n = SIZE_MAX) {
    double a = 0.0;
    n = std::min(n, x.size() - off);
    for (size_t i = 0; i < n; i++) a = fmax_rs(a, std::fabs(x[off + i]));
    return a;
}

const double LN_EPS = 1e-5;

std::vector<double> f_layernorm(const std::vector<double> &x, const std::vector<double> &g,
                                const std::vector<double> &b) {
    const double n = (double)x.size();
    double sum = -0.0;
    for (double v : x) sum += v;
    const double mean = sum / n;
    double vs = -0.0;
    for (double v : x) vs += (v - mean) * (v - mean);
    const double var = vs / n;
    const double inv = 1.0 / std::sqrt(var + LN_EPS);
    std::vector<double> o(x.size());
    for (size_t i = 0; i < x.size(); i++) o[i] = (x[i] - mean) * inv * g[i] + b[i];
    return o;
}

std::vector<double> f_softmax(const std::vector<double> &x) {
    double mx = -INFINITY;
    for (double v : x) mx = fmax_rs(mx, v);
    std::vector<double> e(x.size());
    for (size_t i = 0; i < x.size(); i++) e[i] = det_exp(x[i] - mx);
    double sum = -0.0;
    for (double v : e) sum += v;
    for (auto &v : e) v = v / sum;
    return e;
}

// The float forward pass with calibration (common/reference.rs:113-201).
void float_calibrate(const FloatModel &fm, const std::vector<size_t> &tokens, Calib &c) {
    const Dims d = fm.d;
    const size_t hd = d.d_model / d.n_head, L = d.n_layer, dm = d.d_model;
    const double inv_sqrt = 1.0 / std::sqrt((double)hd);
    c = Calib();
    c.ln1.assign(L, 0.0); c.q.assign(L, 0.0); c.k.assign(L, 0.0); c.v.assign(L, 0.0);
    c.att.assign(L, 0.0); c.ln2.assign(L, 0.0); c.fc.assign(L, 0.0); c.gelu.assign(L, 0.0);
    std::vector<std::vector<std::vector<double>>> kc(L), vc(L);
    for (size_t t = 0; t < tokens.size(); t++) {
        std::vector<double> te = fm.wte.row(tokens[t]), pe = fm.wpe.row(t);
        std::vector<double> x(dm);
        for (size_t i = 0; i < dm; i++) x[i] = te[i] + pe[i];
        c.res = fmax_rs(c.res, amax(x));
        for (size_t l = 0; l < L; l++) {
            const FBlock &b = fm.blocks[l];
            std::vector<double> a = f_layernorm(x, b.ln1_g, b.ln1_b);
            std::vector<double> qkv = b.c_attn.apply(a);
            std::vector<double> q(qkv.begin(), qkv.begin() + dm), k(qkv.begin() + dm, qkv.begin() + 2 * dm),
                v(qkv.begin() + 2 * dm, qkv.end());
            kc[l].push_back(k);
            vc[l].push_back(v);
            std::vector<double> att(dm, 0.0);
            for (size_t h = 0; h < d.n_head; h++) {
                const size_t o = h * hd;
                std::vector<double> scores;
                for (auto &kj : kc[l]) {
                    double s = 0.0;
                    for (size_t cc = 0; cc < hd; cc++) s += q[o + cc] * kj[o + cc];
                    scores.push_back(s * inv_sqrt);
                }
                std::vector<double> p = f_softmax(scores);
                for (size_t j = 0; j < p.size(); j++)
                    for (size_t cc = 0; cc < hd; cc++) att[o + cc] += p[j] * vc[l][j][o + cc];
            }
            std::vector<double> proj = b.c_proj.apply(att);
            for (size_t i = 0; i < dm; i++) x[i] += proj[i];
            std::vector<double> a2 = f_layernorm(x, b.ln2_g, b.ln2_b);
            std::vector<double> fc = b.fc.apply(a2);
            std::vector<double> g(fc.size());
            for (size_t i = 0; i < fc.size(); i++) g[i] = gelu(fc[i]);
            std::vector<double> mp = b.proj.apply(g);
            c.ln1[l] = fmax_rs(c.ln1[l], amax(a));
            c.q[l] = fmax_rs(c.q[l], amax(q));
            c.k[l] = fmax_rs(c.k[l], amax(k));
            c.v[l] = fmax_rs(c.v[l], amax(v));
            c.att[l] = fmax_rs(c.att[l], amax(att));
            c.ln2[l] = fmax_rs(c.ln2[l], amax(a2));
            c.fc[l] = fmax_rs(c.fc[l], amax(fc));
            c.gelu[l] = fmax_rs(c.gelu[l], amax(g));
            c.res = fmax_rs(c.res, amax(x));
            for (size_t i = 0; i < dm; i++) x[i] += mp[i];
            c.res = fmax_rs(c.res, amax(x));
        }
        std::vector<double> a = f_layernorm(x, fm.lnf_g, fm.lnf_b);
        c.lnf = fmax_rs(c.lnf, amax(a));
    }
}

// ---- .hsm writer (hsm/writer.rs:76-156): compact JSON in schema order, align-64 layout ----

struct WTensor {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    std::vector<uint8_t> data;
    int shift = -1;
};

struct HsmWriter {
    uint32_t n_layer = 0, n_head = 0, d_model = 0, d_ff = 0, vocab = 0, n_ctx = 0, eot = 0;
    uint8_t ln_k = 0, ln_j = 0, softmax_p = 0;
    uint64_t ln_eps = 0;
    int ln_f_bits = -1, ln_beta_frac = -1;  // -1: absent
    std::vector<std::vector<uint8_t>> vocabulary;
    std::vector<WTensor> tensors;

    template <typename T>
    void add(const std::string &name, const char *dtype, std::vector<uint64_t> shape,
             const std::vector<T> &v, int shift = -1) {
        WTensor t;
        t.name = name;
        t.dtype = dtype;
        t.shape = std::move(shape);
        t.data.resize(v.size() * sizeof(T));
        std::memcpy(t.data.data(), v.data(), t.data.size());
        t.shift = shift;
        tensors.push_back(std::move(t));
    }

    static uint64_t align64(uint64_t x) { return (x + 63) & ~(uint64_t)63; }

    std::string header(uint64_t header_len, uint64_t vocab_len) const {
        std::string s = "{\"model\":{\"architecture\":\"gpt2\"";
        auto kv = [&](const char *k, uint64_t v) {
            s += ",\"";
            s += k;
            s += "\":" + std::to_string(v);
        };
        kv("n_layer", n_layer); kv("n_head", n_head); kv("d_model", d_model); kv("d_ff", d_ff);
        kv("vocab_size", vocab); kv("n_ctx", n_ctx); kv("eot_token", eot);
        s += ",\"constants\":{\"ln_k\":" + std::to_string(ln_k);
        kv("ln_j", ln_j); kv("ln_eps", ln_eps); kv("softmax_p", softmax_p);
        if (ln_f_bits >= 0) kv("ln_f_bits", (uint64_t)ln_f_bits);
        if (ln_beta_frac >= 0) kv("ln_beta_frac", (uint64_t)ln_beta_frac);
        s += "}}";
        const uint64_t voff = align64(16 + header_len);
        s += ",\"vocabulary\":{\"offset\":" + std::to_string(voff) +
             ",\"length\":" + std::to_string(vocab_len) + "}";
        s += ",\"tensors\":[";
        uint64_t cursor = voff + vocab_len;
        for (size_t i = 0; i < tensors.size(); i++) {
            const WTensor &t = tensors[i];
            const uint64_t off = align64(cursor);
            if (i) s += ",";
            s += "{\"name\":\"" + t.name + "\",\"dtype\":\"" + t.dtype + "\",\"shape\":[";
            for (size_t j = 0; j < t.shape.size(); j++) {
                if (j) s += ",";
                s += std::to_string(t.shape[j]);
            }
            s += "],\"offset\":" + std::to_string(off) +
                 ",\"length\":" + std::to_string(t.data.size());
            if (t.shift >= 0) s += ",\"shift\":" + std::to_string(t.shift);
            s += "}";
            cursor = off + t.data.size();
        }
        s += "]}";
        return s;
    }

    std::vector<uint8_t> finish() const {
        std::vector<uint8_t> vb;
        for (auto &t : vocabulary) {
            uint16_t l = (uint16_t)t.size();
            vb.push_back((uint8_t)(l & 0xFF));
            vb.push_back((uint8_t)(l >> 8));
            vb.insert(vb.end(), t.begin(), t.end());
        }
        uint64_t header_len = 0;
        std::string json;
        for (;;) {
            json = header(header_len, vb.size());
            if (json.size() <= header_len) break;
            header_len = json.size();
        }
        bool v2 = ln_f_bits >= 0 || ln_beta_frac >= 0;
        for (auto &t : tensors) {
            const std::string suffix = ".mlp.gelu";
            if (t.dtype == "i16" && t.name.size() >= suffix.size() &&
                t.name.compare(t.name.size() - suffix.size(), suffix.size(), suffix) == 0)
                v2 = true;
        }
        std::vector<uint8_t> out;
        const char magic[8] = {'H', 'S', 'H', 'L', 'M', 'D', 'L', 0};
        out.insert(out.end(), magic, magic + 8);
        const uint32_t version = v2 ? 2 : 1, hl = (uint32_t)header_len;
        for (int i = 0; i < 4; i++) out.push_back((uint8_t)(version >> (8 * i)));
        for (int i = 0; i < 4; i++) out.push_back((uint8_t)(hl >> (8 * i)));
        out.insert(out.end(), json.begin(), json.end());
        out.resize(16 + header_len, ' ');
        out.resize(align64(out.size()), 0);
        out.insert(out.end(), vb.begin(), vb.end());
        for (auto &t : tensors) {
            out.resize(align64(out.size()), 0);
            out.insert(out.end(), t.data.begin(), t.data.end());
        }
        return out;
    }
};

void add_layernorm(HsmWriter &w, const std::string &p, const std::vector<double> &g,
                   const std::vector<double> &b, double s_out, int frac) {
    double mx = 0.0;
    for (double v : g) mx = fmax_rs(mx, std::fabs(v));
    const double s_gamma = mx / 32767.0;
    std::vector<int16_t> gq;
    for (double v : g) gq.push_back(sat_cast<int16_t>(std::round(v / s_gamma)));
    const double unit = s_out / pow2(frac);
    std::vector<int32_t> bq;
    for (double v : b) bq.push_back(sat_cast<int32_t>(std::round(v / unit)));
    int32_t m;
    uint8_t s;
    quant_mult(s_gamma / (pow2(48 - 8) * s_out), m, s);
    w.add(p + ".g", "i16", {gq.size()}, gq);
    w.add(p + ".b", "i32", {bq.size()}, bq);
    w.add(p + ".rescale", "i32", {1}, std::vector<int32_t>{m}, s);
}

template <typename SOut>
void add_linear(HsmWriter &w, const std::string &p, const FLin &l, double s_in, SOut s_out) {
    const size_t rows = l.w.rows;
    std::vector<double> acc_scale(rows), ratios(rows);
    std::vector<int32_t> bq(rows);
    for (size_t r = 0; r < rows; r++) acc_scale[r] = s_in * l.w.scale[r];
    for (size_t r = 0; r < rows; r++) bq[r] = sat_cast<int32_t>(std::round(l.b[r] / acc_scale[r]));
    for (size_t r = 0; r < rows; r++) ratios[r] = acc_scale[r] / s_out(r);
    std::vector<int32_t> m;
    uint8_t s;
    quant_mult_rows(ratios, m, s);
    w.add(p + ".w", "i8", {l.w.rows, l.w.cols}, l.w.q);
    w.add(p + ".b", "i32", {rows}, bq);
    w.add(p + ".rescale", "i32", {rows}, m, s);
}

std::vector<uint8_t> build_model(const Dims d, uint64_t seed, size_t calib_len, bool wide) {
    const double act_max = wide ? 32767.0 : 127.0;
    Rng rng{seed};
    // random_model (builder.rs:54-79)
    FloatModel fm;
    fm.d = d;
    const double dm = (double)d.d_model;
    const double wte_std = 2.5 / std::sqrt(dm);
    fm.wte = quantise_rows(rng, d.vocab, d.d_model, wte_std);
    fm.wpe = quantise_rows(rng, d.n_ctx, d.d_model, 0.3 * wte_std);
    for (size_t l = 0; l < d.n_layer; l++) {
        FBlock b;
        b.ln1_g = floats(rng, d.d_model, 1.0, 0.1);
        b.ln1_b = floats(rng, d.d_model, 0.0, 0.02);
        b.c_attn = flin(rng, 3 * d.d_model, d.d_model, 1.5 / std::sqrt(dm));
        b.c_proj = flin(rng, d.d_model, d.d_model, 0.5 / std::sqrt(dm));
        b.ln2_g = floats(rng, d.d_model, 1.0, 0.1);
        b.ln2_b = floats(rng, d.d_model, 0.0, 0.02);
        b.fc = flin(rng, d.d_ff, d.d_model, 1.0 / std::sqrt(dm));
        b.proj = flin(rng, d.d_model, d.d_ff, 0.5 / std::sqrt((double)d.d_ff));
        fm.blocks.push_back(std::move(b));
    }
    fm.lnf_g = floats(rng, d.d_model, 1.0, 0.1);
    fm.lnf_b = floats(rng, d.d_model, 0.0, 0.02);
    const size_t eot = d.vocab - 1;
    std::vector<size_t> calib{eot};
    while (calib.size() < std::min(calib_len, d.n_ctx)) calib.push_back(rng.below(d.vocab));
    Calib c;
    float_calibrate(fm, calib, c);

    const double s_res = c.res / pow2(22);
    const double delta = pow2(-8);
    const size_t hd = d.d_model / d.n_head;
    double eps = std::round((LN_EPS / (s_res * s_res)) * pow2(2 * 8));
    eps = fmax_rs(eps, 1.0);
    HsmWriter w;
    w.n_layer = (uint32_t)d.n_layer; w.n_head = (uint32_t)d.n_head; w.d_model = (uint32_t)d.d_model;
    w.d_ff = (uint32_t)d.d_ff; w.vocab = (uint32_t)d.vocab; w.n_ctx = (uint32_t)d.n_ctx;
    w.eot = (uint32_t)eot;
    w.ln_k = 48; w.ln_j = 8; w.ln_eps = sat_cast<uint64_t>(eps); w.softmax_p = 30;
    // vocabulary (builder.rs:82-92)
    for (int b = 0; b < 256; b++) w.vocabulary.push_back({(uint8_t)b});
    for (size_t i = 0; w.vocabulary.size() < d.vocab - 1; i++)
        w.vocabulary.push_back({(uint8_t)('a' + i % 26), (uint8_t)('a' + i / 26 % 26)});
    const char *eot_s = "<|endoftext|>";
    w.vocabulary.push_back(std::vector<uint8_t>(eot_s, eot_s + 13));
    const int frac = wide ? 8 : 0;
    if (wide) {
        w.ln_f_bits = 16;
        w.ln_beta_frac = frac;
    }
    const double s_lnf = c.lnf / act_max;
    w.add("wte", "i8", {fm.wte.rows, fm.wte.cols}, fm.wte.q);
    std::vector<double> rs;
    std::vector<int32_t> m;
    uint8_t s;
    rs.clear();
    for (double sc : fm.wte.scale) rs.push_back(sc / s_res);
    quant_mult_rows(rs, m, s);
    w.add("wte.rescale_embed", "i32", {m.size()}, m, s);
    rs.clear();
    for (double sc : fm.wte.scale) rs.push_back(sc * s_lnf / delta);
    quant_mult_rows(rs, m, s);
    w.add("wte.rescale_logits", "i32", {m.size()}, m, s);
    w.add("wpe", "i8", {fm.wpe.rows, fm.wpe.cols}, fm.wpe.q);
    rs.clear();
    for (double sc : fm.wpe.scale) rs.push_back(sc / s_res);
    quant_mult_rows(rs, m, s);
    w.add("wpe.rescale", "i32", {m.size()}, m, s);
    for (size_t l = 0; l < d.n_layer; l++) {
        const FBlock &b = fm.blocks[l];
        const std::string p = "h." + std::to_string(l);
        const double s_ln1 = c.ln1[l] / 127.0, s_ln2 = c.ln2[l] / 127.0;
        const double s_q = c.q[l] / 127.0, s_k = c.k[l] / 127.0, s_v = c.v[l] / 127.0;
        const double s_att = c.att[l] / 127.0;
        const double s_gin = c.fc[l] / 32767.0;
        const double s_gout = c.gelu[l] / act_max;
        add_layernorm(w, p + ".ln_1", b.ln1_g, b.ln1_b, s_ln1, frac);
        const size_t dmz = d.d_model;
        add_linear(w, p + ".attn.c_attn", b.c_attn, s_ln1,
                   [&](size_t r) { return r < dmz ? s_q : (r < 2 * dmz ? s_k : s_v); });
        int32_t mm;
        uint8_t ss;
        quant_mult(s_q * s_k / (std::sqrt((double)hd) * delta), mm, ss);
        w.add(p + ".attn.score.rescale", "i32", {1}, std::vector<int32_t>{mm}, ss);
        quant_mult(s_v / (pow2(30) * s_att), mm, ss);
        w.add(p + ".attn.out.rescale", "i32", {1}, std::vector<int32_t>{mm}, ss);
        add_linear(w, p + ".attn.c_proj", b.c_proj, s_att, [&](size_t) { return s_res; });
        add_layernorm(w, p + ".ln_2", b.ln2_g, b.ln2_b, s_ln2, frac);
        add_linear(w, p + ".mlp.c_fc", b.fc, s_ln2, [&](size_t) { return s_gin; });
        const int64_t half = (int64_t)1 << 15;
        if (wide) {
            std::vector<int16_t> t;
            for (int64_t q = -half; q < half; q++)
                t.push_back(sat_cast<int16_t>(clamp_rs(std::round(gelu((double)q * s_gin) / s_gout), -32767.0, 32767.0)));
            w.add(p + ".mlp.gelu", "i16", {t.size()}, t);
        } else {
            std::vector<int8_t> t;
            for (int64_t q = -half; q < half; q++)
                t.push_back(sat_cast<int8_t>(clamp_rs(std::round(gelu((double)q * s_gin) / s_gout), -127.0, 127.0)));
            w.add(p + ".mlp.gelu", "i8", {t.size()}, t);
        }
        add_linear(w, p + ".mlp.c_proj", b.proj, s_gout, [&](size_t) { return s_res; });
    }
    add_layernorm(w, "ln_f", fm.lnf_g, fm.lnf_b, s_lnf, frac);
    std::vector<int32_t> ae;
    std::vector<uint64_t> le;
    for (size_t i = 0; i < 8192; i++) {
        ae.push_back(sat_cast<int32_t>(std::round(pow2(30) * det_exp(-(double)i * delta))));
        le.push_back(sat_cast<uint64_t>(std::round(pow2(40) * det_exp(-(double)i * delta))));
    }
    w.add("attn_exp", "i32", {ae.size()}, ae);
    w.add("logits_exp", "u64", {le.size()}, le);
    return w.finish();
}

}  // namespace

extern "C" size_t or_build_model(const uint32_t *dims, uint64_t seed, size_t calib_len, int wide,
                                 uint8_t *out, size_t cap) {
    Dims d{dims[0], dims[1], dims[2], dims[3], dims[4], dims[5]};
    std::vector<uint8_t> b = build_model(d, seed, calib_len, wide != 0);
    if (b.size() <= cap) std::memcpy(out, b.data(), b.size());
    return b.size();
}

// ============================================================================================
// 11. Op-level references for the GPU op tests.
// ============================================================================================

// The c_attn form of a linear (gpt2/reference.rs:239-245): out[i][r] =
// clamp_act_i8(rescale(w[r] . a[i] + b[r], m[r], s)), with the scalar dot product.
extern "C" void or_linear_act_ref(const int8_t *w, const int8_t *a, const int32_t *bias,
                                  const int32_t *mult, uint8_t s, size_t m, size_t n, size_t k,
                                  int8_t *out) {
    for (size_t i = 0; i < m; i++)
        for (size_t r = 0; r < n; r++) {
            const int32_t acc = dot_i8(w + r * k, a + i * k, k);
            out[i * n + r] = clamp_act_i8(rescale((int64_t)acc + bias[r], mult[r], s));
        }
}

// One decode row of attention per stream (gpt2/reference.rs:254-283): q [b][h][hd]; caches
// [b][h][ctx_cap][hd]; keys ctx[b]; out [b][h*hd].
extern "C" void or_attend_decode_ref(const int8_t *q, const int8_t *kc, const int8_t *vc,
                                     const uint32_t *ctx, size_t b, size_t h, size_t hd,
                                     size_t ctx_cap, int32_t score_m, uint8_t score_s,
                                     int32_t out_m, uint8_t out_s, const int32_t *table,
                                     size_t len, uint8_t p, int8_t *out) {
    std::vector<int32_t> t(table, table + len);
    std::vector<int64_t> sc(ctx_cap), pr(ctx_cap), acc(hd);
    for (size_t s = 0; s < b; s++)
        for (size_t hh = 0; hh < h; hh++) {
            const int8_t *qq = q + (s * h + hh) * hd;
            const size_t base = (s * h + hh) * ctx_cap * hd;
            const size_t n = ctx[s];
            for (size_t j = 0; j < n; j++)
                sc[j] = clamp_wide(rescale(dot_i8(qq, kc + base + j * hd, hd), score_m, score_s),
                                   -SCORE_LIMIT, SCORE_LIMIT);
            softmax_row(sc.data(), n, t, p, pr.data());
            std::fill(acc.begin(), acc.end(), 0);
            for (size_t j = 0; j < n; j++)
                for (size_t c = 0; c < hd; c++) acc[c] += pr[j] * (int64_t)vc[base + j * hd + c];
            for (size_t c = 0; c < hd; c++)
                out[s * h * hd + hh * hd + c] = clamp_act_i8(rescale(acc[c], out_m, out_s));
        }
}

// ============================================================================================
// The mixed coder op of the logs profile: the weights of taco_match::Mixer::mix for a given
// probability q of the predicted token (crates/taco-match/src/mixer.rs:256-292, apply :491-516),
// the statistics of its pass 1 and the host record of rule 5
// (crates/hardshell-cuda/src/mixed.rs:36-90).
// ============================================================================================

// Pass 1 of Mixer::mix (mixer.rs:278-288): total = sum w (u128), w[p] (0 if p >= n), top = the
// first index of the largest weight, 0 when every weight is 0. out: total low, total high, w[p],
// top.
extern "C" void or_mix_stats(const uint64_t *w, size_t n, uint32_t p, uint64_t *out) {
    u128 total;
    uint64_t wp;
    size_t top;
    mix_pass1(w, n, p, total, wp, top);
    out[0] = (uint64_t)total;
    out[1] = (uint64_t)(total >> 64);
    out[2] = wp;
    out[3] = top;
}

// mix_record (mixed.rs:65-90): R = max(W - w[p], 1), m = 2^16 - q, k = max(0, bitlen(R) + 16 -
// 62), w'[p] = max(1, (R q) >> k). Returns 1 for q outside 1..=65535, 2 for w[p] > W, 3 for a
// w'[p] of 2^64 or more.
extern "C" int or_mix_record(uint64_t total_lo, uint64_t total_hi, uint64_t wp, uint32_t q,
                             uint32_t *k_out, uint32_t *m_out, uint64_t *wpm_out) {
    if (q == 0 || q >= (1u << 16)) return 1;
    const u128 total = ((u128)total_hi << 64) | total_lo;
    if ((u128)wp > total) return 2;
    u128 r = total - wp;
    if (r < 1) r = 1;
    unsigned bits = 0;
    for (u128 t = r; t; t >>= 1) bits++;
    const unsigned k = bits + 16 > 62 ? bits + 16 - 62 : 0;
    const u128 v = (r * (u128)q) >> k;
    if (v >> 64) return 3;
    *k_out = k;
    *m_out = (1u << 16) - q;
    *wpm_out = v > 1 ? (uint64_t)v : 1;
    return 0;
}

// Mixer::mix's weights for the probability q (mixer.rs:256-292 with apply :491-516): without a
// prediction (p = UINT32_MAX) every weight becomes max(1, w); else rule 6 with the statistics of
// w. Returns or_mix_record's codes, 4 for p >= n.
extern "C" int or_mix_apply(uint64_t *w, size_t n, uint32_t p, uint32_t q) {
    if (p == UINT32_MAX) {
        for (size_t i = 0; i < n; i++) w[i] = w[i] > 1 ? w[i] : 1;
        return 0;
    }
    if (p >= n) return 4;
    u128 total;
    uint64_t wp;
    size_t top;
    mix_pass1(w, n, p, total, wp, top);
    return mix_apply_q(w, n, p, total, q);
}
