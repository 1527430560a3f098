// Strict .hsm reader and GPT-2 model checks. The rules and their order follow
// crates/hardshell/src/hsm/reader.rs:357-430 (file), hsm/header.rs (JSON schema),
// hsm/merges.rs:43-110 (merges) and gpt2/model.rs:117-343 (tensors); the code is this build's.
#include "hsm.h"

#include <cstring>
#include <map>
#include <set>

namespace hs {

bool HostModel::is_wide() const {
    if (ln_f_bits == 16 || ln_beta_frac > 0) return true;
    for (auto &b : blocks)
        if (b.gelu_wide) return true;
    return false;
}

namespace {

// ---------------------------------------------------------------------------------------------
// JSON: a complete RFC 8259 reader (serde_json's grammar: no trailing commas, no leading zeros,
// strict escapes and surrogates, depth limit 128), into a tree that keeps duplicate keys.
// ---------------------------------------------------------------------------------------------

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    std::string text;  // STR: the decoded string; NUM: the number text
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
};

struct Parser {
    const char *p, *e;
    std::string err;
    int depth = 0;

    bool fail(const char *m) {
        if (err.empty()) err = m;
        return false;
    }
    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char *s) {
        size_t n = std::strlen(s);
        if ((size_t)(e - p) < n || std::memcmp(p, s, n) != 0) return fail("expected value");
        p += n;
        return true;
    }
    static void put_utf8(std::string &o, uint32_t c) {
        if (c < 0x80) {
            o.push_back((char)c);
        } else if (c < 0x800) {
            o.push_back((char)(0xC0 | (c >> 6)));
            o.push_back((char)(0x80 | (c & 0x3F)));
        } else if (c < 0x10000) {
            o.push_back((char)(0xE0 | (c >> 12)));
            o.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
            o.push_back((char)(0x80 | (c & 0x3F)));
        } else {
            o.push_back((char)(0xF0 | (c >> 18)));
            o.push_back((char)(0x80 | ((c >> 12) & 0x3F)));
            o.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
            o.push_back((char)(0x80 | (c & 0x3F)));
        }
    }
    bool hex4(uint32_t &v) {
        if (e - p < 4) return fail("EOF while parsing a string");
        v = 0;
        for (int i = 0; i < 4; i++) {
            char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("invalid escape");
        }
        return true;
    }
    bool string(std::string &o) {
        p++;  // opening quote
        while (true) {
            if (p >= e) return fail("EOF while parsing a string");
            unsigned char c = (unsigned char)*p;
            if (c == '"') {
                p++;
                return true;
            }
            if (c < 0x20) return fail("control character while parsing a string");
            if (c == '\\') {
                p++;
                if (p >= e) return fail("EOF while parsing a string");
                char x = *p++;
                switch (x) {
                    case '"': o.push_back('"'); break;
                    case '\\': o.push_back('\\'); break;
                    case '/': o.push_back('/'); break;
                    case 'b': o.push_back('\b'); break;
                    case 'f': o.push_back('\f'); break;
                    case 'n': o.push_back('\n'); break;
                    case 'r': o.push_back('\r'); break;
                    case 't': o.push_back('\t'); break;
                    case 'u': {
                        uint32_t v;
                        if (!hex4(v)) return false;
                        if (v >= 0xDC00 && v <= 0xDFFF) return fail("lone trailing surrogate");
                        if (v >= 0xD800 && v <= 0xDBFF) {
                            uint32_t lo;
                            if (e - p < 2 || p[0] != '\\' || p[1] != 'u')
                                return fail("lone leading surrogate");
                            p += 2;
                            if (!hex4(lo)) return false;
                            if (lo < 0xDC00 || lo > 0xDFFF) return fail("lone leading surrogate");
                            v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
                        }
                        put_utf8(o, v);
                        break;
                    }
                    default: return fail("invalid escape");
                }
            } else {
                o.push_back((char)c);
                p++;
            }
        }
    }
    bool number(Json &v) {
        const char *s = p;
        if (*p == '-') p++;
        if (p >= e) return fail("invalid number");
        if (*p == '0') {
            p++;
        } else if (*p >= '1' && *p <= '9') {
            while (p < e && *p >= '0' && *p <= '9') p++;
        } else {
            return fail("invalid number");
        }
        if (p < e && (*p >= '0' && *p <= '9')) return fail("invalid number");
        if (p < e && *p == '.') {
            p++;
            if (p >= e || !(*p >= '0' && *p <= '9')) return fail("invalid number");
            while (p < e && *p >= '0' && *p <= '9') p++;
        }
        if (p < e && (*p == 'e' || *p == 'E')) {
            p++;
            if (p < e && (*p == '+' || *p == '-')) p++;
            if (p >= e || !(*p >= '0' && *p <= '9')) return fail("invalid number");
            while (p < e && *p >= '0' && *p <= '9') p++;
        }
        v.kind = Json::NUM;
        v.text.assign(s, p);
        return true;
    }
    bool value(Json &v) {
        ws();
        if (p >= e) return fail("EOF while parsing a value");
        if (++depth > 128) return fail("recursion limit exceeded");
        bool ok = true;
        switch (*p) {
            case '{': {
                v.kind = Json::OBJ;
                p++;
                ws();
                if (p < e && *p == '}') {
                    p++;
                    break;
                }
                while (true) {
                    ws();
                    if (p >= e || *p != '"') { ok = fail("key must be a string"); break; }
                    std::string key;
                    if (!string(key)) { ok = false; break; }
                    ws();
                    if (p >= e || *p != ':') { ok = fail("expected ':'"); break; }
                    p++;
                    Json val;
                    if (!value(val)) { ok = false; break; }
                    v.obj.emplace_back(std::move(key), std::move(val));
                    ws();
                    if (p < e && *p == ',') { p++; continue; }
                    if (p < e && *p == '}') { p++; break; }
                    ok = fail("expected ',' or '}'");
                    break;
                }
                break;
            }
            case '[': {
                v.kind = Json::ARR;
                p++;
                ws();
                if (p < e && *p == ']') {
                    p++;
                    break;
                }
                while (true) {
                    Json item;
                    if (!value(item)) { ok = false; break; }
                    v.arr.push_back(std::move(item));
                    ws();
                    if (p < e && *p == ',') { p++; continue; }
                    if (p < e && *p == ']') { p++; break; }
                    ok = fail("expected ',' or ']'");
                    break;
                }
                break;
            }
            case '"':
                v.kind = Json::STR;
                ok = string(v.text);
                break;
            case 't': v.kind = Json::BOOL; ok = lit("true"); break;
            case 'f': v.kind = Json::BOOL; ok = lit("false"); break;
            case 'n': v.kind = Json::NUL; ok = lit("null"); break;
            default:
                if (*p == '-' || (*p >= '0' && *p <= '9')) ok = number(v);
                else ok = fail("expected value");
        }
        depth--;
        return ok;
    }
};

// Typed reads with serde's rules: an unsigned integer field takes a number with no sign,
// fraction or exponent that fits the type.
bool as_uint(const Json &v, uint64_t max, uint64_t &out) {
    if (v.kind != Json::NUM) return false;
    const std::string &t = v.text;
    if (t.empty() || t[0] == '-') return false;
    for (char c : t)
        if (c < '0' || c > '9') return false;
    if (t.size() > 20) return false;
    unsigned __int128 acc = 0;
    for (char c : t) acc = acc * 10 + (unsigned)(c - '0');
    if (acc > max) return false;
    out = (uint64_t)acc;
    return true;
}

// Checks the keys of an object against a schema: unknown, duplicate and missing fields fail.
struct Fields {
    const Json &o;
    std::map<std::string, const Json *> got;
    std::string err;
    Fields(const Json &obj, std::initializer_list<const char *> known) : o(obj) {
        if (o.kind != Json::OBJ) {
            err = "invalid type: expected a struct";
            return;
        }
        std::set<std::string> k;
        for (auto s : known) k.insert(s);
        for (auto &kv : o.obj) {
            if (!k.count(kv.first)) {
                err = "unknown field `" + kv.first + "`";
                return;
            }
            if (got.count(kv.first)) {
                err = "duplicate field `" + kv.first + "`";
                return;
            }
            got[kv.first] = &kv.second;
        }
    }
    // A required field; for an optional field, NULL (absent or null) is allowed.
    const Json *need(const char *k) {
        auto it = got.find(k);
        if (it == got.end()) {
            if (err.empty()) err = std::string("missing field `") + k + "`";
            return nullptr;
        }
        return it->second;
    }
    const Json *opt(const char *k) {
        auto it = got.find(k);
        if (it == got.end() || it->second->kind == Json::NUL) return nullptr;
        return it->second;
    }
    bool uint(const char *k, uint64_t max, uint64_t &out) {
        const Json *v = need(k);
        if (!v) return false;
        if (!as_uint(*v, max, out)) {
            if (err.empty()) err = std::string("invalid value for `") + k + "`";
            return false;
        }
        return true;
    }
    bool opt_uint(const char *k, uint64_t max, bool &present, uint64_t &out) {
        const Json *v = opt(k);
        present = v != nullptr;
        if (!v) return true;
        if (!as_uint(*v, max, out)) {
            if (err.empty()) err = std::string("invalid value for `") + k + "`";
            return false;
        }
        return true;
    }
    bool str(const char *k, std::string &out) {
        const Json *v = need(k);
        if (!v) return false;
        if (v->kind != Json::STR) {
            if (err.empty()) err = std::string("invalid type for `") + k + "`";
            return false;
        }
        out = v->text;
        return true;
    }
};

struct Section {
    uint64_t offset = 0, length = 0;
};

struct Entry {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    uint64_t offset = 0, length = 0;
    bool has_shift = false;
    uint8_t shift = 0;
};

struct Header {
    std::string architecture;
    uint32_t n_layer = 0, n_head = 0, d_model = 0, d_ff = 0, vocab = 0, n_ctx = 0, eot = 0;
    uint8_t ln_k = 0, ln_j = 0, softmax_p = 0;
    uint64_t ln_eps = 0;
    bool has_f_bits = false, has_beta_frac = false;
    uint8_t ln_f_bits = 0, ln_beta_frac = 0;
    Section vocab_sec;
    bool has_merges = false;
    Section merges;
    std::vector<Entry> tensors;
};

bool section(const Json &v, Section &s, std::string &err) {
    Fields f(v, {"offset", "length"});
    bool ok = f.err.empty() && f.uint("offset", UINT64_MAX, s.offset) &&
              f.uint("length", UINT64_MAX, s.length);
    if (!ok) err = f.err;
    return ok;
}

bool parse_header(const Json &root, Header &h, std::string &err) {
    Fields top(root, {"model", "vocabulary", "merges", "tensors"});
    if (!top.err.empty()) { err = top.err; return false; }
    const Json *model = top.need("model");
    if (!model) { err = top.err; return false; }
    {
        Fields m(*model, {"architecture", "n_layer", "n_head", "d_model", "d_ff", "vocab_size",
                          "n_ctx", "eot_token", "constants"});
        uint64_t v[8];
        const char *names[7] = {"n_layer", "n_head", "d_model", "d_ff", "vocab_size", "n_ctx",
                                "eot_token"};
        bool ok = m.err.empty() && m.str("architecture", h.architecture);
        for (int i = 0; ok && i < 7; i++) ok = m.uint(names[i], UINT32_MAX, v[i]);
        const Json *c = ok ? m.need("constants") : nullptr;
        if (!ok || !c) { err = m.err; return false; }
        h.n_layer = (uint32_t)v[0]; h.n_head = (uint32_t)v[1]; h.d_model = (uint32_t)v[2];
        h.d_ff = (uint32_t)v[3]; h.vocab = (uint32_t)v[4]; h.n_ctx = (uint32_t)v[5];
        h.eot = (uint32_t)v[6];
        Fields cf(*c, {"ln_k", "ln_j", "ln_eps", "softmax_p", "ln_f_bits", "ln_beta_frac"});
        uint64_t k, j, eps, sp, fb = 0, bf = 0;
        ok = cf.err.empty() && cf.uint("ln_k", 255, k) && cf.uint("ln_j", 255, j) &&
             cf.uint("ln_eps", UINT64_MAX, eps) && cf.uint("softmax_p", 255, sp) &&
             cf.opt_uint("ln_f_bits", 255, h.has_f_bits, fb) &&
             cf.opt_uint("ln_beta_frac", 255, h.has_beta_frac, bf);
        if (!ok) { err = cf.err; return false; }
        h.ln_k = (uint8_t)k; h.ln_j = (uint8_t)j; h.ln_eps = eps; h.softmax_p = (uint8_t)sp;
        h.ln_f_bits = (uint8_t)fb; h.ln_beta_frac = (uint8_t)bf;
    }
    const Json *voc = top.need("vocabulary");
    if (!voc) { err = top.err; return false; }
    if (!section(*voc, h.vocab_sec, err)) return false;
    if (const Json *mg = top.opt("merges")) {
        h.has_merges = true;
        if (!section(*mg, h.merges, err)) return false;
    }
    const Json *ts = top.need("tensors");
    if (!ts) { err = top.err; return false; }
    if (ts->kind != Json::ARR) { err = "invalid type for `tensors`"; return false; }
    for (const Json &t : ts->arr) {
        Entry e;
        Fields f(t, {"name", "dtype", "shape", "offset", "length", "shift"});
        uint64_t sh = 0;
        bool ok = f.err.empty() && f.str("name", e.name) && f.str("dtype", e.dtype);
        const Json *shape = ok ? f.need("shape") : nullptr;
        if (!ok || !shape) { err = f.err; return false; }
        if (shape->kind != Json::ARR) { err = "invalid type for `shape`"; return false; }
        for (const Json &d : shape->arr) {
            uint64_t x;
            if (!as_uint(d, UINT64_MAX, x)) { err = "invalid value in `shape`"; return false; }
            e.shape.push_back(x);
        }
        ok = f.uint("offset", UINT64_MAX, e.offset) && f.uint("length", UINT64_MAX, e.length) &&
             f.opt_uint("shift", 255, e.has_shift, sh);
        if (!ok) { err = f.err; return false; }
        e.shift = (uint8_t)sh;
        h.tensors.push_back(std::move(e));
    }
    return true;
}

// ---------------------------------------------------------------------------------------------
// File rules.
// ---------------------------------------------------------------------------------------------

bool valid_name(const std::string &s) {
    if (s.empty() || s.size() > 128) return false;
    for (unsigned char c : s)
        if (!((c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_' || c == '.'))
            return false;
    return true;
}

bool align64(uint64_t x, uint64_t &out) {
    if (x > UINT64_MAX - 63) return false;
    out = (x + 63) & ~(uint64_t)63;
    return true;
}

bool valid_utf8(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        uint8_t c = s[i];
        if (c < 0x80) { i++; continue; }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
        else return false;
        if (i + len > n) return false;
        for (int k = 1; k < len; k++) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
            cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += len;
    }
    return true;
}

size_t dtype_size(const std::string &d) {
    if (d == "i8") return 1;
    if (d == "i16") return 2;
    if (d == "i32") return 4;
    if (d == "u64") return 8;
    return 0;
}

struct Stored {
    std::string dtype;
    std::vector<uint64_t> dims;
    const uint8_t *data = nullptr;
    uint64_t length = 0;
    bool has_shift = false;
    uint8_t shift = 0;
};

bool set_err(ModelError &err, hs_model_error k, const std::string &m) {
    err.kind = k;
    err.msg = m;
    return false;
}

}  // namespace

bool load_host_model(const uint8_t *bytes, size_t len, HostModel &out, ModelError &err) {
    const uint64_t file_len = len;
    auto truncated = [&](uint64_t off, uint64_t need) {
        return set_err(err, HS_MODEL_TRUNCATED,
                       "the file is truncated: " + std::to_string(need) + " bytes at offset " +
                           std::to_string(off) + " past the end of a " + std::to_string(file_len) +
                           "-byte file");
    };
    auto in_file = [&](uint64_t off, uint64_t n) {
        return off <= file_len && n <= file_len - off;
    };
    // Preamble: magic, version, header length (reader.rs:358-367).
    if (!in_file(0, 16)) return truncated(0, 16);
    if (std::memcmp(bytes, "HSHLMDL\0", 8) != 0)
        return set_err(err, HS_MODEL_BAD_MAGIC, "the file does not start with the .hsm magic");
    uint32_t version, header_len;
    std::memcpy(&version, bytes + 8, 4);
    std::memcpy(&header_len, bytes + 12, 4);
    if (version != 1 && version != 2)
        return set_err(err, HS_MODEL_UNSUPPORTED_VERSION,
                       "unsupported .hsm version " + std::to_string(version));
    if (!in_file(16, header_len)) return truncated(16, header_len);
    if (!valid_utf8(bytes + 16, header_len))
        return set_err(err, HS_MODEL_HEADER_NOT_UTF8, "the header is not UTF-8");
    Parser ps{(const char *)bytes + 16, (const char *)bytes + 16 + header_len, "", 0};
    Json root;
    bool ok = ps.value(root);
    if (ok) {
        ps.ws();
        if (ps.p != ps.e) ok = ps.fail("trailing characters");
    }
    if (!ok) return set_err(err, HS_MODEL_HEADER_JSON, "header JSON: " + ps.err);
    Header h;
    std::string herr;
    if (!parse_header(root, h, herr)) return set_err(err, HS_MODEL_HEADER_JSON, "header JSON: " + herr);

    // check_config (reader.rs:265-281).
    auto bad = [&](const std::string &field, const std::string &why) {
        return set_err(err, HS_MODEL_INVALID_HEADER, field + ": " + why);
    };
    if (!valid_name(h.architecture))
        return bad("model.architecture", "must have 1 to 128 characters from a-z 0-9 _ .");
    if (h.vocab == 0 || h.vocab > (1u << 20)) return bad("model.vocab_size", "must be in 1..=2^20");
    if (h.eot >= h.vocab) return bad("model.eot_token", "must be less than vocab_size");
    if (h.ln_k > 48) return bad("constants.ln_k", "must be at most 48");
    if (h.ln_j > 16) return bad("constants.ln_j", "must be at most 16");
    if (h.ln_eps == 0 || h.ln_eps > ((uint64_t)1 << 62)) return bad("constants.ln_eps", "must be in 1..=2^62");
    if (h.softmax_p > 30) return bad("model.constants.softmax_p", "must be at most 30");
    // check_version (reader.rs:284-306).
    if (h.has_f_bits && h.ln_f_bits != 16)
        return bad("model.constants.ln_f_bits", "must be 16 (omit the field for 8)");
    if (h.has_beta_frac && (h.ln_beta_frac == 0 || h.ln_beta_frac > 16))
        return bad("model.constants.ln_beta_frac", "must be in 1..=16 (omit the field for 0)");
    {
        bool v2 = h.has_f_bits || h.has_beta_frac;
        const std::string suffix = ".mlp.gelu";
        for (auto &t : h.tensors)
            if (t.dtype == "i16" && t.name.size() >= suffix.size() &&
                t.name.compare(t.name.size() - suffix.size(), suffix.size(), suffix) == 0)
                v2 = true;
        if ((v2 ? 2u : 1u) != version)
            return bad("version", "a file is version 2 if and only if it has a version 2 constant or an i16 GELU table");
    }
    const uint8_t ln_f_bits = h.has_f_bits ? h.ln_f_bits : 8;
    const uint8_t ln_beta_frac = h.has_beta_frac ? h.ln_beta_frac : 0;

    auto layout = [&](const std::string &name, const std::string &why) {
        return set_err(err, HS_MODEL_LAYOUT, "layout of " + name + ": " + why);
    };
    auto padding = [&](uint64_t from, uint64_t to) {
        uint64_t n = to >= from ? to - from : 0;
        if (!in_file(from, n)) return truncated(from, n);
        for (uint64_t i = 0; i < n; i++)
            if (bytes[from + i] != 0)
                return set_err(err, HS_MODEL_NON_ZERO_PADDING,
                               "non-zero padding at offset " + std::to_string(from + i));
        return true;
    };
    // Vocabulary (reader.rs:379-388).
    const uint64_t header_end = 16 + (uint64_t)header_len;
    uint64_t voff;
    if (!align64(header_end, voff)) return layout("vocabulary", "overflow");
    if (h.vocab_sec.offset != voff) return layout("vocabulary", "the offset is not align64(16 + header_len)");
    if (!padding(header_end, voff)) return false;
    if (!in_file(voff, h.vocab_sec.length)) return truncated(voff, h.vocab_sec.length);
    {
        const uint8_t *sec = bytes + voff;
        const uint64_t n = h.vocab_sec.length;
        uint64_t pos = 0;
        out.vocab_ends.clear();
        out.vocab_bytes.clear();
        for (uint32_t t = 0; t < h.vocab; t++) {
            if (n - pos < 2 || pos > n)
                return set_err(err, HS_MODEL_VOCABULARY, "token " + std::to_string(t) + ": the length is outside the section");
            uint16_t l = (uint16_t)(sec[pos] | (sec[pos + 1] << 8));
            pos += 2;
            if (n - pos < l)
                return set_err(err, HS_MODEL_VOCABULARY, "token " + std::to_string(t) + ": the bytes are outside the section");
            out.vocab_bytes.insert(out.vocab_bytes.end(), sec + pos, sec + pos + l);
            out.vocab_ends.push_back((uint32_t)out.vocab_bytes.size());
            pos += l;
        }
        if (pos != n)
            return set_err(err, HS_MODEL_VOCABULARY, "token " + std::to_string(h.vocab) + ": the section has extra bytes");
    }
    uint64_t cursor = voff + h.vocab_sec.length;
    auto tok_bytes = [&](uint32_t id, const uint8_t *&p, size_t &n) {
        uint32_t s = id == 0 ? 0 : out.vocab_ends[id - 1];
        p = out.vocab_bytes.data() + s;
        n = out.vocab_ends[id] - s;
    };
    // Merges (reader.rs:389-402, merges.rs:43-110).
    if (h.has_merges) {
        uint64_t off;
        if (!align64(cursor, off)) return layout("merges", "overflow");
        if (h.merges.offset != off) return layout("merges", "the offset is not align64 of the vocabulary end");
        if (!padding(cursor, std::min(off, file_len))) return false;
        if (!in_file(h.merges.offset, h.merges.length)) return truncated(h.merges.offset, h.merges.length);
        const uint64_t ml = h.merges.length;
        if (ml == 0 || ml % 8 != 0)
            return bad("merges.length", "must be a multiple of 8 and at least 8 (omit the section for no merges)");
        std::map<std::string, int64_t> by_bytes;  // -1: two tokens have these bytes
        for (uint32_t i = 0; i < h.vocab; i++) {
            const uint8_t *p;
            size_t n;
            tok_bytes(i, p, n);
            std::string key((const char *)p, n);
            auto it = by_bytes.find(key);
            if (it == by_bytes.end()) by_bytes[key] = i; else it->second = -1;
        }
        std::set<std::pair<uint32_t, uint32_t>> seen;
        const uint8_t *sec = bytes + h.merges.offset;
        for (uint64_t r = 0; r < ml / 8; r++) {
            uint32_t l, rr;
            std::memcpy(&l, sec + 8 * r, 4);
            std::memcpy(&rr, sec + 8 * r + 4, 4);
            const std::string field = "merges[" + std::to_string(r) + "]";
            if (l >= h.vocab || rr >= h.vocab) return bad(field, "a token id is not less than the vocabulary size");
            const uint8_t *lp, *rp;
            size_t ln, rn;
            tok_bytes(l, lp, ln);
            tok_bytes(rr, rp, rn);
            if (ln == 0 || rn == 0) return bad(field, "a part of the merge has no bytes");
            if (!seen.insert({l, rr}).second) return bad(field, "the pair occurs two times");
            std::string joined((const char *)lp, ln);
            joined.append((const char *)rp, rn);
            auto it = by_bytes.find(joined);
            if (it == by_bytes.end()) return bad(field, "the joined bytes are not a token");
            if (it->second < 0) return bad(field, "two tokens have the joined bytes");
            out.merges.push_back(l);
            out.merges.push_back(rr);
        }
        cursor = off + ml;
    }
    // Tensors (reader.rs:403-427, read_tensor 308-343).
    std::map<std::string, Stored> tensors;
    for (const Entry &e : h.tensors) {
        if (!valid_name(e.name)) return bad("tensors[].name", "must have 1 to 128 characters from a-z 0-9 _ .");
        if (tensors.count(e.name))
            return set_err(err, HS_MODEL_UNEXPECTED_TENSOR, e.name + ": the name occurs two times");
        uint64_t off;
        if (!align64(cursor, off)) return layout(e.name, "overflow");
        if (!padding(cursor, std::min(off, file_len))) return false;
        auto mismatch = [&](const std::string &why) {
            return set_err(err, HS_MODEL_TENSOR_MISMATCH, e.name + ": " + why);
        };
        const size_t sz = dtype_size(e.dtype);
        if (sz == 0) return mismatch("unknown dtype");
        if (e.shape.empty()) return set_err(err, HS_MODEL_INVALID_SHAPE, "a shape needs at least one dimension");
        if (e.shape.size() > 4) return set_err(err, HS_MODEL_INVALID_SHAPE, "a shape has at most 4 dimensions");
        unsigned __int128 numel = 1;
        for (uint64_t d : e.shape) {
            if (d == 0) return set_err(err, HS_MODEL_INVALID_SHAPE, "a dimension is zero");
            numel *= d;
            if (numel > (unsigned __int128)UINT64_MAX)
                return set_err(err, HS_MODEL_INVALID_SHAPE, "the element count overflows");
        }
        if (numel > (unsigned __int128)INT64_MAX)
            return set_err(err, HS_MODEL_INVALID_SHAPE, "the element count is too large");
        const unsigned __int128 want = numel * sz;
        if (want > (unsigned __int128)UINT64_MAX) return mismatch("the byte length overflows");
        if (e.length != (uint64_t)want) return mismatch("length is not product(shape) * dtype size");
        if (e.has_shift && e.dtype != "i32") return mismatch("only an i32 tensor of rescale multipliers has a shift");
        if (e.offset != off) return layout(e.name, "the offset is not align64 of the end of the section before");
        if (!in_file(e.offset, e.length)) return truncated(e.offset, e.length);
        Stored s;
        s.dtype = e.dtype;
        s.dims = e.shape;
        s.data = bytes + e.offset;
        s.length = e.length;
        s.has_shift = e.has_shift;
        s.shift = e.shift;
        tensors[e.name] = s;
        cursor = off + e.length;
    }
    if (cursor != file_len) return layout("file", "the file does not end at the end of the last section");

    // ---- Model::load (gpt2/model.rs:117-152, 292-343) ----
    if (h.architecture != "gpt2") return bad("model.architecture", "this loader reads only \"gpt2\"");
    if (h.n_layer == 0 || h.n_layer > 1024) return bad("model.n_layer", "must be in 1..=1024");
    if (h.d_model == 0 || h.d_model > 65536) return bad("model.d_model", "must be in 1..=65536");
    if (h.d_ff == 0 || h.d_ff > 65536) return bad("model.d_ff", "must be in 1..=65536");
    if (h.n_head == 0 || h.d_model % h.n_head != 0) return bad("model.n_head", "must be at least 1 and divide d_model");
    if (h.n_ctx < 2 || h.n_ctx > 65536) return bad("model.n_ctx", "must be in 2..=65536 (a restart needs two positions)");

    out.file.assign(bytes, bytes + len);
    const uint8_t *base = out.file.data();
    auto rebase = [&](const uint8_t *p) { return base + (p - bytes); };
    std::set<std::string> taken;
    auto take = [&](const std::string &name, std::vector<uint64_t> dims, bool shift, Stored &s) {
        auto it = tensors.find(name);
        if (it == tensors.end() || taken.count(name))
            return set_err(err, HS_MODEL_MISSING_TENSOR, "missing tensor " + name);
        taken.insert(name);
        s = it->second;
        if (s.dims != dims) return set_err(err, HS_MODEL_TENSOR_MISMATCH, name + ": the shape is not the shape that the model needs");
        if (shift && !s.has_shift) return set_err(err, HS_MODEL_TENSOR_MISMATCH, name + ": a rescale tensor needs a shift");
        if (!shift && s.has_shift) return set_err(err, HS_MODEL_TENSOR_MISMATCH, name + ": only a rescale tensor has a shift");
        return true;
    };
    auto wrong_type = [&](const std::string &name) {
        return set_err(err, HS_MODEL_TENSOR_MISMATCH, name + ": the dtype is not the dtype that the model needs");
    };
    auto i8_matrix = [&](const std::string &name, uint64_t r, uint64_t c, const int8_t *&p) {
        Stored s;
        if (!take(name, {r, c}, false, s)) return false;
        if (s.dtype != "i8") return wrong_type(name);
        p = (const int8_t *)rebase(s.data);
        return true;
    };
    auto i32_vec = [&](const std::string &name, uint64_t n, std::vector<int32_t> &v) {
        Stored s;
        if (!take(name, {n}, false, s)) return false;
        if (s.dtype != "i32") return wrong_type(name);
        v.resize(n);
        std::memcpy(v.data(), s.data, 4 * n);
        return true;
    };
    auto i16_vec = [&](const std::string &name, uint64_t n, std::vector<int16_t> &v) {
        Stored s;
        if (!take(name, {n}, false, s)) return false;
        if (s.dtype != "i16") return wrong_type(name);
        v.resize(n);
        std::memcpy(v.data(), s.data, 2 * n);
        return true;
    };
    auto rows_rescale = [&](const std::string &name, uint64_t n, std::vector<int32_t> &m, uint8_t &sh) {
        Stored s;
        if (!take(name, {n}, true, s)) return false;
        sh = s.shift;
        if (s.dtype != "i32") return wrong_type(name);
        m.resize(n);
        std::memcpy(m.data(), s.data, 4 * n);
        return true;
    };
    auto rescale1 = [&](const std::string &name, int32_t &m, uint8_t &sh) {
        std::vector<int32_t> v;
        if (!rows_rescale(name, 1, v, sh)) return false;
        m = v[0];
        return true;
    };
    auto linear = [&](const std::string &p, uint32_t r, uint32_t c, HostLinear &l) {
        l.rows = r;
        l.cols = c;
        return i8_matrix(p + ".w", r, c, l.w) && i32_vec(p + ".b", r, l.b) &&
               rows_rescale(p + ".rescale", r, l.m, l.s);
    };
    auto layernorm = [&](const std::string &p, HostLayerNorm &n) {
        if (!(i16_vec(p + ".g", h.d_model, n.g) && i32_vec(p + ".b", h.d_model, n.b) &&
              rescale1(p + ".rescale", n.m, n.s)))
            return false;
        // LayerNorm::with_beta_frac (layernorm.rs:153-175)
        if (ln_beta_frac > 0) {
            const uint8_t F = ln_beta_frac, s = n.s;
            if (!(F <= 16 && F <= s && s <= 120 && s - F <= 92))
                return bad("model.constants.ln_beta_frac", "must be in 1..=16, with s - ln_beta_frac in 0..=92 and s <= 120");
        }
        return true;
    };
    auto table_len = [&](const std::string &name, uint64_t &n) {
        auto it = tensors.find(name);
        if (it == tensors.end() || taken.count(name))
            return set_err(err, HS_MODEL_MISSING_TENSOR, "missing tensor " + name);
        if (it->second.dims.size() != 1)
            return set_err(err, HS_MODEL_TENSOR_MISMATCH, name + ": a table has one dimension");
        n = it->second.dims[0];
        return true;
    };
    const uint32_t d = h.d_model, f = h.d_ff, V = h.vocab, C = h.n_ctx;
    if (!i8_matrix("wte", V, d, out.wte)) return false;
    if (!rows_rescale("wte.rescale_embed", V, out.embed_m, out.embed_s)) return false;
    if (!rows_rescale("wte.rescale_logits", V, out.logit_m, out.logit_s)) return false;
    if (!i8_matrix("wpe", C, d, out.wpe)) return false;
    if (!rows_rescale("wpe.rescale", C, out.pos_m, out.pos_s)) return false;
    out.blocks.assign(h.n_layer, HostBlock());
    for (uint32_t l = 0; l < h.n_layer; l++) {
        HostBlock &b = out.blocks[l];
        const std::string p = "h." + std::to_string(l);
        if (!layernorm(p + ".ln_1", b.ln1)) return false;
        if (!linear(p + ".attn.c_attn", 3 * d, d, b.c_attn)) return false;
        if (!rescale1(p + ".attn.score.rescale", b.score_m, b.score_s)) return false;
        if (!rescale1(p + ".attn.out.rescale", b.out_m, b.out_s)) return false;
        if (!linear(p + ".attn.c_proj", d, d, b.c_proj)) return false;
        if (!layernorm(p + ".ln_2", b.ln2)) return false;
        if (!linear(p + ".mlp.c_fc", f, d, b.c_fc)) return false;
        {  // Loader::gelu (model.rs:238-252)
            const std::string gname = p + ".mlp.gelu";
            auto it = tensors.find(gname);
            if (it == tensors.end() || taken.count(gname))
                return set_err(err, HS_MODEL_MISSING_TENSOR, "missing tensor " + gname);
            const uint64_t glen = it->second.dims.empty() ? 0 : it->second.dims[0];
            if (glen != 256 && glen != 65536)
                return set_err(err, HS_MODEL_TENSOR_MISMATCH, gname + ": a GELU table has 256 or 65536 entries");
            Stored s;
            if (!take(gname, {glen}, false, s)) return false;
            b.gelu_len = (uint32_t)glen;
            if (s.dtype == "i16") {
                b.gelu_wide = true;
                b.gelu16.resize(glen);
                std::memcpy(b.gelu16.data(), s.data, 2 * glen);
            } else if (s.dtype == "i8") {
                b.gelu8.resize(glen);
                std::memcpy(b.gelu8.data(), s.data, glen);
            } else {
                return wrong_type(gname);
            }
        }
        if (!linear(p + ".mlp.c_proj", d, f, b.mlp_proj)) return false;
    }
    if (!layernorm("ln_f", out.ln_f)) return false;
    uint64_t alen, llen;
    if (!table_len("attn_exp", alen)) return false;
    if (!i32_vec("attn_exp", alen, out.attn_exp)) return false;
    {  // ExpTable::new (softmax.rs:38-49)
        const auto &t = out.attn_exp;
        bool okt = !t.empty() && t[0] >= 1;
        for (size_t i = 0; okt && i < t.size(); i++) okt = t[i] >= 0 && (i == 0 || t[i] <= t[i - 1]);
        if (!okt) return set_err(err, HS_MODEL_TENSOR_MISMATCH, "attn_exp: entries must be >= 0, not increasing, and the first entry >= 1");
    }
    if (!table_len("logits_exp", llen)) return false;
    {
        Stored s;
        if (!take("logits_exp", {llen}, false, s)) return false;
        if (s.dtype != "u64") return wrong_type("logits_exp");
        out.logits_exp.resize(llen);
        std::memcpy(out.logits_exp.data(), s.data, 8 * llen);
        const auto &t = out.logits_exp;  // LogitTable::new (logits.rs:38-49)
        bool okt = !t.empty() && t[0] >= 1;
        for (size_t i = 0; okt && i < t.size(); i++)
            okt = t[i] <= ((uint64_t)1 << 40) && (i == 0 || t[i] <= t[i - 1]);
        if (!okt) return set_err(err, HS_MODEL_TENSOR_MISMATCH, "logits_exp: entries must be <= 2^40, not increasing, and the first entry >= 1");
    }
    for (auto &kv : tensors)  // remaining tensors, in name order (model.rs:316-321)
        if (!taken.count(kv.first))
            return set_err(err, HS_MODEL_UNEXPECTED_TENSOR, kv.first + ": the gpt2 model does not use this tensor");

    out.version = version;
    out.n_layer = h.n_layer; out.n_head = h.n_head; out.d_model = d; out.d_ff = f;
    out.vocab = V; out.n_ctx = C; out.eot = h.eot; out.head_dim = d / h.n_head;
    out.ln_k = h.ln_k; out.ln_j = h.ln_j; out.ln_eps = h.ln_eps; out.softmax_p = h.softmax_p;
    out.ln_f_bits = ln_f_bits; out.ln_beta_frac = ln_beta_frac;
    sha256(bytes, len, out.hash);
    return true;
}

}  // namespace hs
