// The host harness above the HardShell C ABI (include/taco_hip.h): the role of the reference's
// `taco` crate on the fold/unfold path. Restates crates/taco/src/gpu_fold.rs:128-306 (windows
// and their rows), crates/taco/src/codec.rs:72-310 (the block encoder and its stop rule),
// crates/taco/src/payload.rs:20-60 (LEB128), crates/taco-coder/src/{encoder,decoder}.rs (the
// range coder) and crates/taco-format/src/writer.rs:245-288 (the container).
#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../common.h"
#include "hardshell_hip.h"
#include "taco_hip.h"

namespace {

typedef unsigned __int128 u128;
constexpr uint64_t TOP = (uint64_t)1 << 56;
constexpr uint64_t TOTAL = (uint64_t)1 << TC_FREQ_BITS;

// The range encoder (crates/taco-coder/src/encoder.rs:13-212): a 65-bit `low`, the LZMA carry
// rule with a 64-bit window, and a flush that strips trailing zero bytes.
struct Encoder {
    u128 low = 0;
    uint64_t range = UINT64_MAX;
    uint8_t cache = 0;
    size_t pending = 0;
    std::vector<uint8_t> out;
    size_t nonzero_len = 0;  // the lower bound of the final length (encoder.rs:159-167)

    void shift_low() {
        const uint8_t carry = (uint8_t)((low >> 64) & 1);
        const uint64_t window = (uint64_t)low;
        if (pending == 0 || window < 0xFF00000000000000ull || carry) {
            if (pending > 0) {
                const uint8_t first = (uint8_t)(cache + carry);
                out.push_back(first);
                if (first) nonzero_len = out.size();
                const uint8_t fill = (uint8_t)(0xFF + carry);
                out.insert(out.end(), pending - 1, fill);
                if (fill && pending > 1) nonzero_len = out.size();
            }
            cache = (uint8_t)(window >> 56);
            pending = 0;
        }
        pending++;
        low = (u128)(window << 8);
    }
    void encode(uint64_t start, uint64_t freq) {  // encode_interval with T = 2^32
        const uint64_t r = range >> TC_FREQ_BITS;
        const uint64_t off = r * start;
        low += off;
        range = (start + freq == TOTAL) ? range - off : r * freq;
        while (range < TOP) {
            range <<= 8;
            shift_low();
        }
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

// The range decoder (crates/taco-coder/src/decoder.rs:27-135), target/decode_interval form.
struct Decoder {
    const uint8_t *in = nullptr;
    size_t len = 0, pos = 0;
    uint64_t code = 0, range = UINT64_MAX;
    uint8_t next() { return pos < len ? in[pos++] : (pos++, (uint8_t)0); }
    void init(const uint8_t *p, size_t n) {
        in = p;
        len = n;
        for (int i = 0; i < 8; i++) code = (code << 8) | next();
    }
    uint64_t target() const {
        const uint64_t t = code / (range >> TC_FREQ_BITS);
        return t < TOTAL - 1 ? t : TOTAL - 1;
    }
    bool decode(uint64_t start, uint64_t freq) {
        const uint64_t t = target();
        if (!(t >= start && t - start < freq)) return false;
        const uint64_t r = range >> TC_FREQ_BITS;
        const uint64_t off = r * start;
        code -= off;
        range = (start + freq == TOTAL) ? range - off : r * freq;
        while (range < TOP) {
            range <<= 8;
            code = (code << 8) | next();
        }
        return true;
    }
};

void write_varint(uint64_t v, std::vector<uint8_t> &out) {  // payload.rs:20-31
    for (;;) {
        const uint8_t low = (uint8_t)(v & 0x7F);
        v >>= 7;
        if (!v) {
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

bool read_varint(const uint8_t *b, size_t len, uint64_t &value, size_t &used) {  // payload.rs:40-60
    value = 0;
    unsigned shift = 0;
    for (size_t i = 0; i < len && i < 10; i++) {
        const uint64_t group = b[i] & 0x7F;
        if (i == 9 && group > 1) return false;
        value |= group << shift;
        shift += 7;
        if (!(b[i] & 0x80)) {
            if (b[i] == 0 && i > 0) return false;
            used = i + 1;
            return true;
        }
    }
    return false;
}

// A persistent pool of host threads: run(n, f) calls f(0) .. f(n - 1) on the workers and the
// calling thread and returns when all are done. Blocks are independent streams, so their range
// coders run in parallel (the reference codes blocks in parallel too, crates/taco/src/parallel.rs).
// The pool is never destroyed: its threads wait for work until the process ends. run() may be
// called from several host threads; their jobs run one after another.
class Pool {
  public:
    static Pool &get() {
        static Pool *p = new Pool();
        return *p;
    }
    // Runs f(0) .. f(n - 1) on the calling thread and the workers; returns when all are done.
    // Tasks are claimed from one word holding (job number, next index), so a worker still
    // leaving an earlier job can never claim a task of this one.
    void run(size_t n, const std::function<void(size_t)> &f) {
        if (n <= 1 || workers_ == 0) {
            for (size_t i = 0; i < n; i++) f(i);
            return;
        }
        // one job at a time: callers on several host threads (one per batch) take turns
        std::lock_guard<std::mutex> one(run_mu_);
        const uint64_t job = (word_.load(std::memory_order_relaxed) >> 32) + 1;
        fn_ = &f;
        n_ = n;
        done_.store(0, std::memory_order_relaxed);
        word_.store(job << 32, std::memory_order_release);
        {
            std::lock_guard<std::mutex> lk(mu_);
            posted_ = job;
        }
        cv_.notify_all();
        work(job);
        while (done_.load(std::memory_order_acquire) != n) __builtin_ia32_pause();
    }

  private:
    Pool() {
        const unsigned hw = std::thread::hardware_concurrency();
        workers_ = std::min<unsigned>(hw > 1 ? hw - 1 : 0, 15);
        for (unsigned i = 0; i < workers_; i++) std::thread([this] { loop(); }).detach();
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            uint64_t job;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return posted_ != seen; });
                job = seen = posted_;
            }
            work(job);
        }
    }
    void work(uint64_t job) {
        for (;;) {
            uint64_t w = word_.load(std::memory_order_acquire);
            size_t i;
            for (;;) {
                if ((w >> 32) != job) return;
                i = (size_t)(w & 0xffffffffu);
                if (i >= n_) return;
                if (word_.compare_exchange_weak(w, w + 1, std::memory_order_acq_rel)) break;
            }
            (*fn_)(i);
            done_.fetch_add(1, std::memory_order_release);
        }
    }
    unsigned workers_ = 0;
    std::mutex run_mu_, mu_;
    std::condition_variable cv_;
    uint64_t posted_ = 0;            // the last job posted to the workers
    std::atomic<uint64_t> word_{0};  // job number << 32 | next task index
    std::atomic<size_t> done_{0};
    const std::function<void(size_t)> *fn_ = nullptr;
    size_t n_ = 0;
};

// A context window of a block (gpu_fold.rs:128-134).
struct Window {
    size_t block, first, len;
};

// The block encoder with its stop (codec.rs:72-126, 132-252): the candidate dies when the varint
// and the lower bound of the coder output reach the stop length.
struct BlockEnc {
    Encoder enc;
    uint64_t count = 0;
    size_t prefix = 0, stop = SIZE_MAX;
    bool live = true;
    bool stopped() const { return prefix >= stop || !live; }
    void push(uint64_t start, uint64_t freq) {
        if (!live) return;
        enc.encode(start, freq);
        if (prefix + enc.nonzero_len >= stop) live = false;
    }
};

}  // namespace

extern "C" hs_status tc_fold_blocks(hs_batch *batch, uint32_t overlap, const uint32_t *tokens,
                                    const size_t *offsets, size_t count, const size_t *stop,
                                    uint8_t *out, size_t cap, size_t *lens) {
    if (!batch || (count && (!tokens || !offsets || !out || !lens)))
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    // The model constants come through the batch's model (the caller made the batch for it).
    const size_t slots = hs_batch_slots(batch);
    std::vector<BlockEnc> enc(count);
    for (size_t b = 0; b < count; b++) {
        enc[b].count = offsets[b + 1] - offsets[b];
        enc[b].prefix = varint_len(enc[b].count);
        enc[b].stop = stop ? stop[b] : SIZE_MAX;
    }
    // windows_of (gpu_fold.rs:167-186)
    const size_t n_ctx = hs_model_n_ctx(hs_batch_model(batch));
    const uint32_t eot = hs_model_eot(hs_batch_model(batch));
    const size_t k = overlap;
    if (k + 2 > n_ctx) return hs::fail(HS_MODEL_ERROR, HS_MODEL_INVALID_OVERLAP, "the overlap does not fit the context");
    std::vector<Window> windows;
    for (size_t b = 0; b < count; b++) {
        const size_t n = enc[b].count;
        if (n == 0 || enc[b].stopped()) continue;
        size_t first = 0, size = std::max<size_t>(n_ctx, 2);
        while (first < n) {
            const size_t len = std::min(size, n - first);
            windows.push_back(Window{b, first, len});
            first += len;
            size = std::max<size_t>(1, std::max<size_t>(n_ctx, 2) - std::min(std::max<size_t>(n_ctx, 2), 1 + k));
        }
    }
    // Host scratch kept from call to call on this thread (fresh vectors of a fold step's 16k
    // rows would touch new pages of memory on every call). The names below are references to
    // the calling thread's instances, so the range-coder tasks on the pool's threads (which
    // capture them) see this call's rows.
    struct Scratch {
        std::vector<hs_input> inputs;
        std::vector<hs_query> queries;
        std::vector<int64_t> owner;
        std::vector<hs_interval> answers;
    };
    static thread_local Scratch scratch;
    std::vector<hs_input> &inputs = scratch.inputs;
    std::vector<hs_query> &queries = scratch.queries;
    std::vector<int64_t> &owner = scratch.owner;  // the block of each coded row, -1 for a row that codes nothing
    std::vector<hs_interval> &answers = scratch.answers;
    {
        size_t most = 0;  // rows of the largest wave of windows
        for (size_t w0 = 0; w0 < windows.size(); w0 += slots) {
            size_t r = 0;
            for (size_t wi = w0; wi < std::min(windows.size(), w0 + slots); wi++) r += windows[wi].len + k + 1;
            most = std::max(most, r);
        }
        inputs.reserve(most);
        queries.reserve(most);
        owner.reserve(most);
        answers.reserve(most);
    }
    for (size_t w0 = 0; w0 < windows.size(); w0 += slots) {
        const size_t w1 = std::min(windows.size(), w0 + slots);
        inputs.clear();
        queries.clear();
        owner.clear();
        for (size_t wi = w0; wi < w1; wi++) {
            const Window &w = windows[wi];
            if (enc[w.block].stopped()) continue;
            const uint32_t slot = (uint32_t)(wi - w0);
            hs_batch_reset(batch, slot);
            const uint32_t *t = tokens + offsets[w.block];
            // Window::rows (gpu_fold.rs:145-160)
            auto row = [&](uint32_t in, int64_t code) {
                inputs.push_back(hs_input{slot, in});
                queries.push_back(hs_query{0, code >= 0 ? (uint32_t)code : eot});
                owner.push_back(code >= 0 ? (int64_t)w.block : -1);
            };
            if (w.first == 0) {
                row(eot, t[0]);
            } else {
                row(eot, -1);
                const size_t kept0 = w.first >= 1 + k ? w.first - 1 - k : 0;
                for (size_t i = kept0; i < w.first - 1; i++) row(t[i], -1);
                row(t[w.first - 1], t[w.first]);
            }
            for (size_t i = w.first + 1; i < w.first + w.len; i++) row(t[i - 1], t[i]);
        }
        if (inputs.empty()) continue;
        answers.resize(inputs.size());
        hs_status s = hs_batch_run_coded(batch, inputs.data(), queries.data(), inputs.size(),
                                         TC_FREQ_BITS, answers.data());
        if (s != HS_OK) return s;
        // The rows are in window order: the rows of a block in this wave are one run, so each
        // block's tokens reach its encoder in order, and the blocks' coders run in parallel.
        std::vector<std::pair<size_t, size_t>> runs;  // [begin, end) of each block's coded rows
        for (size_t i = 0; i < inputs.size(); i++) {
            if (owner[i] < 0) continue;
            if (runs.empty() || (size_t)owner[runs.back().first] != (size_t)owner[i]) runs.push_back({i, i});
            runs.back().second = i + 1;
        }
        std::atomic<bool> bad(false);
        Pool::get().run(runs.size(), [&](size_t r) {
            BlockEnc &be = enc[(size_t)owner[runs[r].first]];
            for (size_t i = runs[r].first; i < runs[r].second; i++) {
                if (owner[i] < 0) continue;
                const hs_interval &a = answers[i];
                // lanes.rs:121-128: a bad interval or last-symbol flag is a fault of the device
                if (a.freq == 0 || a.start > TOTAL || a.freq > TOTAL - a.start || a.symbol != queries[i].value) {
                    bad = true;
                    return;
                }
                be.push(a.start, a.freq);
            }
        });
        if (bad) return hs::fail(HS_DEVICE_ERROR, 0, "the coder op gave a bad interval");
    }
    for (size_t b = 0; b < count; b++) {
        BlockEnc &e = enc[b];
        if (e.stopped()) {
            lens[b] = SIZE_MAX;
            continue;
        }
        std::vector<uint8_t> p;
        write_varint(e.count, p);
        if (e.count > 0) {
            std::vector<uint8_t> body = e.enc.finish();
            p.insert(p.end(), body.begin(), body.end());
        }
        lens[b] = p.size();
        if (p.size() <= cap) std::memcpy(out + b * cap, p.data(), p.size());
    }
    return HS_OK;
}

extern "C" hs_status tc_unfold_blocks(hs_batch *batch, uint32_t overlap, const uint8_t *payloads,
                                      const size_t *offsets, size_t count, uint32_t *tokens,
                                      size_t cap, size_t *counts) {
    if (!batch || (count && (!payloads || !offsets || !tokens || !counts)))
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    // The lanes of gpu_unfold.rs run at the container's overlap: restarts inside the backend
    // keep that many tokens (the batch refuses an overlap that does not fit its context).
    hs_status s = hs_batch_set_overlap(batch, overlap);
    if (s != HS_OK) return s;
    const size_t slots = hs_batch_slots(batch);
    const uint32_t eot = hs_model_eot(hs_batch_model(batch));
    std::vector<Decoder> dec(count);
    std::vector<uint64_t> total(count, 0), done(count, 0);
    for (size_t b = 0; b < count; b++) {
        const uint8_t *p = payloads + offsets[b];
        const size_t n = offsets[b + 1] - offsets[b];
        size_t used = 0;
        if (!read_varint(p, n, total[b], used) || total[b] > cap)
            return hs::fail(HS_LENGTH_MISMATCH, (int)b, "block " + std::to_string(b) + ": the token count is not valid");
        dec[b].init(p + used, n - used);
        counts[b] = (size_t)total[b];
    }
    // A job queue over the slots (decode_jobs, gpu_unfold.rs:74-196): a slot whose block is
    // complete resets and takes the next waiting block, so a long block does not hold the
    // slots of short ones idle. Blocks of no tokens need no rows.
    std::vector<int64_t> job(slots, -1);
    size_t next = 0;
    auto take = [&](size_t slot) {
        while (next < count && total[next] == 0) next++;
        job[slot] = next < count ? (int64_t)next++ : -1;
        if (job[slot] >= 0) hs_batch_reset(batch, slot);
    };
    for (size_t slot = 0; slot < slots; slot++) take(slot);
    std::vector<hs_input> inputs;
    std::vector<hs_query> queries;
    std::vector<size_t> live;  // the slot of each row
    std::vector<hs_interval> answers;
    for (;;) {
        inputs.clear();
        queries.clear();
        live.clear();
        for (size_t slot = 0; slot < slots; slot++) {
            if (job[slot] < 0) continue;
            const size_t b = (size_t)job[slot];
            const uint32_t prev = done[b] == 0 ? eot : tokens[b * cap + done[b] - 1];
            inputs.push_back(hs_input{(uint32_t)slot, prev});
            queries.push_back(hs_query{1, (uint32_t)dec[b].target()});
            live.push_back(slot);
        }
        if (live.empty()) break;
        answers.resize(inputs.size());
        s = hs_batch_run_coded(batch, inputs.data(), queries.data(), inputs.size(), TC_FREQ_BITS,
                               answers.data());
        if (s != HS_OK) return s;
        for (size_t i = 0; i < live.size(); i++) {
            const size_t slot = live[i], b = (size_t)job[slot];
            const hs_interval &a = answers[i];
            if (!dec[b].decode(a.start, a.freq))
                return hs::fail(HS_DEVICE_ERROR, (int)b, "the coder op gave an interval that does not hold the target");
            tokens[b * cap + done[b]] = (uint32_t)a.symbol;
            if (++done[b] == total[b]) take(slot);
        }
    }
    return HS_OK;
}

extern "C" size_t tc_container_build(const uint8_t model_hash[32], const uint8_t *original, size_t len,
                                     uint32_t block_size, uint32_t overlap, const uint8_t *kinds,
                                     const uint8_t *blocks, const size_t *block_offsets, uint8_t *out,
                                     size_t cap) {
    if (block_size == 0 || !model_hash) return 0;
    const uint64_t count = (len + block_size - 1) / block_size;
    std::vector<uint8_t> o;
    auto put = [&](uint64_t v, int bytes) {
        for (int i = 0; i < bytes; i++) o.push_back((uint8_t)(v >> (8 * i)));
    };
    // Header (taco-format/src/header.rs:200-215, lib.rs:14-36): 104 bytes in version 2.
    o.insert(o.end(), {'T', 'A', 'C', 'O'});
    put(2, 2);
    put(0, 2);
    o.insert(o.end(), model_hash, model_hash + 32);
    put(len, 8);
    uint8_t digest[32];
    hs::sha256(original, len, digest);
    o.insert(o.end(), digest, digest + 32);
    put(block_size, 4);
    put(count, 4);
    o.push_back(0);                 // profile: text
    o.push_back(0);                 // reserved
    put(overlap ? 2 : 0, 2);        // coding parts: bit 1 = the context overlap
    uint8_t params[12] = {0};
    if (overlap) {
        params[2] = (uint8_t)(overlap & 0xFF);
        params[3] = (uint8_t)(overlap >> 8);
    }
    o.insert(o.end(), params, params + 12);
    std::vector<size_t> stored(count);
    for (uint64_t b = 0; b < count; b++) {
        const size_t orig = std::min<size_t>(block_size, len - b * block_size);
        size_t sl = orig;
        if (kinds[b] == 1) {
            sl = block_offsets[b + 1] - block_offsets[b];
            if (sl >= orig) return 0;  // a coded block must be smaller (writer.rs:71-104)
        } else if (kinds[b] != 0) {
            return 0;
        }
        stored[b] = sl;
        o.push_back(kinds[b]);
        put(sl, 4);
    }
    for (uint64_t b = 0; b < count; b++) {
        if (kinds[b] == 1)
            o.insert(o.end(), blocks + block_offsets[b], blocks + block_offsets[b + 1]);
        else
            o.insert(o.end(), original + b * block_size, original + b * block_size + stored[b]);
    }
    if (o.size() <= cap && out) std::memcpy(out, o.data(), o.size());
    return o.size();
}

// The byte-level fold of the text profile (crates/taco/src/fold.rs:502-565): tokenize each
// block (its tokens must restore its bytes, tokens_restore), code the blocks on the batch with a
// stop at the block's length, and store each block as the smaller of its payload and its bytes.
extern "C" hs_status tc_fold_bytes(hs_batch *batch, const tc_tokenizer *tok, const uint8_t *data, size_t len,
                                   uint32_t block_size, uint32_t overlap, uint8_t *out, size_t cap,
                                   size_t *out_len) {
    hs::clear_error();
    if (!batch || !tok || !out_len || (len && !data)) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (block_size == 0) return hs::fail(HS_UNSUPPORTED, 0, "the block size must be at least 1");
    const hs_model *model = hs_batch_model(batch);
    const size_t count = (len + block_size - 1) / block_size;
    std::vector<uint32_t> tokens;
    std::vector<size_t> offsets(count + 1, 0), stop(count);
    std::vector<uint32_t> ids;
    for (size_t b = 0; b < count; b++) {
        const size_t b0 = b * block_size, bl = std::min<size_t>(block_size, len - b0);
        size_t n = 0;
        ids.resize(bl + 1);  // at most one token per byte
        hs_status s = tc_tokenize(tok, data + b0, bl, ids.data(), ids.size(), &n);
        if (s != HS_OK) return s;
        // tokens_restore: the bytes of the tokens are the block's bytes
        size_t at = 0;
        for (size_t i = 0; i < n; i++) {
            const uint8_t *p;
            size_t tl;
            if ((s = hs_model_token(model, ids[i], &p, &tl)) != HS_OK) return s;
            if (at + tl > bl || std::memcmp(data + b0 + at, p, tl) != 0)
                return hs::fail(HS_MODEL_ERROR, HS_MODEL_VOCABULARY,
                                "block " + std::to_string(b) + ": the tokens do not restore the block's bytes");
            at += tl;
        }
        if (at != bl)
            return hs::fail(HS_MODEL_ERROR, HS_MODEL_VOCABULARY,
                            "block " + std::to_string(b) + ": the tokens do not restore the block's bytes");
        tokens.insert(tokens.end(), ids.begin(), ids.begin() + n);
        offsets[b + 1] = tokens.size();
        stop[b] = bl;
    }
    // payloads of at most the block's bytes (a longer one is never chosen)
    const size_t pcap = block_size + 16;
    std::vector<uint8_t> payloads(count * pcap);
    std::vector<size_t> lens(count);
    if (count) {
        hs_status s = tc_fold_blocks(batch, overlap, tokens.data(), offsets.data(), count, stop.data(),
                                     payloads.data(), pcap, lens.data());
        if (s != HS_OK) return s;
    }
    std::vector<uint8_t> kinds(count), blocks;
    std::vector<size_t> boffs(count + 1, 0);
    for (size_t b = 0; b < count; b++) {
        const size_t bl = std::min<size_t>(block_size, len - b * block_size);
        kinds[b] = lens[b] != SIZE_MAX && lens[b] < bl;  // Block::choose_smallest (writer.rs:71-104)
        if (kinds[b]) blocks.insert(blocks.end(), payloads.begin() + b * pcap, payloads.begin() + b * pcap + lens[b]);
        boffs[b + 1] = blocks.size();
    }
    uint8_t hash[32];
    hs_model_hash(model, hash);
    const size_t n = tc_container_build(hash, data, len, block_size, overlap, kinds.data(), blocks.data(),
                                        boffs.data(), out, cap);
    if (n == 0) return hs::fail(HS_DEVICE_ERROR, 0, "the container could not be built");
    *out_len = n;
    return HS_OK;
}
