// The C ABI of libhardshell_hip.so (include/hardshell_hip.h): device, model, batch and op-level
// entry points. Host orchestration of the kernels in kernels.hip.
//
// Mirrors crates/hardshell-cuda/src/{device,model,batch,ops}.rs: the same methods, argument
// meaning and error behaviour (validation before any device work, positions committed only
// after every pass of a call succeeded).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <functional>
#include <vector>

#include "common.h"
#include "hardshell_hip.h"
#include "hsm.h"
#include "kernels.h"

#ifndef HS_SOURCE_SHA256
#define HS_SOURCE_SHA256 "unknown"
#endif

using hs::Epi;
using hs::RowInfo;

namespace {

constexpr size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

hs_status hip_fail(const char *call, hipError_t e) {
    return hs::fail(HS_DEVICE_ERROR, (int)e, std::string(call) + " failed: " + hipGetErrorName(e));
}

#define HIP_TRY(call)                                    \
    do {                                                 \
        hipError_t e_ = (call);                          \
        if (e_ != hipSuccess) return hip_fail(#call, e_); \
    } while (0)

#define HS_TRY(call)                       \
    do {                                   \
        const hs_status s_ = (call);       \
        if (s_ != HS_OK) return s_;        \
    } while (0)

// Device allocations owned by a handle; freed in reverse order.
struct DevMem {
    std::vector<void *> ptrs;
    uint64_t bytes = 0;
    ~DevMem() {
        for (auto it = ptrs.rbegin(); it != ptrs.rend(); ++it) (void)hipFree(*it);
    }
    template <typename T>
    hs_status alloc(T *&p, size_t count) {
        void *v = nullptr;
        const size_t n = std::max<size_t>(count * sizeof(T), 256);
        hipError_t e = hipMalloc(&v, n);
        if (e != hipSuccess) return hip_fail("hipMalloc", e);
        e = hipMemset(v, 0, n);
        if (e != hipSuccess) {
            (void)hipFree(v);
            return hip_fail("hipMemset", e);
        }
        ptrs.push_back(v);
        bytes += n;
        p = (T *)v;
        return HS_OK;
    }
    template <typename T>
    // count entries from src, zero up to alloc_count
    hs_status upload(T *&p, const T *src, size_t count, size_t alloc_count = 0) {
        hs_status st = alloc(p, std::max(count, alloc_count));
        if (st != HS_OK) return st;
        if (count) HIP_TRY(hipMemcpy(p, src, count * sizeof(T), hipMemcpyHostToDevice));
        if (alloc_count > count) HIP_TRY(hipMemset(p + count, 0, (alloc_count - count) * sizeof(T)));
        return HS_OK;
    }
};

}  // namespace

struct hs_device {
    int ordinal = 0;
    std::string name;
    hipStream_t stream = nullptr;
    void *fixed_scratch = nullptr;  // this device's copy of `scratch` (below), a device address
};

// The scratch of hs_op_attend_decode_dev_noalloc: one array per GPU, loaded with the code
// object and held until the process ends. In host code `scratch` names a host-side stand-in,
// never the device memory: every use goes through the per-device address that
// hipGetSymbolAddress gives at hs_device_open (fixed_scratch_of).
constexpr size_t HS_FIXED_SCRATCH_BYTES = (size_t)64 << 20;
static __device__ __align__(256) char scratch[HS_FIXED_SCRATCH_BYTES];

namespace {

std::mutex g_fixed_mu;
std::vector<void *> g_fixed_scratch;  // by device ordinal

// The device address of `scratch` on the current device `ordinal`, looked up once per device.
hipError_t fixed_scratch_of(int ordinal, void **out) {
    std::lock_guard<std::mutex> lock(g_fixed_mu);
    if ((size_t)ordinal >= g_fixed_scratch.size()) g_fixed_scratch.resize((size_t)ordinal + 1, nullptr);
    if (!g_fixed_scratch[ordinal]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_fixed_scratch[ordinal] = p;
    }
    *out = g_fixed_scratch[ordinal];
    return hipSuccess;
}

}  // namespace

namespace {

struct DevLinear {
    int8_t *w = nullptr;  // panels [k_pad / 64][n_pad][64] (hs::panel_off)
    int32_t *b = nullptr, *m = nullptr;
    int s = 0, n = 0, k = 0, n_pad = 0, k_pad = 0;
    int fast32 = 0;  // k * 2^14 + max|b| < 2^31: every acc + b fits i32
    int32_t *wsum = nullptr;  // sum_k w[n][k], for an i16 input as planes (|wsum| <= 2^23)
};

// A GEMM operand of `rows` dense rows of `cols` bytes as the kernels read it: panels of 64 bytes
// of K, [k_pad / 64][rows_pad][64], zero beyond the rows and columns.
std::vector<int8_t> pack_panels(const int8_t *src, size_t rows, size_t cols, size_t rows_pad, size_t k_pad) {
    std::vector<int8_t> p(rows_pad * k_pad, 0);
    for (size_t r = 0; r < rows; r++)
        for (size_t c0 = 0; c0 < cols; c0 += 64)
            std::memcpy(&p[hs::panel_off(r, c0, rows_pad)], src + r * cols + c0, std::min<size_t>(64, cols - c0));
    return p;
}

// The row sums of w [n, k] (i8), exact in i32 (|sum| <= k 2^7 <= 2^23).
std::vector<int32_t> row_sums(const int8_t *w, size_t n, size_t k, size_t n_pad) {
    std::vector<int32_t> s(n_pad, 0);
    for (size_t r = 0; r < n; r++) {
        int32_t t = 0;
        for (size_t c = 0; c < k; c++) t += w[r * k + c];
        s[r] = t;
    }
    return s;
}

// |acc| <= k * 128 * 128 for i8 operands, so acc + b fits i32 when k * 2^14 + max|b| < 2^31.
int fits_i32(size_t k, const int32_t *b, size_t n) {
    int64_t mb = 0;
    for (size_t i = 0; b && i < n; i++) mb = std::max<int64_t>(mb, b[i] < 0 ? -(int64_t)b[i] : b[i]);
    return (int64_t)k * 16384 + mb < ((int64_t)1 << 31) ? 1 : 0;
}

struct DevLn {
    int16_t *g = nullptr;
    int64_t *gm = nullptr;  // g[j] * m
    int32_t *b = nullptr;
    int32_t m = 0;
    int s = 0;
    bool beta_small = false;  // every |b[j]| <= 256
};

struct DevBlock {
    DevLn ln1, ln2;
    DevLinear c_attn, c_proj, c_fc, mlp_proj;
    int32_t score_m = 0, out_m = 0;
    int score_s = 0, out_s = 0;
    int8_t *gelu = nullptr;
    int16_t *gelu16 = nullptr;  // an i16 table (version 2): c_fc writes planes, mlp_proj reads them
    int gelu_off = 0;
    // the span of the i8 table past whose ends the entries repeat (GemmArgs::gelu_lo ..)
    int gelu_lo = 0, gelu_clo = 0, gelu_chi = 0, gelu_shift = 0, gelu_copy = 0;
};

}  // namespace

struct hs_model {
    hs_device *dev = nullptr;
    hs::HostModel host;
    DevMem mem;
    int d = 0, f = 0, V = 0, C = 0, H = 0, hd = 0, L = 0;
    int d_pad = 0, f_pad = 0, V_pad = 0;
    int8_t *wte = nullptr;  // the LM head operand, panels of V_pad rows; the embedding reads row tok
    int32_t *wte_sum = nullptr;  // row sums of wte, for a 16-bit ln_f (version 2)
    bool wide_ln_f = false, wide_gelu = false;
    int8_t *wpe = nullptr;  // [C, d]
    int32_t *embed_m = nullptr, *logit_m = nullptr, *pos_m = nullptr;
    std::vector<DevBlock> blocks;
    DevLn ln_f;
    int32_t *attn_exp = nullptr;
    int attn_exp_last = 0;  // > 0: attn_exp[i] == 0 for every i >= attn_exp_last (AttnArgs::exp_last)
    uint64_t *logits_exp = nullptr;
    uint64_t weight_bytes = 0;
    bool compact = false;  // the LM head writes compact logits (table_len <= CODER_MAX_TABLE)
    int d0 = 0;            // the largest d with logits_exp[d] == logits_exp[0]
    int zcut = 0;          // logits_exp[d] == 0 for every d >= zcut
    int ntiles = 0, ld16 = 0;
};

namespace {

hs_status upload_linear(DevMem &mem, const hs::HostLinear &l, DevLinear &o) {
    o.n = (int)l.rows;
    o.k = (int)l.cols;
    o.n_pad = (int)round_up(l.rows, hs::GEMM_NPAD);
    o.k_pad = (int)round_up(l.cols, hs::GEMM_BK);
    const std::vector<int8_t> w = pack_panels(l.w, l.rows, l.cols, o.n_pad, o.k_pad);
    hs_status st = mem.upload(o.w, w.data(), w.size());
    if (st == HS_OK) st = mem.upload(o.b, l.b.data(), l.b.size(), o.n_pad);
    if (st == HS_OK) st = mem.upload(o.m, l.m.data(), l.m.size(), o.n_pad);
    o.s = l.s;
    o.fast32 = fits_i32(l.cols, l.b.data(), l.b.size());
    return st;
}

hs_status upload_ln(DevMem &mem, const hs::HostLayerNorm &l, DevLn &o) {
    std::vector<int64_t> gm(l.g.size());
    for (size_t j = 0; j < gm.size(); j++) gm[j] = (int64_t)l.g[j] * (int64_t)l.m;
    hs_status st = mem.upload(o.g, l.g.data(), l.g.size());
    if (st == HS_OK) st = mem.upload(o.gm, gm.data(), gm.size());
    if (st == HS_OK) st = mem.upload(o.b, l.b.data(), l.b.size());
    o.m = l.m;
    o.s = l.s;
    o.beta_small = true;
    for (int32_t v : l.b) o.beta_small = o.beta_small && v >= -256 && v <= 256;
    return st;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// Device
// ---------------------------------------------------------------------------------------------

extern "C" const char *hs_version(void) {
    return "hardshell-hip " "0.1.0" " gfx950 kernels sha256:" HS_SOURCE_SHA256;
}

extern "C" hs_status hs_device_open(int ordinal, hs_device **out) {
    hs::clear_error();
    if (!out) return hs::fail(HS_INVALID_ARGUMENT, 0, "out is NULL");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return hs::fail(HS_NO_DEVICE, (int)e, "no HIP device: " + std::string(hipGetErrorName(e)));
    if (ordinal < 0 || ordinal >= count)
        return hs::fail(HS_NO_DEVICE, 0, "no HIP device with ordinal " + std::to_string(ordinal));
    HIP_TRY(hipSetDevice(ordinal));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, ordinal));
    const std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return hs::fail(HS_UNSUPPORTED, 0, "the kernels are built for gfx950 only; this device is " + arch);
    auto dev = std::make_unique<hs_device>();
    dev->ordinal = ordinal;
    dev->name = prop.name[0] ? std::string(prop.name) : "AMD " + arch;
    HIP_TRY(fixed_scratch_of(ordinal, &dev->fixed_scratch));
    HIP_TRY(hipStreamCreate(&dev->stream));
    *out = dev.release();
    return HS_OK;
}

extern "C" void hs_device_close(hs_device *dev) {
    if (!dev) return;
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    delete dev;
}

extern "C" hs_status hs_device_name(const hs_device *dev, char *buf, size_t cap) {
    if (!dev || !buf || cap == 0) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    std::strncpy(buf, dev->name.c_str(), cap - 1);
    buf[cap - 1] = 0;
    return HS_OK;
}

extern "C" hs_status hs_device_kernel_resources(hs_device *dev, char *names, int32_t *regs,
                                                int32_t *private_bytes, int32_t *static_lds_bytes,
                                                size_t cap, size_t *count) {
    hs::clear_error();
    if (!dev || !count || (cap && (!names || !regs || !private_bytes || !static_lds_bytes)))
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    HIP_TRY(hipSetDevice(dev->ordinal));
    std::vector<hs::KernelResource> r(64);
    const int n = hs::kernel_resources(r.data(), (int)r.size());
    if (n < 0) return hip_fail("hipFuncGetAttributes", (hipError_t)(-n));
    for (int i = 0; i < n && (size_t)i < cap; i++) {
        std::memset(names + 64 * (size_t)i, 0, 64);
        std::strncpy(names + 64 * (size_t)i, r[i].name, 63);
        regs[i] = r[i].regs;
        private_bytes[i] = r[i].private_bytes;
        static_lds_bytes[i] = r[i].static_lds_bytes;
    }
    *count = (size_t)n;
    return HS_OK;
}

extern "C" hs_status hs_device_memory(const hs_device *dev, size_t *free_bytes, size_t *total_bytes) {
    if (!dev || !free_bytes || !total_bytes) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    HIP_TRY(hipSetDevice(dev->ordinal));
    HIP_TRY(hipMemGetInfo(free_bytes, total_bytes));
    return HS_OK;
}

// ---------------------------------------------------------------------------------------------
// Model: crates/hardshell-cuda/src/model.rs:242-349
// ---------------------------------------------------------------------------------------------

namespace {

// A copy of a parsed model whose tensor pointers point into the copy's own file bytes.
void copy_host_model(const hs::HostModel &src, hs::HostModel &dst) {
    dst = src;
    const int8_t *s0 = (const int8_t *)src.file.data();
    const int8_t *d0 = (const int8_t *)dst.file.data();
    auto rebase = [&](const int8_t *p) { return p ? d0 + (p - s0) : nullptr; };
    dst.wte = rebase(src.wte);
    dst.wpe = rebase(src.wpe);
    for (size_t l = 0; l < dst.blocks.size(); l++) {
        dst.blocks[l].c_attn.w = rebase(src.blocks[l].c_attn.w);
        dst.blocks[l].c_proj.w = rebase(src.blocks[l].c_proj.w);
        dst.blocks[l].c_fc.w = rebase(src.blocks[l].c_fc.w);
        dst.blocks[l].mlp_proj.w = rebase(src.blocks[l].mlp_proj.w);
    }
}

hs_status upload_model(hs_device *dev, std::unique_ptr<hs_model> &m, hs_model **out);

}  // namespace

extern "C" hs_status hs_model_load(hs_device *dev, const uint8_t *bytes, size_t len, hs_model **out) {
    hs::clear_error();
    if (!dev || !bytes || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    *out = nullptr;
    auto m = std::make_unique<hs_model>();
    hs::ModelError err{};
    if (!hs::load_host_model(bytes, len, m->host, err)) return hs::fail(HS_MODEL_ERROR, err.kind, err.msg);
    return upload_model(dev, m, out);
}

extern "C" hs_status hs_model_load_with(hs_device *dev, const uint8_t *bytes, size_t len,
                                        const hs_model *loaded, hs_model **out) {
    hs::clear_error();
    if (!dev || !bytes || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    *out = nullptr;
    if (!loaded) return hs_model_load(dev, bytes, len, out);
    uint8_t hash[32];
    hs::sha256(bytes, len, hash);
    // the bytes of a model the library already parsed and checked: its parse is reused (the
    // checks are not repeated); any other file gets its own full load (model.rs:259-274)
    if (std::memcmp(hash, loaded->host.hash, 32) != 0) return hs_model_load(dev, bytes, len, out);
    auto m = std::make_unique<hs_model>();
    copy_host_model(loaded->host, m->host);
    return upload_model(dev, m, out);
}

namespace {

hs_status upload_model(hs_device *dev, std::unique_ptr<hs_model> &m, hs_model **out) {
    const hs::HostModel &h = m->host;
    if (h.head_dim % 4 != 0 || h.head_dim > 256)
        return hs::fail(HS_UNSUPPORTED, 0, "head_dim must be a multiple of 4 and at most 256");
    HIP_TRY(hipSetDevice(dev->ordinal));
    m->dev = dev;
    m->d = (int)h.d_model; m->f = (int)h.d_ff; m->V = (int)h.vocab; m->C = (int)h.n_ctx;
    m->H = (int)h.n_head; m->hd = (int)h.head_dim; m->L = (int)h.n_layer;
    m->d_pad = (int)round_up(h.d_model, hs::GEMM_BK);
    m->f_pad = (int)round_up(h.d_ff, hs::GEMM_BK);
    m->V_pad = (int)round_up(h.vocab, hs::GEMM_NPAD);
    DevMem &mem = m->mem;
    hs_status st;
    {
        const std::vector<int8_t> w = pack_panels(h.wte, m->V, m->d, m->V_pad, m->d_pad);
        if ((st = mem.upload(m->wte, w.data(), w.size())) != HS_OK) return st;
    }
    m->wide_ln_f = h.ln_f_bits == 16;
    if (m->wide_ln_f) {
        const std::vector<int32_t> ws = row_sums(h.wte, m->V, m->d, m->V_pad);
        if ((st = mem.upload(m->wte_sum, ws.data(), ws.size())) != HS_OK) return st;
    }
    if ((st = mem.upload(m->wpe, h.wpe, (size_t)m->C * m->d)) != HS_OK) return st;
    if ((st = mem.upload(m->embed_m, h.embed_m.data(), h.embed_m.size())) != HS_OK) return st;
    if ((st = mem.upload(m->logit_m, h.logit_m.data(), h.logit_m.size(), m->V_pad)) != HS_OK) return st;
    if ((st = mem.upload(m->pos_m, h.pos_m.data(), h.pos_m.size())) != HS_OK) return st;
    m->blocks.resize(m->L);
    for (int l = 0; l < m->L; l++) {
        const hs::HostBlock &hb = h.blocks[l];
        DevBlock &b = m->blocks[l];
        if ((st = upload_ln(mem, hb.ln1, b.ln1)) != HS_OK) return st;
        if ((st = upload_ln(mem, hb.ln2, b.ln2)) != HS_OK) return st;
        if ((st = upload_linear(mem, hb.c_attn, b.c_attn)) != HS_OK) return st;
        if ((st = upload_linear(mem, hb.c_proj, b.c_proj)) != HS_OK) return st;
        if ((st = upload_linear(mem, hb.c_fc, b.c_fc)) != HS_OK) return st;
        if ((st = upload_linear(mem, hb.mlp_proj, b.mlp_proj)) != HS_OK) return st;
        b.score_m = hb.score_m; b.score_s = hb.score_s;
        b.out_m = hb.out_m; b.out_s = hb.out_s;
        if (hb.gelu_wide) {
            m->wide_gelu = true;
            if ((st = mem.upload(b.gelu16, hb.gelu16.data(), hb.gelu16.size())) != HS_OK) return st;
            const std::vector<int32_t> ws = row_sums(hb.mlp_proj.w, hb.mlp_proj.rows, hb.mlp_proj.cols, b.mlp_proj.n_pad);
            if ((st = mem.upload(b.mlp_proj.wsum, ws.data(), ws.size())) != HS_OK) return st;
        } else if ((st = mem.upload(b.gelu, hb.gelu8.data(), hb.gelu8.size())) != HS_OK) {
            return st;
        }
        b.gelu_off = (int)hb.gelu_len / 2;
        if (!hb.gelu_wide && hb.gelu8.size() >= 16 && hb.gelu8.size() % 16 == 0) {
            // the span [lo, hi] outside which every entry equals the end entry it lies beyond: the
            // epilogue clamps its index to it and copies only entries lo16 .. (16-byte aligned)
            const std::vector<int8_t> &t = hb.gelu8;
            const int len = (int)t.size();
            int lo = 0, hi = len - 1;
            while (lo + 1 < len && t[lo + 1] == t[0]) lo++;
            while (hi - 1 > lo && t[hi - 1] == t[len - 1]) hi--;
            const int lo16 = lo & ~15, end16 = std::min(len, (hi + 16) & ~15);
            b.gelu_lo = lo16;
            b.gelu_clo = lo - b.gelu_off;
            b.gelu_chi = hi - b.gelu_off;
            b.gelu_shift = b.gelu_off - lo16;
            b.gelu_copy = end16 - lo16;
        }
    }
    if ((st = upload_ln(mem, h.ln_f, m->ln_f)) != HS_OK) return st;
    // padded to a multiple of 256 entries: the prefill attention loads it in 1 KiB chunks
    if ((st = mem.upload(m->attn_exp, h.attn_exp.data(), h.attn_exp.size(), (h.attn_exp.size() + 255) / 256 * 256)) != HS_OK) return st;
    {  // the zero tail of attn_exp: the short prefill kernel copies only the entries before it
        size_t z = h.attn_exp.size();
        while (z > 0 && h.attn_exp[z - 1] == 0) z--;
        m->attn_exp_last = z < h.attn_exp.size() ? (int)z : 0;
    }
    // zero-padded to at least CODER_TABLE_READ entries: the compact coder loads its first bins'
    // entries without bounds tests
    if ((st = mem.upload(m->logits_exp, h.logits_exp.data(), h.logits_exp.size(),
                         std::max<size_t>(h.logits_exp.size(), hs::CODER_TABLE_READ))) != HS_OK)
        return st;
    m->compact = h.logits_exp.size() <= (size_t)hs::CODER_MAX_TABLE;
    while ((size_t)m->d0 + 1 < h.logits_exp.size() && h.logits_exp[m->d0 + 1] == h.logits_exp[0]) m->d0++;
    m->zcut = (int)h.logits_exp.size();
    while (m->zcut > 1 && h.logits_exp[m->zcut - 1] == 0) m->zcut--;
    m->ntiles = (m->V + 63) / 64;
    m->ld16 = (int)round_up(m->V, 64);
    m->weight_bytes = mem.bytes;
    *out = m.release();
    return HS_OK;
}

}  // namespace

extern "C" void hs_model_free(hs_model *model) { delete model; }

extern "C" hs_status hs_model_token(const hs_model *model, uint32_t id, const uint8_t **bytes, size_t *len) {
    hs::clear_error();
    if (!model || !bytes || !len) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    const hs::HostModel &h = model->host;
    if (id >= h.vocab) return hs::fail(HS_MODEL_ERROR, HS_MODEL_TOKEN_OUT_OF_RANGE, "token " + std::to_string(id) + " is not in the vocabulary");
    const uint32_t s = id == 0 ? 0 : h.vocab_ends[id - 1];
    *bytes = h.vocab_bytes.data() + s;
    *len = h.vocab_ends[id] - s;
    return HS_OK;
}

extern "C" size_t hs_model_merges(const hs_model *model, const uint32_t **pairs) {
    if (!model) return 0;
    if (pairs) *pairs = model->host.merges.data();
    return model->host.merges.size() / 2;
}

extern "C" hs_status hs_model_validate(const uint8_t *bytes, size_t len, uint8_t hash[32]) {
    hs::clear_error();
    if (!bytes && len) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    hs::HostModel h;
    hs::ModelError err{};
    if (!hs::load_host_model(bytes ? bytes : (const uint8_t *)"", len, h, err))
        return hs::fail(HS_MODEL_ERROR, err.kind, err.msg);
    if (hash) std::memcpy(hash, h.hash, 32);
    return HS_OK;
}
extern "C" void hs_model_hash(const hs_model *m, uint8_t out[32]) {
    if (m && out) std::memcpy(out, m->host.hash, 32);
}
extern "C" uint32_t hs_model_vocab(const hs_model *m) { return m ? m->host.vocab : 0; }
extern "C" uint32_t hs_model_n_ctx(const hs_model *m) { return m ? m->host.n_ctx : 0; }
extern "C" uint32_t hs_model_eot(const hs_model *m) { return m ? m->host.eot : 0; }
extern "C" int hs_model_is_wide(const hs_model *m) { return m && m->host.is_wide() ? 1 : 0; }
extern "C" uint64_t hs_model_weight_bytes(const hs_model *m) { return m ? m->weight_bytes : 0; }
extern "C" uint64_t hs_model_cache_bytes_per_slot(const hs_model *m) {
    return m ? 2ull * m->host.n_layer * m->host.n_ctx * m->host.d_model : 0;
}

// ---------------------------------------------------------------------------------------------
// Batch: crates/hardshell-cuda/src/batch.rs, batch/plan.rs
// ---------------------------------------------------------------------------------------------

namespace {

struct PassRow {
    uint32_t slot, token, pos;
    int64_t input;  // index of the input it answers, -1 for a restart row
};

// The bookkeeping of the inputs of one slot for a truncation (crates/hardshell/src/gpt2/
// stream.rs:43-204): the inputs since the last reset, the first position of the current context
// that holds an input, one more than the highest position written, and `first` of the context
// before the last restart.
struct StreamState {
    size_t len = 0, first = 0, written = 0;
    bool has_prev = false;
    size_t prev_first = 0;

    // stream.rs:119-121: the inputs a slot at `pos` takes before its next restart.
    static size_t room(size_t pos, size_t n_ctx, size_t k) {
        if (pos >= n_ctx) return n_ctx > k + 1 ? n_ctx - (k + 1) : 0;
        return n_ctx - pos;
    }
    void input(size_t pos) {
        len += 1;
        written = std::max(written, pos + 1);
    }
    void restart(size_t k) {
        prev_first = first;
        has_prev = true;
        first = k + 1;
        written = k + 1;
    }
};

struct Truncation {
    size_t len = 0, pos = 0;
    bool restore = false;
    size_t rebuild_end = 0;  // positions 0 .. rebuild_end run again with the kept history
};

// stream.rs:155-172. Returns false for a truncation the rules refuse (BadTruncate).
bool plan_truncate(const StreamState &st, size_t len, size_t pos, size_t n_ctx, Truncation &t) {
    if (len > st.len) return false;
    const size_t drop = st.len - len;
    const size_t here = pos > st.first ? pos - st.first : 0;
    if (drop <= here) {
        t = Truncation{len, pos - drop, false, 0};
        return true;
    }
    if (!st.has_prev) return false;
    const size_t before = drop - here;
    if (before > (n_ctx > st.prev_first ? n_ctx - st.prev_first : 0)) return false;
    const size_t target = n_ctx - before;  // the old context was full: its position was n_ctx
    t = Truncation{len, target, true, std::min(target, st.written)};
    return true;
}

// stream.rs:176-188.
void commit_truncate(StreamState &st, const Truncation &t, size_t n_ctx) {
    st.len = t.len;
    if (t.restore && st.has_prev) {
        st.first = st.prev_first;
        st.has_prev = false;
        st.written = n_ctx;
    }
}

}  // namespace

struct hs_batch {
    hs_model *model = nullptr;
    size_t slots = 0, max_rows = 0, rows_pad = 0;
    uint32_t overlap = 0;
    std::vector<size_t> pos;
    std::vector<uint32_t> hist;    // [slots, n_ctx]: the token at each position
    std::vector<StreamState> streams;
    std::vector<std::vector<uint32_t>> prev;  // [slot]: the full context before its last restart
    std::vector<uint64_t> host_w;  // [slots, vocab]: weights of the last step
    hipStream_t st = nullptr;
    DevMem mem;
    RowInfo *d_rows = nullptr;
    int32_t *d_x = nullptr, *d_src = nullptr;
    hs::AttnGroup *d_groups = nullptr;
    // Pinned host staging of each pass's rows, groups, output rows, queries and intervals, so
    // the copies run asynchronously on the batch stream.
    RowInfo *h_rows = nullptr;
    hs::AttnGroup *h_groups = nullptr;
    int32_t *h_src = nullptr;
    uint32_t *h_queries = nullptr;
    uint64_t *h_intervals = nullptr;
    // the mixed coder op: records, statistics and the plain intervals of a dual call
    hs::MixRec *h_mix = nullptr, *d_mix = nullptr;
    uint64_t *h_stats = nullptr, *d_stats = nullptr, *h_intervals2 = nullptr, *d_intervals2 = nullptr;
    bool inflight = false;  // a pass returned with copies or kernels still queued on `st`
    void *split = nullptr;  // scratch of the split decode attention (grown on demand)
    size_t split_bytes = 0;
    int32_t *gsplit = nullptr;  // i32 partials of the split-K decode products (grown on demand)
    size_t gsplit_elems = 0;
    int8_t *d_a = nullptr, *d_qkv = nullptr, *d_att = nullptr, *d_g = nullptr, *d_af = nullptr;
    int64_t *d_logits = nullptr;
    uint16_t *d_d16 = nullptr;
    int64_t *d_tmax = nullptr;
    uint32_t *d_queries = nullptr;
    uint64_t *d_intervals = nullptr, *d_weights = nullptr;
    size_t chunk_rows = 0;
    std::vector<int8_t *> kc, vc;  // per layer: [slots][H][n_ctx][hd]
    // Profiling (CudaBatch::profile): per-label GPU time from hipEvents around each launch.
    struct ProfEntry {
        std::string label;
        uint64_t ns = 0, launches = 0, ops = 0;
    };
    struct Pending {
        size_t entry;
        hipEvent_t e0, e1;
        uint64_t ops;
    };
    int profiling = 0;  // 1: an event pair around every launch; 2: one pair around each pass
    std::vector<ProfEntry> prof;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> event_pool;
    ~hs_batch() {
        for (auto &p : pending) {
            event_pool.push_back(p.e0);
            event_pool.push_back(p.e1);
        }
        if (span0) event_pool.push_back(span0);
        for (auto e : event_pool) (void)hipEventDestroy(e);
        if (st) (void)hipStreamSynchronize(st);
        for (void *p : {(void *)h_rows, (void *)h_groups, (void *)h_src, (void *)h_queries, (void *)h_intervals,
                        (void *)h_mix, (void *)h_stats, (void *)h_intervals2})
            if (p) (void)hipHostFree(p);
        if (split) (void)hipFree(split);
        if (gsplit) (void)hipFree(gsplit);
        if (st) (void)hipStreamDestroy(st);
    }
    hipError_t event(hipEvent_t &e) {
        if (!event_pool.empty()) {
            e = event_pool.back();
            event_pool.pop_back();
            return hipSuccess;
        }
        return hipEventCreate(&e);
    }
    size_t entry(const char *label) {
        for (size_t i = 0; i < prof.size(); i++)
            if (prof[i].label == label) return i;
        prof.push_back(ProfEntry{label});
        return prof.size() - 1;
    }
    // Runs `fn` (a launch on the batch stream), bracketed by events when profiling.
    // The op's kernels carry the events on their dispatches (hs::set_op_events): the first one
    // records e0 as it starts, each one e1 as it ends. An op that launched no kernel is timed
    // by a pair recorded around it.
    template <typename F>
    hipError_t launch(const char *label, uint64_t ops, F &&fn) {
        if (profiling != 1) return fn();
        hipEvent_t e0, e1;
        hipError_t e = event(e0);
        if (e == hipSuccess) e = event(e1);
        if (e != hipSuccess) return e;
        hs::set_op_events(e0, e1);
        e = fn();
        const int launched = hs::op_launches();
        hs::set_op_events(nullptr, nullptr);
        if (e != hipSuccess) return e;
        if (launched == 0) {
            if ((e = hipEventRecord(e0, st)) != hipSuccess) return e;
            if ((e = hipEventRecord(e1, st)) != hipSuccess) return e;
        }
        pending.push_back(Pending{entry(label), e0, e1, ops});
        return hipSuccess;
    }
    // Span profiling: an event before the pass's first copy and one after its last launch, so
    // "pass_span" sums the GPU time of the passes, gaps between kernels included.
    hipEvent_t span0 = nullptr;
    hipError_t span_begin() {
        if (profiling != 2) return hipSuccess;
        if (span0) event_pool.push_back(span0);  // a pass that failed after its first event
        hipError_t e = event(span0);
        if (e != hipSuccess) return e;
        return hipEventRecord(span0, st);
    }
    hipError_t span_end() {
        if (profiling != 2 || !span0) return hipSuccess;
        hipEvent_t e1;
        hipError_t e = event(e1);
        if (e != hipSuccess) return e;
        if ((e = hipEventRecord(e1, st)) != hipSuccess) return e;
        pending.push_back(Pending{entry("pass_span"), span0, e1, 0});
        span0 = nullptr;
        return hipSuccess;
    }
    // After a stream synchronisation: adds the event times of the finished launches.
    hipError_t collect() {
        for (auto &p : pending) {
            float ms = 0;
            hipError_t e = hipEventElapsedTime(&ms, p.e0, p.e1);
            if (e != hipSuccess) return e;
            prof[p.entry].ns += (uint64_t)((double)ms * 1e6);
            prof[p.entry].launches += 1;
            prof[p.entry].ops += p.ops;
            event_pool.push_back(p.e0);
            event_pool.push_back(p.e1);
        }
        pending.clear();
        return hipSuccess;
    }
};

extern "C" hs_status hs_batch_new(hs_model *model, size_t slots, size_t max_rows, hs_batch **out) {
    hs::clear_error();
    if (!model || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    *out = nullptr;
    if (slots == 0 || max_rows == 0)
        return hs::fail(HS_UNSUPPORTED, 0, "a batch needs at least one slot and one row");
    HIP_TRY(hipSetDevice(model->dev->ordinal));
    auto b = std::make_unique<hs_batch>();
    const hs_model &m = *model;
    b->model = model;
    b->slots = slots;
    b->max_rows = std::max<size_t>(max_rows, 2);  // a restart needs two rows
    b->rows_pad = round_up(b->max_rows, hs::GEMM_BM);
    b->pos.assign(slots, 0);
    b->hist.assign(slots * m.C, 0);
    b->streams.assign(slots, StreamState{});
    b->prev.assign(slots, {});
    // The LM head runs on chunks of output rows: compact logits (2 B per logit) up to 192 MiB a
    // chunk, so the coder op reads them back from the 256 MB Infinity Cache; i64 logits up to
    // 1 GiB.
    const size_t per_row = m.compact ? 2ull * m.ld16 : 8ull * m.V_pad;
    const size_t budget = m.compact ? (192ull << 20) : (1ull << 30);
    b->chunk_rows = std::max<size_t>(hs::GEMM_BM, round_up(std::min<size_t>(b->rows_pad, budget / per_row), hs::GEMM_BM));
    b->chunk_rows = std::min(b->chunk_rows, b->rows_pad);
    const size_t R = b->max_rows, RP = b->rows_pad;
    DevMem &mem = b->mem;
    hs_status s;
    if ((s = mem.alloc(b->d_rows, R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_src, R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_groups, R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_x, R * m.d)) != HS_OK) return s;
    // the operands of the products (d_a, d_af, d_att, d_g) are panels of RP operand rows (2 RP
    // for i16 activations: each row is two operand rows, its planes)
    if ((s = mem.alloc(b->d_a, RP * m.d_pad)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_af, (m.wide_ln_f ? 2 : 1) * RP * m.d_pad)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_qkv, R * 3 * m.d)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_att, RP * m.d_pad)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_g, (m.wide_gelu ? 2 : 1) * RP * m.f_pad)) != HS_OK) return s;
    if (m.compact) {
        if ((s = mem.alloc(b->d_d16, b->chunk_rows * m.ld16)) != HS_OK) return s;
        if ((s = mem.alloc(b->d_tmax, b->chunk_rows * m.ntiles)) != HS_OK) return s;
    } else if ((s = mem.alloc(b->d_logits, b->chunk_rows * m.V)) != HS_OK) {
        return s;
    }
    if ((s = mem.alloc(b->d_queries, 2 * R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_intervals, 3 * R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_intervals2, 3 * R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_stats, 3 * R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_mix, R)) != HS_OK) return s;
    if ((s = mem.alloc(b->d_weights, b->chunk_rows * m.V)) != HS_OK) return s;
    const size_t cache = slots * (size_t)m.C * m.d;
    b->kc.resize(m.L);
    b->vc.resize(m.L);
    for (int l = 0; l < m.L; l++) {
        if ((s = mem.alloc(b->kc[l], cache)) != HS_OK) return s;
        if ((s = mem.alloc(b->vc[l], cache)) != HS_OK) return s;
    }
    HIP_TRY(hipHostMalloc((void **)&b->h_rows, R * sizeof(RowInfo), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&b->h_groups, R * sizeof(hs::AttnGroup), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&b->h_src, R * sizeof(int32_t), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&b->h_queries, 2 * R * sizeof(uint32_t), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&b->h_intervals, 3 * R * sizeof(uint64_t), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&b->h_intervals2, 3 * R * sizeof(uint64_t), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&b->h_stats, 3 * R * sizeof(uint64_t), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void **)&b->h_mix, R * sizeof(hs::MixRec), hipHostMallocDefault));
    HIP_TRY(hipStreamCreate(&b->st));
    *out = b.release();
    return HS_OK;
}

extern "C" void hs_batch_free(hs_batch *b) { delete b; }

extern "C" hs_status hs_batch_set_overlap(hs_batch *b, uint32_t k) {
    hs::clear_error();
    if (!b) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL batch");
    const uint32_t n_ctx = b->model->host.n_ctx;
    if ((uint64_t)k + 2 > n_ctx)
        return hs::fail(HS_MODEL_ERROR, HS_MODEL_INVALID_OVERLAP,
                        "the overlap " + std::to_string(k) + " does not fit a context of " + std::to_string(n_ctx));
    b->overlap = k;
    return HS_OK;
}

extern "C" size_t hs_batch_slots(const hs_batch *b) { return b ? b->slots : 0; }
extern "C" const hs_model *hs_batch_model(const hs_batch *b) { return b ? b->model : nullptr; }
extern "C" size_t hs_batch_max_rows(const hs_batch *b) { return b ? b->max_rows : 0; }
extern "C" uint64_t hs_batch_gpu_bytes(const hs_batch *b) { return b ? b->mem.bytes : 0; }
extern "C" size_t hs_batch_position(const hs_batch *b, size_t slot) {
    return (b && slot < b->slots) ? b->pos[slot] : 0;
}
extern "C" void hs_batch_reset(hs_batch *b, size_t slot) {
    if (b && slot < b->slots) {
        b->pos[slot] = 0;
        b->streams[slot] = StreamState{};
    }
}

namespace {

// The plan of a call (batch/plan.rs:60-117): inputs -> rows -> passes of <= max_rows rows; a
// restart of a slot that already has rows in the current pass starts a new pass.
struct Plan {
    std::vector<std::vector<PassRow>> passes;  // the first n_passes hold this call's passes
    size_t n_passes = 0;
    std::vector<size_t> pos;
    std::vector<size_t> touched;  // the slots of the call, in first-use order
    std::vector<uint32_t> hist;   // their token histories after the call, n_ctx entries each
    std::vector<StreamState> streams;
    std::unordered_map<size_t, std::vector<uint32_t>> prev;
};

// Builds the plan into `p`, whose vectors keep their capacity from call to call (a fold step's
// 16k rows would otherwise touch fresh pages of host memory on every call).
void make_plan(const hs_batch &b, const hs_input *in, size_t n, Plan &p) {
    const size_t C = b.model->host.n_ctx;
    const size_t k = std::min<size_t>(b.overlap, C - 2);
    const uint32_t eot = b.model->host.eot;
    p.n_passes = 0;
    p.pos = b.pos;
    p.streams = b.streams;
    p.touched.clear();
    p.hist.clear();
    p.prev.clear();
    auto open_pass = [&]() -> std::vector<PassRow> & {
        if (p.passes.size() <= p.n_passes) p.passes.emplace_back();
        std::vector<PassRow> &v = p.passes[p.n_passes];
        v.clear();
        v.reserve(std::min(n + b.slots, b.max_rows));
        return v;
    };
    std::vector<PassRow> *cur = &open_pass();
    std::vector<char> in_pass(b.slots, 0);
    auto flush = [&]() {
        if (!cur->empty()) {
            p.n_passes++;
            cur = &open_pass();
        }
        std::fill(in_pass.begin(), in_pass.end(), 0);
    };
    auto push = [&](PassRow r) {
        if (cur->size() >= b.max_rows) flush();
        in_pass[r.slot] = 1;
        cur->push_back(r);
    };
    std::vector<int32_t> index(b.slots, -1);  // slot -> its entry in p.touched / p.hist
    p.touched.reserve(std::min(n, b.slots));
    p.hist.reserve(std::min(n, b.slots) * C);
    for (size_t i = 0; i < n; i++) {
        const size_t slot = in[i].slot;
        if (index[slot] < 0) {
            index[slot] = (int32_t)p.touched.size();
            p.touched.push_back(slot);
            p.hist.insert(p.hist.end(), b.hist.begin() + slot * C, b.hist.begin() + (slot + 1) * C);
        }
        uint32_t *h = p.hist.data() + (size_t)index[slot] * C;
        size_t at = p.pos[slot];
        if (at >= C) {
            if (in_pass[slot]) flush();
            p.prev[slot].assign(h, h + C);  // the full context before the restart, for a truncation
            p.streams[slot].restart(k);
            if (k > 0) std::memmove(&h[1], &h[C - k], k * sizeof(uint32_t));
            h[0] = eot;
            for (size_t q = 0; q <= k; q++) push(PassRow{(uint32_t)slot, h[q], (uint32_t)q, -1});
            at = k + 1;
        }
        h[at] = in[i].token;
        p.streams[slot].input(at);
        push(PassRow{(uint32_t)slot, in[i].token, (uint32_t)at, (int64_t)i});
        p.pos[slot] = at + 1;
    }
    if (!cur->empty()) p.n_passes++;
}

void commit(hs_batch &b, Plan &p) {
    const size_t C = b.model->host.n_ctx;
    b.pos = p.pos;
    b.streams = p.streams;
    for (size_t t = 0; t < p.touched.size(); t++)
        std::memcpy(&b.hist[p.touched[t] * C], p.hist.data() + t * C, C * sizeof(uint32_t));
    for (auto &kv : p.prev) b.prev[kv.first] = std::move(kv.second);
}

enum class Out { Weights, Intervals, Nothing };  // Nothing: the weights, not read back

// The tables of a mixed call (batch/mixed.rs:23-33): the table word of each input
// (HS_MIX_PLAIN, HS_MIX_NONE or the predicted token), the host mixer, and for a dual call the
// intervals of GPT-2 alone.
struct Mixing {
    const uint32_t *tables = nullptr;
    hs_mixer_fn fn = nullptr;
    void *user = nullptr;
    uint64_t *plain_sink = nullptr;
};

// mix_record (crates/hardshell-cuda/src/mixed.rs:65-90): R = max(W - w[p], 1), m = 2^16 - q,
// k = max(0, bitlen(R) + 16 - 62), w'[p] = max(1, (R q) >> k) (below 2^62).
hs_status mix_record(const hs_mix_stats &st, uint32_t p, uint32_t q, hs::MixRec &r) {
    if (q == 0 || q >= (1u << 16)) return hs::fail(HS_UNSUPPORTED, 0, "the mixer probability q must be in 1..=65535");
    if (st.predicted > st.total) return hs::fail(HS_UNSUPPORTED, 0, "the weight of the prediction is above the sum");
    const uint64_t R = std::max<uint64_t>(st.total - st.predicted, 1);
    const uint32_t bits = 64 - (uint32_t)__builtin_clzll(R);
    const uint32_t k = bits + 16 > 62 ? bits + 16 - 62 : 0;
    const unsigned __int128 v = ((unsigned __int128)R * q) >> k;
    r = hs::MixRec{p, k, (1u << 16) - q, 0, v > 1 ? (uint64_t)v : 1, 0};
    return HS_OK;
}

// One forward pass over `rows`, then the LM head and the coder op for the rows with an input.
// The mixed coder op of one LM-head chunk (batch/mixed.rs:128-188): the statistics kernel
// (launch(0)) on records that carry p only, a read back, the host mixer for each output row in
// input order and the records of rule 5, then the coder of GPT-2 alone for a dual call
// (launch(1)) and the mixed coder (launch(2)).
template <typename L>
hs_status mix_chunk(hs_batch &b, const Mixing &mx, const std::vector<int64_t> &owner, int c0, int cn, L launch) {
    hipStream_t st = b.st;
    for (int r = 0; r < cn; r++) b.h_mix[c0 + r] = hs::MixRec{mx.tables[owner[c0 + r]], 0, 0, 0, 0, 0};
    HIP_TRY(hipMemcpyAsync(b.d_mix + c0, b.h_mix + c0, cn * sizeof(hs::MixRec), hipMemcpyHostToDevice, st));
    HIP_TRY(launch(0));
    HIP_TRY(hipMemcpyAsync(b.h_stats + 3 * (size_t)c0, b.d_stats + 3 * (size_t)c0, 24 * (size_t)cn,
                           hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    for (int r = 0; r < cn; r++) {
        const uint32_t t = mx.tables[owner[c0 + r]];
        if (t == HS_MIX_PLAIN || t == HS_MIX_NONE) continue;  // the record stays {t}
        const uint64_t *w = b.h_stats + 3 * (size_t)(c0 + r);
        const hs_mix_stats stats{w[0], w[1], (uint32_t)w[2], 0};
        const uint32_t q = mx.fn(mx.user, (size_t)owner[c0 + r], &stats);
        const hs_status s = mix_record(stats, t, q, b.h_mix[c0 + r]);
        if (s != HS_OK) return s;
    }
    HIP_TRY(hipMemcpyAsync(b.d_mix + c0, b.h_mix + c0, cn * sizeof(hs::MixRec), hipMemcpyHostToDevice, st));
    if (mx.plain_sink) HIP_TRY(launch(1));
    HIP_TRY(launch(2));
    return HS_OK;
}

hs_status run_pass(hs_batch &b, const std::vector<PassRow> &rows, Out out, const uint32_t *queries,
                   uint32_t bits, uint64_t *sink, const Mixing *mx = nullptr) {
    const hs_model &m = *b.model;
    hipStream_t st = b.st;
    const int n = (int)rows.size();
    if (b.inflight) {  // the staging buffers may still feed the previous pass's copies
        HIP_TRY(hipStreamSynchronize(st));
        b.inflight = false;
    }
    RowInfo *info = b.h_rows;
    int32_t *src = b.h_src;
    uint32_t *q = b.h_queries;
    static thread_local std::vector<int64_t> owner;
    owner.clear();
    owner.reserve(n);
    int n_out = 0;
    for (int r = 0; r < n; r++) {
        info[r] = RowInfo{(int32_t)rows[r].slot, (int32_t)rows[r].token, (int32_t)rows[r].pos, -1};
        if (rows[r].input >= 0) {
            info[r].out = n_out;
            src[n_out] = r;
            owner.push_back(rows[r].input);
            if (out == Out::Intervals) {
                q[2 * n_out] = queries[2 * rows[r].input];
                q[2 * n_out + 1] = queries[2 * rows[r].input + 1];
            }
            n_out++;
        }
    }
    HIP_TRY(b.span_begin());
    HIP_TRY(hipMemcpyAsync(b.d_rows, info, n * sizeof(RowInfo), hipMemcpyHostToDevice, st));
    // Attention groups (runs of one slot at consecutive positions, at most 64 rows each) for
    // the MFMA prefill kernel; decode-shaped passes (short runs) use the row kernel.
    int n_groups = 0, group_keys = 1;  // the largest key count of a group
    for (int r = 0; r < n;) {
        int c = 1;
        while (r + c < n && c < 64 && rows[r + c].slot == rows[r].slot && rows[r + c].pos == rows[r].pos + (uint32_t)c) c++;
        b.h_groups[n_groups++] = hs::AttnGroup{r, c, (int32_t)rows[r].slot, (int32_t)rows[r].pos};
        group_keys = std::max<int>(group_keys, std::min<int>((int)rows[r].pos + c, (int)m.C));
        r += c;
    }
    const bool mfma_attn = m.hd == 64 && n >= 16 * n_groups;
    // the largest key counts first: the persistent prefill kernel pairs long and short groups
    // in its rounds (every group writes only its own rows, so the order changes no output)
    if (mfma_attn)
        std::stable_sort(b.h_groups, b.h_groups + n_groups, [](const hs::AttnGroup &x, const hs::AttnGroup &y) {
            return x.pos0 + x.count > y.pos0 + y.count;
        });
    if (mfma_attn)
        HIP_TRY(hipMemcpyAsync(b.d_groups, b.h_groups, n_groups * sizeof(hs::AttnGroup), hipMemcpyHostToDevice, st));
    if (n_out) HIP_TRY(hipMemcpyAsync(b.d_src, src, n_out * sizeof(int32_t), hipMemcpyHostToDevice, st));
    if (out == Out::Intervals && n_out)
        HIP_TRY(hipMemcpyAsync(b.d_queries, q, 2 * (size_t)n_out * sizeof(uint32_t), hipMemcpyHostToDevice, st));

    uint64_t attn_keys = 0;  // sum over rows of the keys each row reads
    for (int r = 0; r < n; r++) attn_keys += (uint64_t)rows[r].pos + 1;
    HIP_TRY(b.launch("embed", 0, [&] {
        return hs::launch_embed(b.d_rows, n, m.wte, m.V_pad, m.wpe, m.embed_m, m.host.embed_s,
                                m.pos_m, m.host.pos_s, m.d, b.d_x, st);
    }));
    const int RP = (int)b.rows_pad;  // the panel rows of the operand buffers (per plane)
    auto ln = [&](const DevLn &l, const int32_t *src_rows, int rows_n, int8_t *dst, int out_bits = 8) {
        hs::LnArgs a;
        a.bits = out_bits;
        a.x = b.d_x; a.d = m.d; a.gamma = l.g; a.beta = l.b; a.m = l.m; a.s = l.s;
        a.beta_frac = m.host.ln_beta_frac; a.k = m.host.ln_k; a.j = m.host.ln_j; a.eps = m.host.ln_eps;
        a.out = dst; a.out_rows = (out_bits == 16 ? 2 : 1) * RP;
        a.src = src_rows; a.gm = l.gm; a.beta_small = l.beta_small;
        return b.launch("layer_norm", 0, [&] { return hs::launch_layernorm(a, rows_n, st); });
    };
    // The LM head: the rows of a chunk (at most a few MB of A) stay in every XCD's L2 while
    // each XCD streams its own slice of wte once (all M-tiles in one group, N outermost).
    auto head_group = [](int rows) { return (rows + hs::GEMM_BM - 1) / hs::GEMM_BM; };
    // `a` holds panels of a_rows rows; the GELU products write panels of the same row count (RP
    // rows per plane)
    auto gemm = [&](const char *label, Epi epi, const DevLinear &lin, const int8_t *a, int a_rows, int rows_n,
                    void *o, int ldo, const int8_t *gelu = nullptr, int gelu_off = 0,
                    const int16_t *gelu16 = nullptr, int group = 0, const DevBlock *gspan = nullptr) {
        hs::GemmArgs g;
        g.group = group;
        g.a = a; g.a_rows = a_rows; g.w = lin.w; g.w_rows = lin.n_pad; g.m = rows_n; g.n = lin.n; g.k_pad = lin.k_pad;
        g.bias = lin.b; g.mult = lin.m; g.shift = lin.s; g.out = o; g.ldo = ldo;
        g.params_padded = 1;
        g.out_rows = (epi == Epi::GeluWide ? 2 : 1) * RP;
        g.fast32 = epi == Epi::ResidualWide ? 0 : lin.fast32;
        g.gelu = gelu; g.gelu16 = gelu16; g.gelu_off = gelu_off; g.wsum = lin.wsum;
        if (gspan && gspan->gelu_copy > 0) {
            g.gelu_lo = gspan->gelu_lo; g.gelu_clo = gspan->gelu_clo; g.gelu_chi = gspan->gelu_chi;
            g.gelu_shift = gspan->gelu_shift; g.gelu_copy = gspan->gelu_copy;
        }
        g.partials = b.gsplit; g.partials_cap = b.gsplit_elems;
        const uint64_t ops = 2ull * (uint64_t)rows_n * (uint64_t)lin.n * (uint64_t)lin.k;
        return b.launch(label, ops, [&] { return hs::launch_gemm(epi, g, st); });
    };
    const bool kv_fused = m.hd % 16 == 0 && m.d % 16 == 0;
    // Decode-shaped passes (at most two 256-row tiles): the layer products split K where the
    // launcher's plan says so; their partials need a scratch, grown here before any launch.
    if (n <= 2 * hs::GEMM_BM) {
        size_t need = 0;
        auto want = [&](Epi e, const DevLinear &lin) {
            const int sp = hs::gemm_split_plan(e, n, lin.n, lin.k_pad, 0);
            if (sp > 1) need = std::max(need, hs::gemm_split_elems(n, lin.n, sp));
        };
        for (const DevBlock &blk : m.blocks) {
            want(Epi::Act, blk.c_attn);
            want(Epi::Residual, blk.c_proj);
            want(blk.gelu16 ? Epi::GeluWide : Epi::Gelu, blk.c_fc);
            if (!blk.gelu16) want(Epi::Residual, blk.mlp_proj);
        }
        if (need > b.gsplit_elems) {
            if (b.gsplit) {
                HIP_TRY(hipStreamSynchronize(st));
                HIP_TRY(hipFree(b.gsplit));
                b.gsplit = nullptr;
                b.gsplit_elems = 0;
            }
            HIP_TRY(hipMalloc((void **)&b.gsplit, need * sizeof(int32_t)));
            b.gsplit_elems = need;
        }
    }
    // Decode-shaped passes (short runs): attention split over key chunks when the scratch fits
    // (at most 1 GiB), else the row kernel.
    bool split_attn = false;
    hs::SplitPlan split_plan;
    if (!mfma_attn && hs::attend_split_ok(m.hd)) {
        int max_keys = 1;
        for (int r = 0; r < n; r++) max_keys = std::max<int>(max_keys, (int)rows[r].pos + 1);
        split_plan = hs::attend_split_plan(n, m.H, max_keys);
        hs::AttnArgs probe;
        probe.n_head = m.H; probe.hd = m.hd; probe.ctx_cap = m.C;
        const size_t need = hs::attend_split_bytes(probe, n, split_plan);  // 0: one launch
        if (need <= (1ull << 30)) {
            if (need > b.split_bytes) {
                if (b.split) {
                    HIP_TRY(hipStreamSynchronize(st));
                    HIP_TRY(hipFree(b.split));
                    b.split = nullptr;
                    b.split_bytes = 0;
                }
                HIP_TRY(hipMalloc(&b.split, need));
                b.split_bytes = need;
            }
            split_attn = true;
        }
    }
    for (int l = 0; l < m.L; l++) {
        const DevBlock &blk = m.blocks[l];
        HIP_TRY(ln(blk.ln1, nullptr, n, b.d_a));
        if (kv_fused) {  // K and V go from the c_attn epilogue straight into the caches
            hs::GemmArgs g;
            g.a = b.d_a; g.a_rows = RP; g.w = blk.c_attn.w; g.w_rows = blk.c_attn.n_pad;
            g.m = n; g.n = blk.c_attn.n; g.k_pad = blk.c_attn.k_pad;
            g.bias = blk.c_attn.b; g.mult = blk.c_attn.m; g.shift = blk.c_attn.s; g.out = b.d_qkv;
            g.params_padded = 1;
            g.ldo = 3 * m.d; g.fast32 = blk.c_attn.fast32;
            g.kv_rows = b.d_rows; g.kc = b.kc[l]; g.vc = b.vc[l];
            g.kv_d = m.d; g.kv_hd = m.hd; g.kv_h = m.H; g.kv_ctx = m.C;
            g.partials = b.gsplit; g.partials_cap = b.gsplit_elems;
            const uint64_t ops = 2ull * (uint64_t)n * (uint64_t)blk.c_attn.n * (uint64_t)blk.c_attn.k;
            HIP_TRY(b.launch("gemm_qkv", ops, [&] { return hs::launch_gemm(Epi::Act, g, st); }));
        } else {
            HIP_TRY(gemm("gemm_qkv", Epi::Act, blk.c_attn, b.d_a, RP, n, b.d_qkv, 3 * m.d));
            HIP_TRY(b.launch("kv_store", 0, [&] {
                return hs::launch_kv_store(b.d_rows, n, b.d_qkv, m.d, m.H, m.hd, m.C, b.kc[l], b.vc[l], st);
            }));
        }
        hs::AttnArgs at;
        at.rows = b.d_rows; at.q = b.d_qkv; at.ldq = 3 * m.d; at.kc = b.kc[l]; at.vc = b.vc[l];
        at.n_head = m.H; at.hd = m.hd; at.ctx_cap = m.C; at.score_m = blk.score_m; at.score_s = blk.score_s;
        at.out_m = blk.out_m; at.out_s = blk.out_s; at.exp_table = m.attn_exp;
        at.exp_len = (int)m.host.attn_exp.size(); at.exp_last = m.attn_exp_last;
        at.softmax_p = m.host.softmax_p;
        at.out = b.d_att; at.out_rows = RP;
        HIP_TRY(b.launch("attention", 4ull * attn_keys * (uint64_t)m.d, [&] {
            if (mfma_attn) return hs::launch_attend_groups(at, b.d_groups, n_groups, group_keys, st);
            if (split_attn) return hs::launch_attend_split(at, n, split_plan, b.split, st);
            return hs::launch_attend(at, n, st);
        }));
        HIP_TRY(gemm("gemm_proj", Epi::Residual, blk.c_proj, b.d_att, RP, n, b.d_x, m.d));
        HIP_TRY(ln(blk.ln2, nullptr, n, b.d_a));
        if (blk.gelu16) {  // i16 GELU outputs as planes, mlp_proj over 2n operand rows
            HIP_TRY(gemm("gemm_fc", Epi::GeluWide, blk.c_fc, b.d_a, RP, n, b.d_g, 0, nullptr, blk.gelu_off,
                         blk.gelu16));
            HIP_TRY(gemm("gemm_mlp", Epi::ResidualWide, blk.mlp_proj, b.d_g, 2 * RP, 2 * n, b.d_x, m.d));
        } else {
            HIP_TRY(gemm("gemm_fc", Epi::Gelu, blk.c_fc, b.d_a, RP, n, b.d_g, 0, blk.gelu, blk.gelu_off, nullptr, 0,
                         &blk));
            HIP_TRY(gemm("gemm_mlp", Epi::Residual, blk.mlp_proj, b.d_g, RP, n, b.d_x, m.d));
        }
    }
    if (n_out == 0) {
        HIP_TRY(b.span_end());
        b.inflight = true;
        if (b.profiling && b.pending.size() > 8192) {
            HIP_TRY(hipStreamSynchronize(st));
            b.inflight = false;
            HIP_TRY(b.collect());
        }
        return HS_OK;
    }
    // a 16-bit ln_f (version 2) writes two operand rows (planes) per output row
    const int pr = m.wide_ln_f ? 2 : 1;
    HIP_TRY(ln(m.ln_f, b.d_src, n_out, b.d_af, m.wide_ln_f ? 16 : 8));
    DevLinear head;
    head.w = m.wte; head.m = m.logit_m; head.s = m.host.logit_s; head.n = m.V; head.k = m.d;
    head.n_pad = m.V_pad; head.k_pad = m.d_pad; head.wsum = m.wte_sum;
    const size_t per_row = out == Out::Intervals ? 3 : (size_t)m.V;
    std::vector<uint64_t> host(out == Out::Weights ? (size_t)n_out * per_row : 0);
    for (int c0 = 0; c0 < n_out; c0 += (int)b.chunk_rows) {
        const int cn = std::min<int>((int)b.chunk_rows, n_out - c0);
        if (m.compact) {
            hs::GemmArgs g;
            // the chunk's operand rows start at row pr c0 of the panels of pr RP rows
            g.a = b.d_af + (size_t)pr * c0 * 64; g.a_rows = pr * RP; g.w = m.wte; g.w_rows = m.V_pad;
            g.m = pr * cn; g.n = m.V; g.k_pad = m.d_pad;
            g.mult = m.logit_m; g.shift = m.host.logit_s; g.out = b.d_d16; g.ldo = m.ld16;
            g.params_padded = 1;
            g.tmax = b.d_tmax; g.tmax_ld = m.ntiles; g.cap16 = (int)m.host.logits_exp.size() - 1;
            g.wsum = m.wte_sum;
            g.group = head_group(g.m);
            const uint64_t ops = 2ull * (uint64_t)pr * cn * (uint64_t)m.V * (uint64_t)m.d;
            const Epi epi = m.wide_ln_f ? Epi::LogitsCompactWide : Epi::LogitsCompact;
            HIP_TRY(b.launch("gemm_logits", ops, [&] { return hs::launch_gemm(epi, g, st); }));
            hs::CompactCoderArgs ca;
            ca.d16 = b.d_d16; ca.ld16 = m.ld16; ca.tmax = b.d_tmax; ca.ntiles = m.ntiles; ca.vocab = m.V;
            ca.table = m.logits_exp; ca.table_len = (int)m.host.logits_exp.size(); ca.d0 = m.d0;
            ca.zcut = m.zcut;
            ca.queries = out == Out::Intervals ? b.d_queries + 2 * c0 : nullptr;
            ca.bits = (int)bits;
            ca.intervals = out == Out::Intervals ? b.d_intervals + 3 * (size_t)c0 : nullptr;
            ca.weights = out != Out::Intervals ? b.d_weights : nullptr;
            if (mx) {
                ca.mix = b.d_mix + c0;
                ca.stats = b.d_stats + 3 * (size_t)c0;
                HS_TRY(mix_chunk(b, *mx, owner, c0, cn, [&](int what) -> hipError_t {
                    if (what == 0) return b.launch("mix_stats", 0, [&] { return hs::launch_mix_stats_compact(ca, cn, st); });
                    if (what == 1) {
                        hs::CompactCoderArgs cp = ca;
                        cp.intervals = b.d_intervals2 + 3 * (size_t)c0;
                        return b.launch("coder", 0, [&] { return hs::launch_coder_compact(cp, cn, st); });
                    }
                    return b.launch("coder_mixed", 0, [&] { return hs::launch_coder_compact_mixed(ca, cn, st); });
                }));
            } else {
                HIP_TRY(b.launch("coder", 0, [&] { return hs::launch_coder_compact(ca, cn, st); }));
            }
        } else {
            HIP_TRY(gemm("gemm_logits", m.wide_ln_f ? Epi::LogitsWide : Epi::Logits, head,
                         b.d_af + (size_t)pr * c0 * 64, pr * RP, pr * cn, b.d_logits, m.V, nullptr, 0,
                         nullptr, head_group(pr * cn)));
            hs::CoderArgs ca;
            ca.logits = b.d_logits; ca.ld = m.V; ca.vocab = m.V; ca.table = m.logits_exp;
            ca.table_len = (int)m.host.logits_exp.size();
            ca.queries = out == Out::Intervals ? b.d_queries + 2 * c0 : nullptr;
            ca.bits = (int)bits;
            ca.intervals = out == Out::Intervals ? b.d_intervals + 3 * (size_t)c0 : nullptr;
            ca.weights = out != Out::Intervals ? b.d_weights : nullptr;
            if (mx) {
                ca.mix = b.d_mix + c0;
                ca.stats = b.d_stats + 3 * (size_t)c0;
                HS_TRY(mix_chunk(b, *mx, owner, c0, cn, [&](int what) -> hipError_t {
                    if (what == 0) return b.launch("mix_stats", 0, [&] { return hs::launch_mix_stats(ca, cn, st); });
                    if (what == 1) {
                        hs::CoderArgs cp = ca;
                        cp.intervals = b.d_intervals2 + 3 * (size_t)c0;
                        return b.launch("coder", 0, [&] { return hs::launch_coder(cp, cn, st); });
                    }
                    return b.launch("coder_mixed", 0, [&] { return hs::launch_coder_mixed(ca, cn, st); });
                }));
            } else {
                HIP_TRY(b.launch("coder", 0, [&] { return hs::launch_coder(ca, cn, st); }));
            }
        }
        if (out == Out::Weights)
            HIP_TRY(hipMemcpyAsync(host.data() + (size_t)c0 * m.V, b.d_weights, (size_t)cn * m.V * 8,
                                   hipMemcpyDeviceToHost, st));
    }
    HIP_TRY(b.span_end());
    if (out == Out::Intervals)
        HIP_TRY(hipMemcpyAsync(b.h_intervals, b.d_intervals, (size_t)n_out * 24, hipMemcpyDeviceToHost, st));
    if (mx && mx->plain_sink)
        HIP_TRY(hipMemcpyAsync(b.h_intervals2, b.d_intervals2, (size_t)n_out * 24, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    if (out == Out::Nothing) {  // batch.rs:549: wait for the GPU, read nothing back
        if (b.profiling && b.pending.size() > 8192) HIP_TRY(b.collect());
        return HS_OK;
    }
    const uint64_t *res = out == Out::Intervals ? b.h_intervals : host.data();
    // The event times are read back in bulk (hs_batch_profile), not inside every call.
    if (b.profiling && b.pending.size() > 8192) HIP_TRY(b.collect());
    for (int i = 0; i < n_out; i++)
        std::memcpy(sink + (size_t)owner[i] * per_row, res + (size_t)i * per_row, per_row * 8);
    if (mx && mx->plain_sink)
        for (int i = 0; i < n_out; i++)
            std::memcpy(mx->plain_sink + (size_t)owner[i] * 3, b.h_intervals2 + (size_t)i * 3, 24);
    return HS_OK;
}

hs_status check_inputs(const hs_batch *b, const hs_input *in, size_t n) {
    if (!b || (n && !in)) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    const uint32_t V = b->model->host.vocab;
    for (size_t i = 0; i < n; i++) {
        if (in[i].slot >= b->slots)
            return hs::fail(HS_BAD_SLOT, (int)in[i].slot, "slot " + std::to_string(in[i].slot) +
                            " is not valid in a batch of " + std::to_string(b->slots) + " slots");
        if (in[i].token >= V)
            return hs::fail(HS_MODEL_ERROR, HS_MODEL_TOKEN_OUT_OF_RANGE,
                            "token " + std::to_string(in[i].token) + " is not in the vocabulary of " +
                                std::to_string(V) + " tokens");
    }
    return HS_OK;
}

hs_status run(hs_batch *b, const hs_input *in, size_t n, Out out, const uint32_t *queries,
              uint32_t bits, uint64_t *sink, const Mixing *mx = nullptr) {
    HIP_TRY(hipSetDevice(b->model->dev->ordinal));
    static thread_local Plan plan;  // host scratch kept from call to call (one call per thread at a time)
    make_plan(*b, in, n, plan);
    for (size_t i = 0; i < plan.n_passes; i++) {
        hs_status s = run_pass(*b, plan.passes[i], out, queries, bits, sink, mx);
        if (s != HS_OK) return s;  // no position changes after an error
    }
    commit(*b, plan);
    return HS_OK;
}

}  // namespace

extern "C" hs_status hs_batch_run_without_readback(hs_batch *b, const hs_input *in, size_t n) {
    hs::clear_error();
    hs_status s = check_inputs(b, in, n);
    if (s != HS_OK) return s;
    return run(b, in, n, Out::Nothing, nullptr, 0, nullptr);
}

extern "C" hs_status hs_batch_run_weights(hs_batch *b, const hs_input *in, size_t n, uint64_t *out) {
    hs::clear_error();
    hs_status s = check_inputs(b, in, n);
    if (s != HS_OK) return s;
    if (n && !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "out is NULL");
    return run(b, in, n, Out::Weights, nullptr, 0, out);
}

namespace {

// coder_words (batch.rs:647-666): the query words, each checked against the vocabulary and
// the total 2^freq_bits.
hs_status coder_words(const hs_query *queries, size_t n, uint32_t V, uint32_t freq_bits,
                      std::vector<uint32_t> &words) {
    if (freq_bits == 0 || freq_bits > 32 || (uint64_t)V > (1ull << freq_bits))
        return hs::fail(HS_UNSUPPORTED, 0, "freq_bits must be in 1..=32 and 2^freq_bits >= vocab");
    words.resize(2 * n);
    for (size_t i = 0; i < n; i++) {
        const bool ok = (queries[i].kind == 0 && queries[i].value < V) ||
                        (queries[i].kind == 1 && (uint64_t)queries[i].value < (1ull << freq_bits));
        if (!ok) return hs::fail(HS_UNSUPPORTED, 0, "a coder token or target is out of range");
        words[2 * i] = queries[i].kind;
        words[2 * i + 1] = queries[i].value;
    }
    return HS_OK;
}

// table_words / prediction_words (mixed.rs:120-158): a predicted token must be in the vocabulary.
hs_status check_tables(const uint32_t *tables, size_t n, uint32_t V, bool allow_plain) {
    for (size_t i = 0; i < n; i++) {
        const uint32_t t = tables[i];
        if (t == HS_MIX_NONE || (allow_plain && t == HS_MIX_PLAIN) || t < V) continue;
        return hs::fail(HS_UNSUPPORTED, 0, "a predicted token is out of range");
    }
    return HS_OK;
}

bool needs_mixer(const uint32_t *tables, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (tables[i] != HS_MIX_NONE && tables[i] != HS_MIX_PLAIN) return true;
    return false;
}

}  // namespace

extern "C" hs_status hs_batch_run_coded(hs_batch *b, const hs_input *in, const hs_query *queries,
                                        size_t n, uint32_t freq_bits, hs_interval *out) {
    hs::clear_error();
    hs_status s = check_inputs(b, in, n);
    if (s != HS_OK) return s;
    if (n && (!queries || !out)) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    static thread_local std::vector<uint32_t> words;
    HS_TRY(coder_words(queries, n, b->model->host.vocab, freq_bits, words));
    return run(b, in, n, Out::Intervals, words.data(), freq_bits, (uint64_t *)out);
}

extern "C" hs_status hs_batch_run_coded_mixed(hs_batch *b, const hs_input *in, const hs_query *queries,
                                              const uint32_t *tables, size_t n, uint32_t freq_bits,
                                              hs_mixer_fn mixer, void *user, hs_interval *out) {
    hs::clear_error();
    HS_TRY(check_inputs(b, in, n));
    if (n && (!queries || !tables || !out)) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    const uint32_t V = b->model->host.vocab;
    std::vector<uint32_t> words;
    HS_TRY(coder_words(queries, n, V, freq_bits, words));
    HS_TRY(check_tables(tables, n, V, true));
    if (!mixer && needs_mixer(tables, n)) return hs::fail(HS_INVALID_ARGUMENT, 0, "mixer is NULL");
    Mixing mx;
    mx.tables = tables; mx.fn = mixer; mx.user = user;
    return run(b, in, n, Out::Intervals, words.data(), freq_bits, (uint64_t *)out, &mx);
}

extern "C" hs_status hs_batch_run_coded_dual(hs_batch *b, const hs_input *in, const uint32_t *tokens,
                                             const uint32_t *predictions, size_t n, uint32_t freq_bits,
                                             hs_mixer_fn mixer, void *user, hs_interval *plain,
                                             hs_interval *mixed) {
    hs::clear_error();
    HS_TRY(check_inputs(b, in, n));
    if (n && (!tokens || !predictions || !plain || !mixed)) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    const uint32_t V = b->model->host.vocab;
    std::vector<hs_query> queries(n);
    for (size_t i = 0; i < n; i++) queries[i] = hs_query{0, tokens[i]};
    std::vector<uint32_t> words;
    HS_TRY(coder_words(queries.data(), n, V, freq_bits, words));
    HS_TRY(check_tables(predictions, n, V, false));
    if (!mixer && needs_mixer(predictions, n)) return hs::fail(HS_INVALID_ARGUMENT, 0, "mixer is NULL");
    Mixing mx;
    mx.tables = predictions; mx.fn = mixer; mx.user = user; mx.plain_sink = (uint64_t *)plain;
    return run(b, in, n, Out::Intervals, words.data(), freq_bits, (uint64_t *)mixed, &mx);
}

extern "C" hs_status hs_batch_step(hs_batch *b, const hs_input *in, size_t n) {
    hs::clear_error();
    hs_status s = check_inputs(b, in, n);
    if (s != HS_OK) return s;
    std::vector<char> seen(b->slots, 0);
    for (size_t i = 0; i < n; i++) {
        if (seen[in[i].slot]) return hs::fail(HS_BAD_SLOT, (int)in[i].slot, "a slot occurs two times in one step");
        seen[in[i].slot] = 1;
    }
    const size_t V = b->model->host.vocab;
    std::vector<uint64_t> w(n * V);
    if ((s = run(b, in, n, Out::Weights, nullptr, 0, w.data())) != HS_OK) return s;
    if (b->host_w.empty()) b->host_w.assign(b->slots * V, 0);
    for (size_t i = 0; i < n; i++) std::memcpy(&b->host_w[in[i].slot * V], &w[i * V], V * 8);
    return HS_OK;
}

extern "C" hs_status hs_batch_weights(const hs_batch *b, size_t slot, uint64_t *out) {
    if (!b || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (slot >= b->slots) return hs::fail(HS_BAD_SLOT, (int)slot, "slot is not valid");
    const size_t V = b->model->host.vocab;
    if (b->host_w.empty()) std::memset(out, 0, V * 8);
    else std::memcpy(out, &b->host_w[slot * V], V * 8);
    return HS_OK;
}

// The stream of a slot (crates/hardshell-cuda/src/batch/stream.rs:15-75): the inputs since the
// last reset, the room before the next restart, and the truncation of speculative decoding.
extern "C" size_t hs_batch_stream_len(const hs_batch *b, size_t slot) {
    return (b && slot < b->slots) ? b->streams[slot].len : 0;
}
extern "C" size_t hs_batch_room(const hs_batch *b, size_t slot) {
    if (!b || slot >= b->slots) return 0;
    return StreamState::room(b->pos[slot], b->model->host.n_ctx, b->overlap);
}
extern "C" hs_status hs_batch_truncate(hs_batch *b, size_t slot, size_t len) {
    hs::clear_error();
    if (!b) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL batch");
    if (slot >= b->slots)
        return hs::fail(HS_BAD_SLOT, (int)slot, "slot " + std::to_string(slot) + " is not valid in a batch of " +
                                                     std::to_string(b->slots) + " slots");
    const size_t C = b->model->host.n_ctx;
    Truncation t;
    if (!plan_truncate(b->streams[slot], len, b->pos[slot], C, t))
        return hs::fail(HS_MODEL_ERROR, HS_MODEL_BAD_TRUNCATE,
                        "cannot truncate a stream of " + std::to_string(b->streams[slot].len) + " inputs to " +
                            std::to_string(len));
    if (t.restore) {
        // The rows of the old context that the new context wrote again, with the kept history
        // (no weights); positions the new context did not write keep their old cache entries.
        HIP_TRY(hipSetDevice(b->model->dev->ordinal));
        const std::vector<uint32_t> &prev = b->prev[slot];
        std::vector<PassRow> rows;
        for (size_t q = 0; q < t.rebuild_end && q < prev.size(); q++)
            rows.push_back(PassRow{(uint32_t)slot, prev[q], (uint32_t)q, -1});
        for (size_t r0 = 0; r0 < rows.size(); r0 += b->max_rows) {
            std::vector<PassRow> pass(rows.begin() + r0, rows.begin() + std::min(rows.size(), r0 + b->max_rows));
            hs_status s = run_pass(*b, pass, Out::Weights, nullptr, 0, nullptr);
            if (s != HS_OK) return s;
        }
        HIP_TRY(hipStreamSynchronize(b->st));
        if (prev.size() == C) std::memcpy(&b->hist[slot * C], prev.data(), C * sizeof(uint32_t));
    }
    commit_truncate(b->streams[slot], t, C);
    b->pos[slot] = t.pos;
    return HS_OK;
}

// ---------------------------------------------------------------------------------------------
// Op-level entry points: crates/hardshell-cuda/src/ops.rs:142-335
// ---------------------------------------------------------------------------------------------

extern "C" void hs_op_gemm_layout(size_t m, size_t n, size_t k, size_t *m_pad, size_t *n_pad, size_t *k_pad) {
    if (m_pad) *m_pad = round_up(std::max<size_t>(m, 1), hs::GEMM_BM);
    if (n_pad) *n_pad = round_up(std::max<size_t>(n, 1), hs::GEMM_NPAD);
    if (k_pad) *k_pad = round_up(std::max<size_t>(k, 1), hs::GEMM_BK);
}

namespace {

// `splits`: 0 lets the launcher choose the K slices (as the forward pass does), 1 runs one
// workgroup per tile over all of K, 2..16 forces that many slices.
hs_status gemm_host(hs_device *dev, Epi epi, const int8_t *w, const int8_t *a, const int32_t *bias,
                    const int32_t *mult, uint8_t shift, size_t m, size_t n, size_t k, void *out,
                    int splits = 0) {
    hs::clear_error();
    if (!dev || !w || !a || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (m == 0 || n == 0 || k == 0) return HS_OK;
    if (k > 65536) return hs::fail(HS_MODEL_ERROR, HS_MODEL_DOT_TOO_LONG, "a dot product is longer than 2^16");
    if (m > (1u << 30) || n > (1u << 30)) return hs::fail(HS_UNSUPPORTED, 0, "the product is too large");
    HIP_TRY(hipSetDevice(dev->ordinal));
    size_t mp, np, kp;
    hs_op_gemm_layout(m, n, k, &mp, &np, &kp);
    const std::vector<int8_t> wp = pack_panels(w, n, k, np, kp), ap = pack_panels(a, m, k, mp, kp);
    DevMem mem;
    int8_t *dw, *da;
    int32_t *db = nullptr, *dm = nullptr;
    void *dout;
    hs_status s;
    if ((s = mem.upload(dw, wp.data(), wp.size())) != HS_OK) return s;
    if ((s = mem.upload(da, ap.data(), ap.size())) != HS_OK) return s;
    if (bias && (s = mem.upload(db, bias, n, np)) != HS_OK) return s;
    if (mult && (s = mem.upload(dm, mult, n, np)) != HS_OK) return s;
    const size_t esz = epi == Epi::Raw ? 4 : 1;
    int8_t *o8;
    if ((s = mem.alloc(o8, m * n * esz)) != HS_OK) return s;
    dout = o8;
    hs::GemmArgs g;
    g.a = da; g.w = dw; g.m = (int)m; g.n = (int)n; g.k_pad = (int)kp;
    g.bias = db; g.mult = dm; g.shift = shift; g.out = dout; g.ldo = (int)n;
    g.params_padded = 1;
    g.fast32 = fits_i32(k, bias, bias ? n : 0);
    g.splits = splits;
    const int sp = hs::gemm_split_plan(epi, (int)m, (int)n, (int)kp, splits);
    if (sp > 1) {
        g.partials_cap = hs::gemm_split_elems((int)m, (int)n, sp);
        if ((s = mem.alloc(g.partials, g.partials_cap)) != HS_OK) return s;
    }
    HIP_TRY(hs::launch_gemm(epi, g, dev->stream));
    HIP_TRY(hipMemcpyAsync(out, dout, m * n * esz, hipMemcpyDeviceToHost, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return HS_OK;
}

}  // namespace

extern "C" hs_status hs_op_gemm_i8(hs_device *dev, const int8_t *w, const int8_t *a, size_t m, size_t n,
                                   size_t k, int32_t *out) {
    return gemm_host(dev, Epi::Raw, w, a, nullptr, nullptr, 0, m, n, k, out);
}

extern "C" hs_status hs_op_gemm_i8_split(hs_device *dev, const int8_t *w, const int8_t *a, size_t m,
                                         size_t n, size_t k, uint32_t splits, int32_t *out) {
    hs::clear_error();
    if (splits == 0 || splits > 16) return hs::fail(HS_UNSUPPORTED, 0, "splits must be in 1..=16");
    return gemm_host(dev, Epi::Raw, w, a, nullptr, nullptr, 0, m, n, k, out, (int)splits);
}

extern "C" hs_status hs_op_gemm_i8_i16(hs_device *dev, const int8_t *w, const int16_t *a, size_t m,
                                       size_t n, size_t k, uint32_t splits, int64_t *out) {
    hs::clear_error();
    if (!dev || !w || !a || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (splits == 0 || splits > 16) return hs::fail(HS_UNSUPPORTED, 0, "splits must be in 1..=16");
    if (m == 0 || n == 0 || k == 0) return HS_OK;
    if (k > 65536) return hs::fail(HS_MODEL_ERROR, HS_MODEL_DOT_TOO_LONG, "a dot product is longer than 2^16");
    if (m > (1u << 29) || n > (1u << 30)) return hs::fail(HS_UNSUPPORTED, 0, "the product is too large");
    HIP_TRY(hipSetDevice(dev->ordinal));
    // the i16 rows as two i8 plane rows (hi = v >> 8, lo = (v & 255) - 128), one i8 product of
    // 2m rows, then 256 hi + lo + 128 wsum per output
    size_t mp, np, kp;
    hs_op_gemm_layout(2 * m, n, k, &mp, &np, &kp);
    const std::vector<int8_t> wp = pack_panels(w, n, k, np, kp);
    const std::vector<int32_t> wsum = row_sums(w, n, k, n);
    std::vector<int8_t> ap(mp * kp, 0);
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < k; j++) {
            const int32_t v = a[i * k + j];
            ap[hs::panel_off(2 * i, j, mp)] = (int8_t)(v >> 8);
            ap[hs::panel_off(2 * i + 1, j, mp)] = (int8_t)((v & 255) - 128);
        }
    DevMem mem;
    int8_t *dw, *da;
    int32_t *dsum, *planes;
    int64_t *dout;
    hs_status s;
    if ((s = mem.upload(dw, wp.data(), wp.size())) != HS_OK) return s;
    if ((s = mem.upload(da, ap.data(), ap.size())) != HS_OK) return s;
    if ((s = mem.upload(dsum, wsum.data(), n)) != HS_OK) return s;
    if ((s = mem.alloc(planes, 2 * m * n)) != HS_OK) return s;
    if ((s = mem.alloc(dout, m * n)) != HS_OK) return s;
    hs::GemmArgs g;
    g.a = da; g.w = dw; g.m = (int)(2 * m); g.n = (int)n; g.k_pad = (int)kp;
    g.out = planes; g.ldo = (int)n; g.splits = (int)splits;
    const int sp = hs::gemm_split_plan(Epi::Raw, g.m, g.n, g.k_pad, g.splits);
    if (sp > 1) {
        g.partials_cap = hs::gemm_split_elems(g.m, g.n, sp);
        if ((s = mem.alloc(g.partials, g.partials_cap)) != HS_OK) return s;
    }
    HIP_TRY(hs::launch_gemm(Epi::Raw, g, dev->stream));
    HIP_TRY(hs::launch_wide_combine(planes, dsum, (int)m, (int)n, dout, dev->stream));
    HIP_TRY(hipMemcpyAsync(out, dout, m * n * sizeof(int64_t), hipMemcpyDeviceToHost, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return HS_OK;
}

extern "C" hs_status hs_op_gemm_requant_i8(hs_device *dev, const int8_t *w, const int8_t *a,
                                           const int32_t *bias, const int32_t *mult, uint8_t shift,
                                           size_t m, size_t n, size_t k, int8_t *out) {
    if (!bias || !mult) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    return gemm_host(dev, Epi::Act, w, a, bias, mult, shift, m, n, k, out);
}

extern "C" hs_status hs_op_gemm_requant_i8_dev(hs_device *dev, const int8_t *w, const int8_t *a,
                                               const int32_t *bias, const int32_t *mult, uint8_t shift,
                                               size_t m, size_t n, size_t k, int8_t *out, void *stream) {
    hs::clear_error();
    if (!dev || !w || !a || !bias || !mult || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (m == 0 || n == 0 || k == 0) return HS_OK;
    if (k > 65536) return hs::fail(HS_MODEL_ERROR, HS_MODEL_DOT_TOO_LONG, "a dot product is longer than 2^16");
    size_t kp;
    hs_op_gemm_layout(m, n, k, nullptr, nullptr, &kp);
    hs::GemmArgs g;
    g.a = a; g.w = w; g.m = (int)m; g.n = (int)n; g.k_pad = (int)kp;
    g.bias = bias; g.mult = mult; g.shift = shift; g.out = out; g.ldo = (int)n;
    hipStream_t st = stream ? (hipStream_t)stream : dev->stream;
    const int sp = hs::gemm_split_plan(Epi::Act, (int)m, (int)n, (int)kp, 0);
    if (sp > 1) {  // the split-K partials in stream-ordered memory
        g.partials_cap = hs::gemm_split_elems((int)m, (int)n, sp);
        void *p = nullptr;
        HIP_TRY(hipMallocAsync(&p, g.partials_cap * sizeof(int32_t), st));
        g.partials = (int32_t *)p;
        const hipError_t e = hs::launch_gemm(Epi::Act, g, st);
        const hipError_t f = hipFreeAsync(p, st);
        HIP_TRY(e);
        HIP_TRY(f);
        return HS_OK;
    }
    HIP_TRY(hs::launch_gemm(Epi::Act, g, st));
    return HS_OK;
}

extern "C" hs_status hs_op_attend_decode_dev(hs_device *dev, const int8_t *q, const int8_t *k_cache,
                                             const int8_t *v_cache, const uint32_t *ctx, size_t b,
                                             size_t h, size_t hd, size_t ctx_cap, int32_t score_m,
                                             uint8_t score_s, int32_t out_m, uint8_t out_s,
                                             const int32_t *attn_exp, size_t len, uint8_t softmax_p,
                                             int8_t *out, void *stream) {
    hs::clear_error();
    if (!dev || !q || !k_cache || !v_cache || !ctx || !attn_exp || !out)
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (hd == 0 || hd % 4 != 0 || hd > 256 || h == 0 || len == 0 || softmax_p > 30 || ctx_cap == 0)
        return hs::fail(HS_UNSUPPORTED, 0, "head_dim must be a multiple of 4 in 4..=256; h, len and ctx_cap >= 1; P <= 30");
    if (b == 0) return HS_OK;
    hs::AttnArgs at;
    at.rows = nullptr; at.keys = ctx; at.q = q; at.ldq = (int)(h * hd); at.kc = k_cache; at.vc = v_cache;
    at.n_head = (int)h; at.hd = (int)hd; at.ctx_cap = (int)ctx_cap; at.score_m = score_m;
    at.score_s = score_s; at.out_m = out_m; at.out_s = out_s; at.exp_table = attn_exp;
    at.exp_len = (int)len; at.softmax_p = softmax_p; at.out = out; at.ldo = (int)(h * hd);
    hipStream_t st = stream ? (hipStream_t)stream : dev->stream;
    HIP_TRY(hipSetDevice(dev->ordinal));
    if (hs::attend_split_ok((int)hd)) {  // split over key chunks, scratch ordered on the stream
        const hs::SplitPlan plan = hs::attend_split_plan((int)b, (int)h, (int)ctx_cap);
        const size_t bytes = hs::attend_split_bytes(at, (int)b, plan);
        if (bytes == 0) {  // the one-launch kernel: no scratch
            HIP_TRY(hs::launch_attend_split(at, (int)b, plan, nullptr, st));
            return HS_OK;
        }
        void *scratch = nullptr;
        HIP_TRY(hipMallocAsync(&scratch, bytes, st));
        const hipError_t e = hs::launch_attend_split(at, (int)b, plan, scratch, st);
        const hipError_t f = hipFreeAsync(scratch, st);
        HIP_TRY(e);
        HIP_TRY(f);
        return HS_OK;
    }
    HIP_TRY(hs::launch_attend(at, (int)b, st));
    return HS_OK;
}

// hs_op_attend_decode_dev without allocation: the split launches take their partials in this
// device's fixed scratch array instead of hipMallocAsync memory. Calls that overlap on one GPU
// share that array and race; every part a launch reads is written earlier in the same call, so
// nothing has to be cleared between calls.
extern "C" hs_status hs_op_attend_decode_dev_noalloc(hs_device *dev, const int8_t *q,
                                                     const int8_t *k_cache, const int8_t *v_cache,
                                                     const uint32_t *ctx, size_t b, size_t h,
                                                     size_t hd, size_t ctx_cap, int32_t score_m,
                                                     uint8_t score_s, int32_t out_m, uint8_t out_s,
                                                     const int32_t *attn_exp, size_t len,
                                                     uint8_t softmax_p, int8_t *out, void *stream) {
    hs::clear_error();
    if (!dev || !q || !k_cache || !v_cache || !ctx || !attn_exp || !out)
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (hd == 0 || hd % 4 != 0 || hd > 256 || h == 0 || len == 0 || softmax_p > 30 || ctx_cap == 0)
        return hs::fail(HS_UNSUPPORTED, 0, "head_dim must be a multiple of 4 in 4..=256; h, len and ctx_cap >= 1; P <= 30");
    if (b == 0) return HS_OK;
    if (b * h > (size_t)INT32_MAX || ctx_cap > (size_t)INT32_MAX)
        return hs::fail(HS_UNSUPPORTED, 0, "too many rows or keys");
    hs::AttnArgs at;
    at.rows = nullptr; at.keys = ctx; at.q = q; at.ldq = (int)(h * hd); at.kc = k_cache; at.vc = v_cache;
    at.n_head = (int)h; at.hd = (int)hd; at.ctx_cap = (int)ctx_cap; at.score_m = score_m;
    at.score_s = score_s; at.out_m = out_m; at.out_s = out_s; at.exp_table = attn_exp;
    at.exp_len = (int)len; at.softmax_p = softmax_p; at.out = out; at.ldo = (int)(h * hd);
    hipStream_t st = stream ? (hipStream_t)stream : dev->stream;
    if (!hs::attend_split_ok((int)hd)) {  // the row kernel uses no scratch
        HIP_TRY(hipSetDevice(dev->ordinal));
        HIP_TRY(hs::launch_attend(at, (int)b, st));
        return HS_OK;
    }
    const hs::SplitPlan plan = hs::attend_split_plan((int)b, (int)h, (int)ctx_cap);
    const size_t bytes = hs::attend_split_bytes(at, (int)b, plan);
    if (bytes > HS_FIXED_SCRATCH_BYTES)
        return hs::fail(HS_UNSUPPORTED, 0, "the split attention needs " + std::to_string(bytes) +
                                               " bytes of scratch; the fixed scratch holds " +
                                               std::to_string(HS_FIXED_SCRATCH_BYTES));
    HIP_TRY(hipSetDevice(dev->ordinal));
    HIP_TRY(hs::launch_attend_split(at, (int)b, plan, bytes ? dev->fixed_scratch : nullptr, st));
    return HS_OK;
}

// ---------------------------------------------------------------------------------------------
// Profiling, GPU timers and device memory
// ---------------------------------------------------------------------------------------------

extern "C" hs_status hs_batch_set_profiling(hs_batch *b, int on) {
    if (!b) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL batch");
    if (on) {
        // Events for the next few thousand launches, made now rather than inside timed calls.
        HIP_TRY(hipSetDevice(b->model->dev->ordinal));
        while (b->event_pool.size() < 8192) {
            hipEvent_t e;
            HIP_TRY(hipEventCreate(&e));
            b->event_pool.push_back(e);
        }
    }
    if (on < 0 || on > 2) return hs::fail(HS_INVALID_ARGUMENT, 0, "profiling mode must be 0, 1 or 2");
    b->profiling = on;
    return HS_OK;
}

extern "C" size_t hs_batch_profile(hs_batch *b, char *labels, uint64_t *ns, uint64_t *launches,
                                   uint64_t *ops, size_t cap, int clear) {
    if (!b) return 0;
    if (!b->pending.empty()) {  // every pending launch finished: each call synchronizes its stream
        if (hipStreamSynchronize(b->st) != hipSuccess || b->collect() != hipSuccess) return 0;
    }
    const size_t n = b->prof.size();
    for (size_t i = 0; i < n && i < cap; i++) {
        if (labels) {
            std::memset(labels + 32 * i, 0, 32);
            std::strncpy(labels + 32 * i, b->prof[i].label.c_str(), 31);
        }
        if (ns) ns[i] = b->prof[i].ns;
        if (launches) launches[i] = b->prof[i].launches;
        if (ops) ops[i] = b->prof[i].ops;
    }
    if (clear) b->prof.clear();
    return n;
}

namespace {

template <typename F>
hs_status time_reps(hs_device *dev, size_t reps, uint64_t *ns, F &&fn) {
    if (!ns) return hs::fail(HS_INVALID_ARGUMENT, 0, "ns is NULL");
    HIP_TRY(hipSetDevice(dev->ordinal));
    hipEvent_t e0, e1;
    HIP_TRY(hipEventCreate(&e0));
    HIP_TRY(hipEventCreate(&e1));
    hs_status s = HS_OK;
    hipError_t e = hipEventRecord(e0, dev->stream);
    for (size_t i = 0; e == hipSuccess && i < reps; i++) e = fn();
    if (e == hipSuccess) e = hipEventRecord(e1, dev->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e != hipSuccess) s = hip_fail("timed launches", e);
    *ns = (uint64_t)((double)ms * 1e6);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return s;
}

}  // namespace

extern "C" hs_status hs_op_gemm_requant_gpu_ns(hs_device *dev, const int8_t *w, const int8_t *a,
                                               const int32_t *bias, const int32_t *mult, uint8_t shift,
                                               size_t m, size_t n, size_t k, int8_t *out, size_t reps,
                                               uint64_t *ns) {
    hs::clear_error();
    if (!dev || !w || !a || !bias || !mult || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (m == 0 || n == 0 || k == 0 || k > 65536) return hs::fail(HS_UNSUPPORTED, 0, "bad GEMM shape");
    size_t kp;
    hs_op_gemm_layout(m, n, k, nullptr, nullptr, &kp);
    HIP_TRY(hipSetDevice(dev->ordinal));
    std::vector<int32_t> hb(n);  // the bias bound of the fast epilogue, as the forward pass has it
    HIP_TRY(hipMemcpy(hb.data(), bias, n * sizeof(int32_t), hipMemcpyDeviceToHost));
    hs::GemmArgs g;
    g.a = a; g.w = w; g.m = (int)m; g.n = (int)n; g.k_pad = (int)kp;
    g.bias = bias; g.mult = mult; g.shift = shift; g.out = out; g.ldo = (int)n;
    g.fast32 = fits_i32(k, hb.data(), n);
    // the split-K scratch of decode-shaped products, as the forward pass has it (outside the
    // timed launches)
    const int sp = hs::gemm_split_plan(Epi::Act, (int)m, (int)n, (int)kp, 0);
    DevMem mem;
    if (sp > 1) {
        g.partials_cap = hs::gemm_split_elems((int)m, (int)n, sp);
        hs_status s = mem.alloc(g.partials, g.partials_cap);
        if (s != HS_OK) return s;
    }
    return time_reps(dev, reps, ns, [&] { return hs::launch_gemm(Epi::Act, g, dev->stream); });
}

extern "C" hs_status hs_read_bw(hs_device *dev, size_t bytes, size_t reps, uint64_t *ns) {
    hs::clear_error();
    if (!dev || !ns) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (bytes == 0 || bytes % 16 != 0) return hs::fail(HS_UNSUPPORTED, 0, "bytes must be a positive multiple of 16");
    HIP_TRY(hipSetDevice(dev->ordinal));
    void *buf = nullptr;
    int *sink = nullptr;
    HIP_TRY(hipMalloc(&buf, bytes));
    hipError_t e = hipMalloc((void **)&sink, (size_t)hs::READ_BW_GRID * 256 * sizeof(int));
    if (e == hipSuccess) e = hipMemsetAsync(buf, 0x5A, bytes, dev->stream);  // a defined buffer
    hs_status st = e == hipSuccess ? HS_OK : hip_fail("read probe buffers", e);
    if (st == HS_OK) {  // one untimed read first (page mappings, clocks)
        e = hs::launch_read_bw(buf, bytes / 16, sink, hs::READ_BW_GRID, dev->stream);
        if (e != hipSuccess) st = hip_fail("read probe", e);
    }
    if (st == HS_OK)
        st = time_reps(dev, reps, ns, [&] { return hs::launch_read_bw(buf, bytes / 16, sink, hs::READ_BW_GRID, dev->stream); });
    (void)hipStreamSynchronize(dev->stream);
    if (sink) (void)hipFree(sink);
    (void)hipFree(buf);
    return st;
}

extern "C" hs_status hs_probe_issue(hs_device *dev, uint32_t op, uint32_t waves_per_simd, uint32_t iters,
                                    uint64_t *ns) {
    hs::clear_error();
    if (!dev || !ns) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (op > 8 || waves_per_simd < 1 || waves_per_simd > 8 || iters < 1 || iters > (1u << 20) ||
        ((op == 7 || op == 8) && waves_per_simd % 2))
        return hs::fail(HS_UNSUPPORTED, 0, "op must be 0..8, waves_per_simd 1..8 (even for the mixed ops 7 "
                                           "and 8), iters 1..2^20");
    HIP_TRY(hipSetDevice(dev->ordinal));
    int *sink = nullptr;
    HIP_TRY(hipMalloc((void **)&sink, 256 * sizeof(int)));
    hipError_t e = hs::launch_issue_probe((int)op, (int)waves_per_simd, (int)iters, sink, dev->stream);  // untimed
    hs_status st = e == hipSuccess ? HS_OK : hip_fail("issue probe", e);
    if (st == HS_OK)
        st = time_reps(dev, 1, ns, [&] { return hs::launch_issue_probe((int)op, (int)waves_per_simd, (int)iters, sink, dev->stream); });
    (void)hipStreamSynchronize(dev->stream);
    (void)hipFree(sink);
    return st;
}

extern "C" hs_status hs_op_attend_decode_gpu_ns(hs_device *dev, const int8_t *q, const int8_t *k_cache,
                                                const int8_t *v_cache, const uint32_t *ctx, size_t b,
                                                size_t h, size_t hd, size_t ctx_cap, int32_t score_m,
                                                uint8_t score_s, int32_t out_m, uint8_t out_s,
                                                const int32_t *attn_exp, size_t len, uint8_t softmax_p,
                                                int8_t *out, size_t reps, uint64_t *ns) {
    hs::clear_error();
    if (!dev || !q || !k_cache || !v_cache || !ctx || !attn_exp || !out)
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (hd == 0 || hd % 4 != 0 || hd > 256 || h == 0 || len == 0 || softmax_p > 30 || ctx_cap == 0 || b == 0)
        return hs::fail(HS_UNSUPPORTED, 0, "bad attention shape");
    hs::AttnArgs at;
    at.rows = nullptr; at.keys = ctx; at.q = q; at.ldq = (int)(h * hd); at.kc = k_cache; at.vc = v_cache;
    at.n_head = (int)h; at.hd = (int)hd; at.ctx_cap = (int)ctx_cap; at.score_m = score_m;
    at.score_s = score_s; at.out_m = out_m; at.out_s = out_s; at.exp_table = attn_exp;
    at.exp_len = (int)len; at.softmax_p = softmax_p; at.out = out; at.ldo = (int)(h * hd);
    HIP_TRY(hipSetDevice(dev->ordinal));
    if (hs::attend_split_ok((int)hd)) {
        const hs::SplitPlan plan = hs::attend_split_plan((int)b, (int)h, (int)ctx_cap);
        const size_t bytes = hs::attend_split_bytes(at, (int)b, plan);
        void *scratch = nullptr;
        if (bytes) HIP_TRY(hipMalloc(&scratch, bytes));
        const hs_status st = time_reps(dev, reps, ns, [&] {
            return hs::launch_attend_split(at, (int)b, plan, scratch, dev->stream);
        });
        if (scratch) (void)hipFree(scratch);
        return st;
    }
    return time_reps(dev, reps, ns, [&] { return hs::launch_attend(at, (int)b, dev->stream); });
}

extern "C" hs_status hs_op_attend_decode_sets_gpu_ns(
    hs_device *dev, const int8_t *q, const int8_t *const *k_caches, const int8_t *const *v_caches,
    size_t sets, const uint32_t *ctx, size_t b, size_t h, size_t hd, size_t ctx_cap, int32_t score_m,
    uint8_t score_s, int32_t out_m, uint8_t out_s, const int32_t *attn_exp, size_t len,
    uint8_t softmax_p, int8_t *out, uint64_t *ns) {
    hs::clear_error();
    if (!dev || !q || !k_caches || !v_caches || !ctx || !attn_exp || !out)
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (sets == 0) return hs::fail(HS_INVALID_ARGUMENT, 0, "no cache sets");
    for (size_t i = 0; i < sets; i++)
        if (!k_caches[i] || !v_caches[i]) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL cache");
    if (hd == 0 || hd % 4 != 0 || hd > 256 || h == 0 || len == 0 || softmax_p > 30 || ctx_cap == 0 || b == 0)
        return hs::fail(HS_UNSUPPORTED, 0, "bad attention shape");
    hs::AttnArgs at;
    at.rows = nullptr; at.keys = ctx; at.q = q; at.ldq = (int)(h * hd);
    at.n_head = (int)h; at.hd = (int)hd; at.ctx_cap = (int)ctx_cap; at.score_m = score_m;
    at.score_s = score_s; at.out_m = out_m; at.out_s = out_s; at.exp_table = attn_exp;
    at.exp_len = (int)len; at.softmax_p = softmax_p; at.out = out; at.ldo = (int)(h * hd);
    HIP_TRY(hipSetDevice(dev->ordinal));
    size_t next = 0;  // the launches take the sets in turn, one each
    auto use_next = [&] {
        at.kc = k_caches[next];
        at.vc = v_caches[next];
        next++;
    };
    if (hs::attend_split_ok((int)hd)) {
        const hs::SplitPlan plan = hs::attend_split_plan((int)b, (int)h, (int)ctx_cap);
        const size_t bytes = hs::attend_split_bytes(at, (int)b, plan);
        void *scratch = nullptr;
        if (bytes) HIP_TRY(hipMalloc(&scratch, bytes));
        const hs_status st = time_reps(dev, sets, ns, [&] {
            use_next();
            return hs::launch_attend_split(at, (int)b, plan, scratch, dev->stream);
        });
        if (scratch) (void)hipFree(scratch);
        return st;
    }
    return time_reps(dev, sets, ns, [&] {
        use_next();
        return hs::launch_attend(at, (int)b, dev->stream);
    });
}

extern "C" hs_status hs_device_alloc(hs_device *dev, size_t bytes, void **out) {
    hs::clear_error();
    if (!dev || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    *out = nullptr;
    HIP_TRY(hipSetDevice(dev->ordinal));
    HIP_TRY(hipMalloc(out, std::max<size_t>(bytes, 256)));
    HIP_TRY(hipMemset(*out, 0, std::max<size_t>(bytes, 256)));
    return HS_OK;
}

extern "C" void hs_device_free(hs_device *dev, void *ptr) {
    if (dev && ptr) {
        (void)hipSetDevice(dev->ordinal);
        (void)hipFree(ptr);
    }
}

extern "C" hs_status hs_device_upload(hs_device *dev, void *dst, const void *src, size_t bytes) {
    if (!dev || (bytes && (!dst || !src))) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return HS_OK;
}

extern "C" hs_status hs_device_download(hs_device *dev, void *dst, const void *src, size_t bytes) {
    if (!dev || (bytes && (!dst || !src))) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return HS_OK;
}

extern "C" hs_status hs_device_synchronize(hs_device *dev) {
    if (!dev) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL device");
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return HS_OK;
}

extern "C" hs_status hs_device_copy(hs_device *dev, void *dst, const void *src, size_t bytes) {
    if (!dev || (bytes && (!dst || !src))) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return HS_OK;
}

// mixed_intervals_of_weights (crates/hardshell-cuda/src/mixed.rs:160-233): the statistics
// kernel and the mixed coder kernel on given weights, with the host mixer between them.
extern "C" hs_status hs_op_mixed_coder(hs_device *dev, const uint64_t *weights, size_t rows, size_t vocab,
                                       const hs_query *queries, const uint32_t *predictions,
                                       uint32_t freq_bits, hs_mixer_fn mixer, void *user,
                                       hs_mix_stats *stats, hs_interval *out) {
    hs::clear_error();
    if (!dev || (rows && (!weights || !queries || !predictions || !out)))
        return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (rows == 0) return HS_OK;
    if (vocab == 0 || vocab > (1u << 30)) return hs::fail(HS_UNSUPPORTED, 0, "the vocabulary is too large");
    std::vector<uint32_t> q;
    HS_TRY(coder_words(queries, rows, (uint32_t)vocab, freq_bits, q));
    HS_TRY(check_tables(predictions, rows, (uint32_t)vocab, false));
    if (!mixer && needs_mixer(predictions, rows)) return hs::fail(HS_INVALID_ARGUMENT, 0, "mixer is NULL");
    for (size_t r = 0; r < rows; r++) {  // each row's sum below 2^64
        uint64_t sum = 0;
        for (size_t j = 0; j < vocab; j++)
            if (__builtin_add_overflow(sum, weights[r * vocab + j], &sum))
                return hs::fail(HS_UNSUPPORTED, 0, "a weight sum is 2^64 or more");
    }
    HIP_TRY(hipSetDevice(dev->ordinal));
    DevMem mem;
    uint64_t *dw, *dst, *di;
    uint32_t *dq;
    hs::MixRec *dm;
    std::vector<hs::MixRec> rec(rows);
    for (size_t r = 0; r < rows; r++) rec[r] = hs::MixRec{predictions[r], 0, 0, 0, 0, 0};
    HS_TRY(mem.upload(dw, weights, rows * vocab));
    HS_TRY(mem.upload(dq, q.data(), q.size()));
    HS_TRY(mem.upload(dm, rec.data(), rows));
    HS_TRY(mem.alloc(dst, 3 * rows));
    HS_TRY(mem.alloc(di, 3 * rows));
    hs::CoderArgs ca;
    ca.wsrc = dw; ca.vocab = (int)vocab; ca.queries = dq; ca.bits = (int)freq_bits; ca.intervals = di;
    ca.mix = dm; ca.stats = dst;
    HIP_TRY(hs::launch_mix_stats(ca, (int)rows, dev->stream));
    std::vector<uint64_t> sv(3 * rows);
    HIP_TRY(hipMemcpyAsync(sv.data(), dst, 24 * rows, hipMemcpyDeviceToHost, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    for (size_t r = 0; r < rows; r++) {
        const hs_mix_stats st{sv[3 * r], sv[3 * r + 1], (uint32_t)sv[3 * r + 2], 0};
        if (stats) stats[r] = st;
        if (predictions[r] == HS_MIX_NONE) continue;
        HS_TRY(mix_record(st, predictions[r], mixer(user, r, &st), rec[r]));
    }
    HIP_TRY(hipMemcpyAsync(dm, rec.data(), rows * sizeof(hs::MixRec), hipMemcpyHostToDevice, dev->stream));
    HIP_TRY(hs::launch_coder_mixed(ca, (int)rows, dev->stream));
    HIP_TRY(hipMemcpyAsync(out, di, 24 * rows, hipMemcpyDeviceToHost, dev->stream));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return HS_OK;
}

namespace {

// The coder op on given i64 logits (the compact form when the table has at most
// CODER_MAX_TABLE entries, else the i64 kernel): plain, or with `predictions` the mixer
// statistics, the host mixer and the mixed coder (the three weight sources of
// crates/hardshell-cuda/kernels/hardshell.cu:1682-1814).
hs_status coder_on_logits(hs_device *dev, const int64_t *logits, size_t rows, size_t vocab,
                          const uint64_t *table, size_t len, const hs_query *queries, uint32_t freq_bits,
                          const uint32_t *predictions, hs_mixer_fn mixer, void *user,
                          hs_mix_stats *stats, hs_interval *out) {
    if (!dev || !logits || !table || !queries || !out) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    if (rows == 0) return HS_OK;
    if (vocab == 0 || vocab > (1u << 20) || len == 0)
        return hs::fail(HS_UNSUPPORTED, 0, "vocab in 1..=2^20, len >= 1, freq_bits in 1..=32 with 2^freq_bits >= vocab");
    // The table rule of the model loader's logits table (crates/hardshell/src/logits.rs:38-49):
    // non-increasing, first entry >= 1, entries <= 2^40.
    if (table[0] < 1 || table[0] > (1ull << 40))
        return hs::fail(HS_UNSUPPORTED, 0, "the table must start in 1..=2^40");
    for (size_t i = 1; i < len; i++)
        if (table[i] > table[i - 1]) return hs::fail(HS_UNSUPPORTED, 0, "the table must be non-increasing");
    std::vector<uint32_t> q;
    HS_TRY(coder_words(queries, rows, (uint32_t)vocab, freq_bits, q));
    if (predictions) {
        HS_TRY(check_tables(predictions, rows, (uint32_t)vocab, true));
        if (!mixer && needs_mixer(predictions, rows)) return hs::fail(HS_INVALID_ARGUMENT, 0, "mixer is NULL");
    }
    HIP_TRY(hipSetDevice(dev->ordinal));
    DevMem mem;
    uint64_t *dt, *di, *dst = nullptr;
    uint32_t *dq;
    hs::MixRec *dm = nullptr;
    std::vector<hs::MixRec> rec(predictions ? rows : 0);
    for (size_t r = 0; r < rec.size(); r++) rec[r] = hs::MixRec{predictions[r], 0, 0, 0, 0, 0};
    HS_TRY(mem.upload(dt, table, len, std::max<size_t>(len, hs::CODER_TABLE_READ)));  // as the model's
    HS_TRY(mem.upload(dq, q.data(), q.size()));
    HS_TRY(mem.alloc(di, 3 * rows));
    if (predictions) {
        HS_TRY(mem.upload(dm, rec.data(), rows));
        HS_TRY(mem.alloc(dst, 3 * rows));
    }
    hipStream_t st = dev->stream;
    // launch(0): statistics, launch(1): the mixed coder, launch(2): the plain coder
    std::function<hipError_t(int)> launch;
    hs::CompactCoderArgs cca;
    hs::CoderArgs ca;
    if (len <= (size_t)hs::CODER_MAX_TABLE) {
        // the compact form the LM head writes: the max of each 64-column tile and
        // min(tilemax - l, 65535) as u16 (its narrow form; every index min(d, len - 1) follows)
        const size_t nt = (vocab + 63) / 64, ld16 = round_up(vocab, 64);
        std::vector<int64_t> tm(rows * nt, INT64_MIN);
        std::vector<uint16_t> dd(rows * ld16, 0);
        for (size_t r = 0; r < rows; r++)
            for (size_t j = 0; j < vocab; j++)
                tm[r * nt + j / 64] = std::max(tm[r * nt + j / 64], logits[r * vocab + j]);
        for (size_t r = 0; r < rows; r++)
            for (size_t j = 0; j < vocab; j++) {
                const int64_t d = tm[r * nt + j / 64] - logits[r * vocab + j];
                dd[r * ld16 + j] = (uint16_t)std::min<int64_t>(d, 65535);
            }
        uint16_t *d16;
        int64_t *dtm;
        HS_TRY(mem.upload(d16, dd.data(), dd.size()));
        HS_TRY(mem.upload(dtm, tm.data(), tm.size()));
        int d0 = 0;
        while ((size_t)d0 + 1 < len && table[d0 + 1] == table[0]) d0++;
        int zcut = (int)len;
        while (zcut > 1 && table[zcut - 1] == 0) zcut--;
        cca.d16 = d16; cca.ld16 = (int)ld16; cca.tmax = dtm; cca.ntiles = (int)nt; cca.vocab = (int)vocab;
        cca.table = dt; cca.table_len = (int)len; cca.d0 = d0; cca.zcut = zcut; cca.queries = dq;
        cca.bits = (int)freq_bits; cca.intervals = di; cca.mix = dm; cca.stats = dst;
        launch = [&](int what) {
            if (what == 0) return hs::launch_mix_stats_compact(cca, (int)rows, st);
            if (what == 1) return hs::launch_coder_compact_mixed(cca, (int)rows, st);
            return hs::launch_coder_compact(cca, (int)rows, st);
        };
    } else {
        int64_t *dl;
        HS_TRY(mem.upload(dl, logits, rows * vocab));
        ca.logits = dl; ca.ld = (int)vocab; ca.vocab = (int)vocab; ca.table = dt; ca.table_len = (int)len;
        ca.queries = dq; ca.bits = (int)freq_bits; ca.intervals = di; ca.mix = dm; ca.stats = dst;
        launch = [&](int what) {
            if (what == 0) return hs::launch_mix_stats(ca, (int)rows, st);
            if (what == 1) return hs::launch_coder_mixed(ca, (int)rows, st);
            return hs::launch_coder(ca, (int)rows, st);
        };
    }
    if (predictions) {
        HIP_TRY(launch(0));
        std::vector<uint64_t> sv(3 * rows);
        HIP_TRY(hipMemcpyAsync(sv.data(), dst, 24 * rows, hipMemcpyDeviceToHost, st));
        HIP_TRY(hipStreamSynchronize(st));
        for (size_t r = 0; r < rows; r++) {
            const hs_mix_stats s{sv[3 * r], sv[3 * r + 1], (uint32_t)sv[3 * r + 2], 0};
            if (stats) stats[r] = s;
            if (predictions[r] == HS_MIX_NONE || predictions[r] == HS_MIX_PLAIN) continue;
            HS_TRY(mix_record(s, predictions[r], mixer(user, r, &s), rec[r]));
        }
        HIP_TRY(hipMemcpyAsync(dm, rec.data(), rows * sizeof(hs::MixRec), hipMemcpyHostToDevice, st));
        HIP_TRY(launch(1));
    } else {
        HIP_TRY(launch(2));
    }
    HIP_TRY(hipMemcpyAsync(out, di, rows * 24, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    return HS_OK;
}

}  // namespace

extern "C" hs_status hs_op_coder(hs_device *dev, const int64_t *logits, size_t rows, size_t vocab,
                                 const uint64_t *table, size_t len, const hs_query *queries,
                                 uint32_t freq_bits, hs_interval *out) {
    hs::clear_error();
    return coder_on_logits(dev, logits, rows, vocab, table, len, queries, freq_bits, nullptr, nullptr,
                           nullptr, nullptr, out);
}

extern "C" hs_status hs_op_mixed_coder_logits(hs_device *dev, const int64_t *logits, size_t rows,
                                              size_t vocab, const uint64_t *table, size_t len,
                                              const hs_query *queries, const uint32_t *tables,
                                              uint32_t freq_bits, hs_mixer_fn mixer, void *user,
                                              hs_mix_stats *stats, hs_interval *out) {
    hs::clear_error();
    if (rows && !tables) return hs::fail(HS_INVALID_ARGUMENT, 0, "NULL argument");
    return coder_on_logits(dev, logits, rows, vocab, table, len, queries, freq_bits, tables, mixer, user,
                           stats, out);
}
