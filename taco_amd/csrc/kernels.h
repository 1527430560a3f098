// Launch wrappers of the gfx950 kernels (kernels.hip). All pointers are device pointers; every
// launch goes on `stream`. The host checks shapes before it calls these.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace hs {

// One row of a pass: slot, token, position, and the packed output index (-1: no output).
struct RowInfo {
    int32_t slot, token, pos, out;
};

enum class Epi : int {
    Raw = 0, Act = 1, Residual = 2, Gelu = 3, Logits = 4, LogitsCompact = 5,
    // Model-file version 2 (i16 activations, crates/hardshell/src/gpt2/ops.rs:178-206,246-277).
    // An i16 activation v is stored as two i8 planes in adjacent operand rows: row 2r holds
    // hi = v >> 8, row 2r + 1 holds lo = (v & 255) - 128, so v = 256 hi + lo + 128.
    GeluWide = 6,          // c_fc + i16 GELU table (gelu16), out: the two planes of each row
    ResidualWide = 7,      // m = 2 x rows of planes; x += rescale(256 hi + lo + 128 wsum + b)
    LogitsWide = 8,        // as Logits over planes (i64 out)
    LogitsCompactWide = 9  // as LogitsCompact over planes
};

// GEMM operands are stored as panels of 64 bytes of K: an operand of R rows and K columns (a
// multiple of 64) holds element (r, k) at ((k / 64) * R + r) * 64 + k % 64, so the 16 rows x 64
// bytes of an MFMA fragment are 1 KiB of contiguous memory (full cache lines for the loads).
// panel_off gives the byte offset; R is the operand's panel row count (its padded rows).
__host__ __device__ inline size_t panel_off(size_t r, size_t k, size_t rows) {
    return ((k >> 6) * rows + r) * 64 + (k & 63);
}

struct GemmArgs {
    const int8_t *a = nullptr;  // panels [k_pad / 64][a_rows][64], rows m_pad and more
    const int8_t *w = nullptr;  // panels [k_pad / 64][w_rows][64], w_rows >= n_pad
    int a_rows = 0, w_rows = 0;  // the panel row counts (0: m_pad and n_pad)
    int m = 0, n = 0, k_pad = 0;
    const int32_t *bias = nullptr;  // [n] (Act, Residual, Gelu)
    const int32_t *mult = nullptr;  // [n]
    int params_padded = 0;          // 1: bias and mult hold round_up(n, 256) entries (zeros past n)
    int shift = 0;
    void *out = nullptr;  // Raw: i32; Act/Gelu: i8; Residual: i32 x (read-modify-write); Logits: i64
    int ldo = 0;          // elements per output row
    int out_rows = 0;     // Gelu/GeluWide: the output is an operand, in panels of out_rows rows
    const int8_t *gelu = nullptr;     // Gelu table, i8 entries
    const int16_t *gelu16 = nullptr;  // GeluWide table, i16 entries
    int gelu_off = 0;                 // half the table length (128 or 32768)
    // Gelu: the span of the i8 table the epilogue reads. Every entry below gelu_clo + gelu_off
    // equals that one and every entry above gelu_chi + gelu_off equals that one, so clamping the
    // rescaled value to [gelu_clo, gelu_chi] (inside [-gelu_off, gelu_off - 1]) changes no output;
    // entries gelu_lo .. gelu_lo + gelu_copy - 1 (gelu_lo and gelu_copy multiples of 16) hold the
    // span, and value r reads entry gelu_lo + (clamp(r) + gelu_shift), gelu_shift = gelu_off -
    // gelu_lo. gelu_copy 0: the whole table (the launcher fills the fields).
    int gelu_lo = 0, gelu_clo = 0, gelu_chi = 0, gelu_shift = 0, gelu_copy = 0;
    const int32_t *wsum = nullptr;    // the wide epilogues: sum_k w[n][k] per output column
    // LogitsCompact: out is u16 [m, ldo] = tilemax - logit capped at 65535 (NARROW) or cap16
    // (at least min(tilemax - logit, cap16) either way, all the readers need) and tmax
    // [m, tmax_ld] is the largest logit of each 64-column tile.
    int64_t *tmax = nullptr;
    int tmax_ld = 0;
    int cap16 = 0;
    int group = 0;  // M-tiles per group of the tile order (0: gemm_group(m))
    // 1 if the caller has shown |acc + bias| < 2^31 for every output (K * 2^14 + max|bias|
    // < 2^31: |a|, |w| <= 128); the epilogue then rescales with one i64 multiply-add.
    int fast32 = 0;
    // Act only: when kv_rows is set, columns kv_d .. 3 kv_d (K and V of a c_attn output) go to
    // the caches kc, vc [slot][kv_h][kv_ctx][kv_hd] at the row's slot and position instead of
    // `out` (kv_d and kv_hd multiples of 16).
    const struct RowInfo *kv_rows = nullptr;
    int8_t *kc = nullptr, *vc = nullptr;
    int kv_d = 0, kv_hd = 0, kv_h = 0, kv_ctx = 0;
    // Split-K (decode-shaped products: one or two M-tiles, few N tiles): when `partials` is set
    // and the shape gains from it, the workgroups of a tile take slices of K and write exact i32
    // partials, and an elementwise pass sums them and applies the epilogue. partials_cap is the
    // scratch size in i32 elements (gemm_split_elems of the chosen split must fit).
    int32_t *partials = nullptr;
    size_t partials_cap = 0;
    int splits = 0;  // 0: chosen by gemm_split_plan; 1: no split; 2..16: that many slices
    int kslice = 0;  // set by the launcher: bytes of K per slice (a multiple of GEMM_BK)
};


// Tile sizes of the MFMA GEMM (256 x 128 or 256 x 256 by N): a rows are padded to GEMM_BM, w rows
// to GEMM_NPAD, k to GEMM_BK.
constexpr int GEMM_BM = 256, GEMM_BK = 64, GEMM_NPAD = 256;

// The group size of the XCD-aware tile order: one band of M-tiles per XCD.
inline int gemm_group(int m) {
    const int gm = (m + GEMM_BM - 1) / GEMM_BM;
    return gm < 8 ? 1 : (gm + 7) / 8;
}

hipError_t launch_gemm(Epi epi, const GemmArgs &g, hipStream_t stream);

// Profiling: the kernels launched on this host thread until the next call record `start` (the
// first one, as it begins) and `stop` (each one, as it ends) on their dispatches; null stops
// it. op_launches counts the kernels launched since the events were set.
void set_op_events(hipEvent_t start, hipEvent_t stop);
int op_launches();

// The compiled resources of the main kernels: fills up to cap entries and returns the number of
// kernels (or minus a hipError_t).
struct KernelResource {
    const char *name;
    int regs, private_bytes, static_lds_bytes;
};
int kernel_resources(KernelResource *out, int cap);

// The split-K plan of a product: the number of K slices (1 = no split) for m rows, n columns and
// k_pad bytes of K with the given epilogue, and the i32 partial elements it needs.
int gemm_split_plan(Epi epi, int m, int n, int k_pad, int splits_wanted);
size_t gemm_split_elems(int m, int n, int splits);
// out[i][r] = 256 planes[2i][r] + planes[2i + 1][r] + 128 wsum[r] (i64), planes [2m, n] i32.
hipError_t launch_wide_combine(const int32_t *planes, const int32_t *wsum, int m, int n, int64_t *out,
                               hipStream_t stream);

hipError_t launch_embed(const RowInfo *rows, int n_rows, const int8_t *wte, int wte_rows,
                        const int8_t *wpe, const int32_t *embed_m, int embed_s,
                        const int32_t *pos_m, int pos_s, int d, int32_t *x, hipStream_t stream);

struct LnArgs {
    const int32_t *x = nullptr;  // [rows, d]
    int d = 0;
    const int16_t *gamma = nullptr;
    const int32_t *beta = nullptr;
    int32_t m = 0;
    int s = 0;
    int beta_frac = 0;
    int k = 0, j = 0;
    uint64_t eps = 1;
    int8_t *out = nullptr;  // the operand panels [d_pad / 64][out_rows][64]
    int out_rows = 0;
    const int32_t *src = nullptr;  // optional: output row i reads x row src[i]
    const int64_t *gm = nullptr;   // gamma[j] * m, exact in i64 (|gamma m| < 2^46)
    int bits = 8;                  // 16: clamp to +-32767 and write the two i8 planes of each row
                                   // (hi to out row 2i, lo to row 2i + 1), as the wide GEMMs read
    int beta_small = 0;            // every |beta[j]| <= 256 (allows the single-precision rule)
};
hipError_t launch_layernorm(const LnArgs &a, int n_rows, hipStream_t stream);

// The stream-read probe: every 16-byte word of buf[0 .. n16) read once (one xor per word folded
// into sink[grid x 256] so the loads are kept).
hipError_t launch_read_bw(const void *buf, size_t n16, int *sink, int grid, hipStream_t stream);
// op: 0 v_add_u32, 1 v_mad_i64_i32, 2 v_fma_f64 (8 chains each), 3 v_mfma_i32_16x16x64_i8 (8
// accumulators), 4 v_mfma_i32_32x32x32_i8 (4); 256 x waves_per_simd workgroups of 4 waves; sink
// holds 256 ints.
hipError_t launch_issue_probe(int op, int waves_per_simd, int iters, int *sink, hipStream_t stream);
constexpr int READ_BW_GRID = 2048;  // 8 workgroups of 256 threads per CU

// K and V of each row into the caches [L][slots][H][n_ctx][hd] (layer base pointers given).
hipError_t launch_kv_store(const RowInfo *rows, int n_rows, const int8_t *qkv, int d, int n_head,
                           int hd, int n_ctx, int8_t *kc, int8_t *vc, hipStream_t stream);

struct AttnArgs {
    const RowInfo *rows = nullptr;
    const int8_t *q = nullptr;  // row r, head h at q[r * ldq + h * hd]
    int ldq = 0;
    const int8_t *kc = nullptr, *vc = nullptr;  // [slots][H][ctx_cap][hd] (one layer)
    int n_head = 0, hd = 0, ctx_cap = 0;
    const uint32_t *keys = nullptr;  // optional: keys of row r (default rows[r].pos + 1)
    int32_t score_m = 0;
    int score_s = 0;
    int32_t out_m = 0;
    int out_s = 0;
    const int32_t *exp_table = nullptr;
    int exp_len = 0;
    // > 0: every entry from exp_last on is 0, so table[min(d, exp_last)] = table[min(d, exp_len - 1)]
    // (the short prefill kernel copies and indexes table[0 .. exp_last] only); 0: not known
    int exp_last = 0;
    int softmax_p = 0;
    int8_t *out = nullptr;  // row r, head h at out[r * ldo + h * hd] (out_rows 0)
    int ldo = 0;
    int out_rows = 0;  // > 0: out is an operand in panels of out_rows rows (panel_off)
};
hipError_t launch_attend(const AttnArgs &a, int n_rows, hipStream_t stream);

// Decode attention (head_dim 16, 32, 64, 128 or 256). head_dim 64 with at most 1,024 keys: one
// launch, a workgroup per (row, head), `scratch` unused. Otherwise split over key chunks: four
// launches over (row, head, chunk) with exact integer partials in `scratch` (attend_split_bytes
// bytes, 256-byte aligned). The plan's `max_keys` bounds every row's key count.
struct SplitPlan {
    int chunks = 1, chunk_keys = 64;
    int max_keys = 0;  // the bound on every row's key count the plan was made for
};
inline bool attend_split_ok(int hd) { return hd >= 16 && hd <= 256 && (hd & (hd - 1)) == 0; }
SplitPlan attend_split_plan(int n_rows, int n_head, int max_keys);
// True when the plan takes the one-launch kernel (head_dim 64, at most 1,024 keys): no scratch.
bool attend_split_one_launch(int hd, int ctx_cap, const SplitPlan &p);
// The scratch bytes of the split launches (0 when the plan takes the one-launch kernel).
size_t attend_split_bytes(const AttnArgs &a, int n_rows, const SplitPlan &p);
hipError_t launch_attend_split(const AttnArgs &a, int n_rows, const SplitPlan &p, void *scratch,
                               hipStream_t stream);

// Prefill attention on MFMA for head_dim 64: a group is up to 64 consecutive rows of one slot
// at consecutive positions (rows first .. first + count - 1 at positions pos0 ..).
struct AttnGroup {
    int32_t first, count, slot, pos0;
};
// max_keys bounds every group's key count (pos0 + count, at most ctx_cap); at most 256 keys take a
// kernel without the recompute path of longer contexts, which reads exp_table in whole 1 KiB
// chunks: the table must be readable (device memory) up to a multiple of 256 entries.
// out + row ldo + head 64 must be 4-byte aligned.
hipError_t launch_attend_groups(const AttnArgs &a, const AttnGroup *groups, int n_groups, int max_keys,
                                hipStream_t stream);

// The mix record of a row for the mixed coder op of the logs profile (8 u32 words, the layout of
// crates/hardshell-cuda/src/mixed.rs:54-90): the predicted token p (MIX_NONE: no prediction,
// weights max(1, w); MIX_PLAIN: the weights of GPT-2 alone), k and m of rule 5 (w'[i] = max(1,
// (w[i] m) >> k) for i != p) and w'[p].
constexpr uint32_t MIX_NONE = 0xFFFFFFFFu, MIX_PLAIN = 0xFFFFFFFEu;
struct MixRec {
    uint32_t p, k, m, pad0;
    uint64_t wp, pad1;
};

struct CoderArgs {
    const int64_t *logits = nullptr;  // [rows, ld]
    const uint64_t *wsrc = nullptr;   // instead of logits + table: the weights [rows, vocab]
    int ld = 0;
    int vocab = 0;
    const uint64_t *table = nullptr;  // logits_exp
    int table_len = 0;
    const uint32_t *queries = nullptr;  // [rows][2]: kind, value
    int bits = 32;
    uint64_t *intervals = nullptr;  // [rows][3]
    uint64_t *weights = nullptr;    // optional [rows, vocab]: the weights themselves
    const MixRec *mix = nullptr;    // launch_mix_stats: p of each row; launch_coder_mixed: records
    uint64_t *stats = nullptr;      // launch_mix_stats: [rows][3] = sum w, w[p], top
};
hipError_t launch_coder(const CoderArgs &a, int n_rows, hipStream_t stream);
// The statistics of pass 1 of taco_match::Mixer::mix (crates/taco-match/src/mixer.rs:278-288)
// of each row's GPT-2 weights, and the coder op on the mixed weights of each row's record.
hipError_t launch_mix_stats(const CoderArgs &a, int n_rows, hipStream_t stream);
hipError_t launch_coder_mixed(const CoderArgs &a, int n_rows, hipStream_t stream);

// The coder op over compact logits (the LogitsCompact GEMM epilogue): d16 [rows, ld16] u16 and
// tmax [rows, ntiles] i64, with a non-increasing table of table_len <= CODER_MAX_TABLE entries.
constexpr int CODER_MAX_TABLE = 16384;
// The table buffer of the compact coder holds at least this many entries (zeros past table_len).
constexpr int CODER_TABLE_READ = 8192;
struct CompactCoderArgs {
    const uint16_t *d16 = nullptr;
    int ld16 = 0;
    const int64_t *tmax = nullptr;
    int ntiles = 0;
    int vocab = 0;
    const uint64_t *table = nullptr;  // max(table_len, CODER_TABLE_READ) entries readable
    int table_len = 0;
    int d0 = 0;    // the largest d with table[d] == table[0]
    int zcut = 0;  // every table[d] with d >= zcut is 0 (1 <= zcut <= table_len)
    const uint32_t *queries = nullptr;
    int bits = 32;
    uint64_t *intervals = nullptr;
    uint64_t *weights = nullptr;
    const MixRec *mix = nullptr;  // as CoderArgs
    uint64_t *stats = nullptr;
};
hipError_t launch_coder_compact(const CompactCoderArgs &a, int n_rows, hipStream_t stream);
hipError_t launch_mix_stats_compact(const CompactCoderArgs &a, int n_rows, hipStream_t stream);
hipError_t launch_coder_compact_mixed(const CompactCoderArgs &a, int n_rows, hipStream_t stream);

}  // namespace hs
