/*
 * hardshell_hip.h — the C ABI of the MI355X (gfx950) HardShell backend, libhardshell_hip.so.
 *
 * It replaces the public API of the reference's CUDA backend crate, crates/hardshell-cuda
 * (CudaDevice, CudaModel, CudaBatch, CudaSession and the op-level test entry points,
 * crates/hardshell-cuda/src/lib.rs:36-43), one function per method, so that a thin FFI
 * wrapper (a `hardshell-hip` crate) implements taco's `Lanes` trait
 * (crates/taco/src/lanes.rs:61-113) on it exactly as `CudaLanes` does on `CudaBatch`.
 *
 * Rules of the ABI:
 *  - Plain pointers and sizes; no C++ or torch types. All output arrays are caller-allocated
 *    with the sizes documented below.
 *  - Every function that can fail returns an hs_status. After a failure,
 *    hs_last_error_message() and hs_last_error_code() describe it (thread-local).
 *  - Handles are not thread-safe; the caller serialises calls on one device
 *    (crates/hardshell-cuda/src/device.rs:8-9: CudaDevice is not Send). The device outlives its
 *    models and a model outlives its batches; free in reverse order.
 *  - Calls are synchronous: they return after the results are in host memory
 *    (crates/hardshell-cuda/src/batch.rs:546-567).
 *  - After an error, no slot position changes (crates/hardshell-cuda/src/batch.rs:444-446).
 *  - Results are bit-identical to the CPU reference crate crates/hardshell.
 */
#ifndef HARDSHELL_HIP_H
#define HARDSHELL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HS_ABI_VERSION 1

typedef struct hs_device hs_device;
typedef struct hs_model hs_model;
typedef struct hs_batch hs_batch;

/* The error variants of crates/hardshell-cuda/src/error.rs:9-51. */
typedef enum hs_status {
    HS_OK = 0,
    HS_NO_DEVICE = 1,        /* Error::NoDevice: no HIP runtime or no device; use another backend */
    HS_DEVICE_ERROR = 2,     /* Error::Cuda: a HIP runtime call failed (code: hs_last_error_code) */
    HS_UNSUPPORTED = 3,      /* Error::Unsupported: shape, device or request not supported */
    HS_MODEL_ERROR = 4,      /* Error::Model: model file or token error (kind: hs_last_error_code) */
    HS_BAD_SLOT = 5,         /* Error::BadSlot */
    HS_LENGTH_MISMATCH = 6,  /* Error::LengthMismatch */
    HS_INVALID_ARGUMENT = 7  /* a NULL handle or pointer (no counterpart: Rust references) */
} hs_status;

/* The kind of an HS_MODEL_ERROR: the variants of crates/hardshell/src/error.rs:13-154. */
typedef enum hs_model_error {
    HS_MODEL_INVALID_SHAPE = 1,
    HS_MODEL_LENGTH_MISMATCH = 2,
    HS_MODEL_DOT_TOO_LONG = 3,
    HS_MODEL_BAD_MAGIC = 4,
    HS_MODEL_UNSUPPORTED_VERSION = 5,
    HS_MODEL_TRUNCATED = 6,
    HS_MODEL_HEADER_NOT_UTF8 = 7,
    HS_MODEL_HEADER_JSON = 8,
    HS_MODEL_INVALID_HEADER = 9,
    HS_MODEL_LAYOUT = 10,
    HS_MODEL_NON_ZERO_PADDING = 11,
    HS_MODEL_VOCABULARY = 12,
    HS_MODEL_MISSING_TENSOR = 13,
    HS_MODEL_UNEXPECTED_TENSOR = 14,
    HS_MODEL_TENSOR_MISMATCH = 15,
    HS_MODEL_TOKEN_OUT_OF_RANGE = 16,
    HS_MODEL_INVALID_OVERLAP = 17,
    HS_MODEL_BAD_TRUNCATE = 18,
    HS_MODEL_TOO_LARGE = 19,
    HS_MODEL_UNSUPPORTED = 20
} hs_model_error;

/* The message and code of the last failure on this thread ("" and 0 if none). */
const char *hs_last_error_message(void);
int hs_last_error_code(void);
/* Library version and the SHA-256 of the kernel sources it was built from
 * (crates/hardshell-cuda/src/kernels.rs:9-22 records the PTX source hash the same way). */
const char *hs_version(void);

/* ---- Device: crates/hardshell-cuda/src/device.rs:29-74 ---------------------------------- */
/* Opens HIP device `ordinal`. HS_NO_DEVICE if there is no runtime or no such device;
 * HS_UNSUPPORTED if it is not a gfx950 (MI355X-class) GPU. */
hs_status hs_device_open(int ordinal, hs_device **out);
void hs_device_close(hs_device *dev);
/* The device name ("AMD Instinct MI355X" ...), NUL-terminated, truncated to cap bytes. */
hs_status hs_device_name(const hs_device *dev, char *buf, size_t cap);
hs_status hs_device_memory(const hs_device *dev, size_t *free_bytes, size_t *total_bytes);
/* CudaDevice::kernel_resources (crates/hardshell-cuda/src/device.rs:65-74): for each of the main
 * kernels, its name (NUL-terminated in 64-byte slots of `names`), vector registers per thread,
 * private (spill) bytes per thread and static LDS bytes, as the compiler built them. Writes up
 * to cap entries; *count is the number of kernels. For measurements. */
hs_status hs_device_kernel_resources(hs_device *dev, char *names, int32_t *regs,
                                     int32_t *private_bytes, int32_t *static_lds_bytes, size_t cap,
                                     size_t *count);

/* ---- Model: crates/hardshell-cuda/src/model.rs:242-398 ---------------------------------- */
/* Loads a .hsm file with exactly the accept/reject rules of hardshell::gpt2::Model::load
 * (crates/hardshell/src/gpt2/model.rs:292-343, hsm/reader.rs:357-430) and uploads it. */
hs_status hs_model_load(hs_device *dev, const uint8_t *bytes, size_t len, hs_model **out);
/* CudaModel::load_with (crates/hardshell-cuda/src/model.rs:259-349): as hs_model_load, but when
 * `bytes` hash to the file of `loaded` (a model this library already loaded, on any device),
 * that model's parse is reused and the file's checks are not repeated; any other file (or
 * loaded == NULL) gets the full hs_model_load. The result has the hash of `bytes`. */
hs_status hs_model_load_with(hs_device *dev, const uint8_t *bytes, size_t len, const hs_model *loaded,
                             hs_model **out);
void hs_model_free(hs_model *model);
/* Model::load on the host alone (gpt2/model.rs:292-343): validates the file with the same
 * rules as hs_model_load and gives its SHA-256, without a device. HS_OK or HS_MODEL_ERROR. */
hs_status hs_model_validate(const uint8_t *bytes, size_t len, uint8_t hash[32]);
/* The SHA-256 of the model file (model.rs:353: CudaModel::hash). */
void hs_model_hash(const hs_model *model, uint8_t out[32]);
uint32_t hs_model_vocab(const hs_model *model);
uint32_t hs_model_n_ctx(const hs_model *model);
uint32_t hs_model_eot(const hs_model *model);
/* 1 if the model uses a rule of model-file version 2 (gpt2/model.rs:379-384). */
int hs_model_is_wide(const hs_model *model);
/* Vocabulary::token (crates/hardshell/src/hsm/mod.rs): the bytes of token `id`, a pointer into
 * the model's copy of its vocabulary (valid while the model lives; EOT's bytes are
 * "<|endoftext|>"). */
hs_status hs_model_token(const hs_model *model, uint32_t id, const uint8_t **bytes, size_t *len);
/* Model::merges (crates/hardshell/src/hsm/merges.rs): the BPE merges of the file in rank order,
 * as (left id, right id) pairs at *pairs (valid while the model lives); the count of merges. */
size_t hs_model_merges(const hs_model *model, const uint32_t **pairs);
uint64_t hs_model_weight_bytes(const hs_model *model);
/* KV-cache bytes of one slot: 2 * n_layer * n_ctx * d_model (model.rs:392-398). */
uint64_t hs_model_cache_bytes_per_slot(const hs_model *model);

/* ---- Batch: crates/hardshell-cuda/src/batch.rs:237-476, batch/stream.rs:19-75 ----------- */
typedef struct hs_input {   /* one (slot, token) input (batch.rs:447) */
    uint32_t slot;
    uint32_t token;
} hs_input;

typedef struct hs_query {   /* CoderQuery (batch.rs:38-43) */
    uint32_t kind;          /* 0: Encode(token = value); 1: Decode(target = value) */
    uint32_t value;
} hs_query;

typedef struct hs_interval {  /* CoderInterval (batch.rs:49-58); is_last is symbol + 1 == vocab */
    uint64_t symbol;
    uint64_t start;
    uint64_t freq;
} hs_interval;

/* CudaBatch::new: `slots` independent sessions, passes of up to `max_rows` rows (1 becomes 2). */
hs_status hs_batch_new(hs_model *model, size_t slots, size_t max_rows, hs_batch **out);
void hs_batch_free(hs_batch *batch);
/* CudaBatch::set_overlap: the context overlap K (ADR 0015); HS_MODEL_ERROR
 * (HS_MODEL_INVALID_OVERLAP) if K > n_ctx - 2. */
hs_status hs_batch_set_overlap(hs_batch *batch, uint32_t k);
size_t hs_batch_slots(const hs_batch *batch);
/* The model of the batch (CudaBatch<'m> holds &'m CudaModel). */
const hs_model *hs_batch_model(const hs_batch *batch);
size_t hs_batch_max_rows(const hs_batch *batch);
uint64_t hs_batch_gpu_bytes(const hs_batch *batch);
/* The number of tokens in the context of `slot` (0 for a slot that is not valid). */
size_t hs_batch_position(const hs_batch *batch, size_t slot);
/* Empties the context of `slot`. */
void hs_batch_reset(hs_batch *batch, size_t slot);
/* CudaBatch::run_weights: out holds n * vocab u64 values, in input order. A slot can occur many
 * times (prefill); a full context restarts with EOT and the last K tokens. */
hs_status hs_batch_run_weights(hs_batch *batch, const hs_input *inputs, size_t n, uint64_t *out);
/* CudaBatch::run_without_readback (crates/hardshell-cuda/src/batch.rs:478-484): runs the inputs
 * as hs_batch_run_weights does (positions commit the same way), waits for the GPU and reads
 * nothing back. For measurements. */
hs_status hs_batch_run_without_readback(hs_batch *batch, const hs_input *inputs, size_t n);
/* CudaBatch::run_coded: the interval of FreqTable::from_weights(weights, freq_bits) for each
 * input (queries[i] belongs to inputs[i]). 1 <= freq_bits <= 32 and 2^freq_bits >= vocab. */
hs_status hs_batch_run_coded(hs_batch *batch, const hs_input *inputs, const hs_query *queries,
                             size_t n, uint32_t freq_bits, hs_interval *out);
/* CudaBatch::step + weights: each listed slot at most once; keeps the weights of each slot. */
hs_status hs_batch_step(hs_batch *batch, const hs_input *inputs, size_t n);
/* The weights (vocab values) of the last hs_batch_step that included `slot`. */
hs_status hs_batch_weights(const hs_batch *batch, size_t slot, uint64_t *out);
/* batch/stream.rs: the tokens of the current stream of `slot`, the free positions before the
 * next restart, and truncation to `len` stream tokens (ADR 0017). */
size_t hs_batch_stream_len(const hs_batch *batch, size_t slot);
size_t hs_batch_room(const hs_batch *batch, size_t slot);
hs_status hs_batch_truncate(hs_batch *batch, size_t slot, size_t len);

/* ---- The mixed coder op of the logs profile: crates/hardshell-cuda/src/batch/mixed.rs:23-126,
 * src/mixed.rs:24-233 (ADR 0010 section 3) ---------------------------------------------------
 * The GPU gives the statistics of each row's GPT-2 weights w; the host mixer gives q; the GPU
 * codes with the weights of taco_match::Mixer::mix(w, p): w'[i] = max(1, (w[i] m) >> k) for
 * i != p and w'[p] = max(1, (R q) >> k), R = max(W - w[p], 1), m = 2^16 - q,
 * k = max(0, bitlen(R) + 16 - 62) (mixed.rs:65-90); without a prediction max(1, w[i]). */
#define HS_MIX_NONE 0xFFFFFFFFu   /* a mixed table without a prediction */
#define HS_MIX_PLAIN 0xFFFFFFFEu  /* the table of GPT-2 alone (MixInput::Plain) */
typedef struct hs_mix_stats {     /* MixStats (mixed.rs:36-49) */
    uint64_t total;               /* W = sum(w) (below 2^64: weights <= 2^40, vocab <= 2^20) */
    uint64_t predicted;           /* w[p] */
    uint32_t top;                 /* the token of the largest weight, the lowest id on a tie,
                                     0 if every weight is 0; the agreement bit is top == p */
    uint32_t pad;
} hs_mix_stats;
/* The host step (the mixer of FnMut(usize, MixStats) -> u32): called once for each input with a
 * prediction, in input order, with `input` its index; returns q in 1..=65535. */
typedef uint32_t (*hs_mixer_fn)(void *user, size_t input, const hs_mix_stats *stats);
/* CudaBatch::run_coded_mixed (batch/mixed.rs:48-93): as hs_batch_run_coded, with the table of
 * input i named by tables[i]: HS_MIX_PLAIN, HS_MIX_NONE or a predicted token (< vocab). A q
 * outside 1..=65535 or a predicted token out of range is HS_UNSUPPORTED. After an error no
 * position changed, but the mixer can have been called. */
hs_status hs_batch_run_coded_mixed(hs_batch *batch, const hs_input *inputs,
                                   const hs_query *queries, const uint32_t *tables, size_t n,
                                   uint32_t freq_bits, hs_mixer_fn mixer, void *user,
                                   hs_interval *out);
/* CudaBatch::run_coded_dual (batch/mixed.rs:95-126): for each input the interval of tokens[i]
 * in the table of GPT-2 alone (plain[i]) and in the mixed table with the prediction
 * predictions[i] (HS_MIX_NONE: none) (mixed[i]), from one forward pass. */
hs_status hs_batch_run_coded_dual(hs_batch *batch, const hs_input *inputs, const uint32_t *tokens,
                                  const uint32_t *predictions, size_t n, uint32_t freq_bits,
                                  hs_mixer_fn mixer, void *user, hs_interval *plain,
                                  hs_interval *mixed);
/* mixed_intervals_of_weights (mixed.rs:160-233), for tests: the op on given weights [rows,
 * vocab] (host; each row's sum below 2^64), predictions[r] a token or HS_MIX_NONE; `stats`
 * (may be NULL) receives each row's statistics. */
hs_status hs_op_mixed_coder(hs_device *dev, const uint64_t *weights, size_t rows, size_t vocab,
                            const hs_query *queries, const uint32_t *predictions,
                            uint32_t freq_bits, hs_mixer_fn mixer, void *user,
                            hs_mix_stats *stats, hs_interval *out);
/* The same op on given i64 logits and a logits table, as hs_op_coder (the compact form of the LM
 * head for tables of at most 16,384 entries, else i64 logits), for tests: tables[r] is
 * HS_MIX_PLAIN, HS_MIX_NONE or a predicted token (the mix_stats_* and coder_mixed_* kernels of
 * crates/hardshell-cuda/kernels/hardshell.cu:1682-1814 on their logits and d16 sources). */
hs_status hs_op_mixed_coder_logits(hs_device *dev, const int64_t *logits, size_t rows,
                                   size_t vocab, const uint64_t *table, size_t len,
                                   const hs_query *queries, const uint32_t *tables,
                                   uint32_t freq_bits, hs_mixer_fn mixer, void *user,
                                   hs_mix_stats *stats, hs_interval *out);

/* ---- Op-level entry points (crates/hardshell-cuda/src/ops.rs:142-335) --------------------- */
/* out[i * n + r] = w[r] . a[i] for w [n, k] and a [m, k] i8 (host pointers), exact i32; the same
 * values as hardshell::kernels::matvec_i8 (ops.rs:142-161 matmul_i8). */
hs_status hs_op_gemm_i8(hs_device *dev, const int8_t *w, const int8_t *a, size_t m, size_t n,
                        size_t k, int32_t *out);
/* As hs_op_gemm_i8 with the K dimension cut into `splits` slices (1..=16; a slice holds at
 * least 64 of K, so fewer slices run when K is short) whose exact i32 partial products are
 * summed on the GPU (ops.rs:163-184 matmul_i8_split). The forward pass uses the same split for
 * decode-shaped products (at most 512 rows). */
hs_status hs_op_gemm_i8_split(hs_device *dev, const int8_t *w, const int8_t *a, size_t m, size_t n,
                              size_t k, uint32_t splits, int32_t *out);
/* out[i * n + r] = w[r] . a[i] for i16 activations a [m, k] (host pointers), exact i64: the two
 * i8 planes of each row (hi = v >> 8, lo = (v & 255) - 128), one i8 product of 2m rows in
 * `splits` slices (1..=16), and 256 hi + lo + 128 sum(w[r]) per output, the result of
 * hardshell::kernels::matvec_i8_i16 (ops.rs:220-282 matmul_i8_i16). */
hs_status hs_op_gemm_i8_i16(hs_device *dev, const int8_t *w, const int16_t *a, size_t m, size_t n,
                            size_t k, uint32_t splits, int64_t *out);
/* The c_attn linear of the forward pass (gpt2/ops.rs:123-130): out[i * n + r] =
 * clamp(rescale(w[r] . a[i] + bias[r], mult[r], shift), -127, 127) as i8 (host pointers). */
hs_status hs_op_gemm_requant_i8(hs_device *dev, const int8_t *w, const int8_t *a,
                                const int32_t *bias, const int32_t *mult, uint8_t shift, size_t m,
                                size_t n, size_t k, int8_t *out);
/* The same product on device-resident operands (device pointers, `stream` a hipStream_t or
 * NULL), with w and a in the operand layout of hs_op_gemm_layout(). For measurements. */
hs_status hs_op_gemm_requant_i8_dev(hs_device *dev, const int8_t *w, const int8_t *a,
                                    const int32_t *bias, const int32_t *mult, uint8_t shift,
                                    size_t m, size_t n, size_t k, int8_t *out, void *stream);
/* The operand layout of the _dev and _gpu_ns entry points: an operand of R padded rows (w:
 * R = n_pad, a: R = m_pad) and k_pad columns is stored as k_pad / 64 panels of R rows x 64 bytes,
 * element (r, c) at byte ((c / 64) * R + r) * 64 + c % 64, zero beyond the real rows and
 * columns; out is [m, n] dense. */
void hs_op_gemm_layout(size_t m, size_t n, size_t k, size_t *m_pad, size_t *n_pad,
                       size_t *k_pad);
/* Integer decode attention, one query row per stream (batch rows of the decode path):
 * q [b, h, hd] i8; k_cache, v_cache [b, h, ctx_cap, hd] i8; ctx[b] keys per stream
 * (1 <= ctx[b] <= ctx_cap); out [b, h * hd] i8 = clamp_act_i8(rescale(sum_j p_j v_j, out_m,
 * out_s)) with p = softmax(clamp(rescale(q . k_j, score_m, score_s), +-2^40)) over the table
 * attn_exp (len entries), P = softmax_p (crates/hardshell/src/gpt2/reference.rs:254-283).
 * Device pointers; `stream` a hipStream_t or NULL. */
hs_status hs_op_attend_decode_dev(hs_device *dev, const int8_t *q, const int8_t *k_cache,
                                  const int8_t *v_cache, const uint32_t *ctx, size_t b, size_t h,
                                  size_t hd, size_t ctx_cap, int32_t score_m, uint8_t score_s,
                                  int32_t out_m, uint8_t out_s, const int32_t *attn_exp,
                                  size_t len, uint8_t softmax_p, int8_t *out, void *stream);

/* hs_op_attend_decode_dev without any allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The split launches keep their partials in a fixed
 * 64 MiB array per GPU (held until the process ends) instead of stream-ordered allocations;
 * a shape that needs more (row-heads x ctx_cap x 4 bytes plus the chunk partials) is refused
 * with HS_UNSUPPORTED. Calls that overlap on one GPU share that array and race. */
hs_status hs_op_attend_decode_dev_noalloc(hs_device *dev, const int8_t *q, const int8_t *k_cache,
                                          const int8_t *v_cache, const uint32_t *ctx, size_t b,
                                          size_t h, size_t hd, size_t ctx_cap, int32_t score_m,
                                          uint8_t score_s, int32_t out_m, uint8_t out_s,
                                          const int32_t *attn_exp, size_t len, uint8_t softmax_p,
                                          int8_t *out, void *stream);

/* The coder op alone (the logits_weights + coder_interval kernels of
 * crates/hardshell-cuda/kernels/hardshell.cu:1393-1611, no public counterpart; for tests): for
 * each of `rows` rows of i64 logits [rows, vocab] (host pointers, each within +-2^40), the
 * weights table[min(max - l, len - 1)] (crates/hardshell/src/logits.rs:62-72) and the interval
 * of FreqTable::from_weights(weights, freq_bits) for queries[r] (Encode or Decode). */
hs_status hs_op_coder(hs_device *dev, const int64_t *logits, size_t rows, size_t vocab,
                      const uint64_t *table, size_t len, const hs_query *queries,
                      uint32_t freq_bits, hs_interval *out);

/* The GPU time of `reps` launches of the requant GEMM on device operands (hipEvents on the
 * device stream), as matmul_gpu_ns (crates/hardshell-cuda/src/ops.rs:284-335). */
hs_status hs_op_gemm_requant_gpu_ns(hs_device *dev, const int8_t *w, const int8_t *a,
                                    const int32_t *bias, const int32_t *mult, uint8_t shift,
                                    size_t m, size_t n, size_t k, int8_t *out, size_t reps,
                                    uint64_t *ns);
/* The GPU time of `reps` launches of hs_op_attend_decode_dev (hipEvents on the device stream). */
hs_status hs_op_attend_decode_gpu_ns(hs_device *dev, const int8_t *q, const int8_t *k_cache,
                                     const int8_t *v_cache, const uint32_t *ctx, size_t b,
                                     size_t h, size_t hd, size_t ctx_cap, int32_t score_m,
                                     uint8_t score_s, int32_t out_m, uint8_t out_s,
                                     const int32_t *attn_exp, size_t len, uint8_t softmax_p,
                                     int8_t *out, size_t reps, uint64_t *ns);
/* The GPU time of `sets` launches of hs_op_attend_decode_dev, one on each cache set in turn
 * (k_caches[i], v_caches[i]: device caches of set i, each [b][h][ctx_cap][hd]), back to back on
 * the device stream between one hipEvent pair. No counterpart in the reference (a measurement
 * entry, as read_gpu_ns, crates/hardshell-cuda/src/ops.rs:328-335): launches over distinct
 * caches read HBM rather than the Infinity Cache, and the events' own cost is shared by all the
 * launches instead of falling on each. */
hs_status hs_op_attend_decode_sets_gpu_ns(hs_device *dev, const int8_t *q,
                                          const int8_t *const *k_caches,
                                          const int8_t *const *v_caches, size_t sets,
                                          const uint32_t *ctx, size_t b, size_t h, size_t hd,
                                          size_t ctx_cap, int32_t score_m, uint8_t score_s,
                                          int32_t out_m, uint8_t out_s, const int32_t *attn_exp,
                                          size_t len, uint8_t softmax_p, int8_t *out,
                                          uint64_t *ns);

/* The GPU time of `reps` reads of a device buffer of `bytes` bytes (a multiple of 16) by a
 * streaming kernel (hipEvents on the device stream): the HBM read bandwidth a kernel reaches,
 * as read_gpu_ns (crates/hardshell-cuda/src/ops.rs:328-335). */
hs_status hs_read_bw(hs_device *dev, size_t bytes, size_t reps, uint64_t *ns);
/* The GPU time of one launch of `iters` rounds of independent instructions of one kind on every
 * SIMD (256 x waves_per_simd workgroups of 4 waves, one wave on each SIMD of a CU): op 0 v_add_u32, 1 v_mad_i64_i32,
 * 2 v_fma_f64 (8 chains per wave), 3 v_mfma_i32_16x16x64_i8 (8 accumulators per wave), 4
 * v_mfma_i32_32x32x32_i8 (4 accumulators), 5 v_ashrrev_i64, 6 v_mul_hi_i32 (8 chains); 7 and 8
 * run workgroups of 8 waves (waves_per_simd even) in which waves 0-3 run op 3's MFMA chains and
 * waves 4-7 three times as many rounds of v_add_u32 (7) or v_mad_i64_i32 (8), which shows whether
 * one wave's VALU work issues beside another wave's MFMAs. No counterpart in the reference: it measures the issue
 * rates that bound the kernels here (clocks per instruction = ns x clock / instructions per SIMD).
 * Allocates a 1 KiB sink for the call. */
hs_status hs_probe_issue(hs_device *dev, uint32_t op, uint32_t waves_per_simd, uint32_t iters,
                         uint64_t *ns);

/* ---- Batch profiling: CudaBatch::profile (crates/hardshell-cuda/src/batch.rs:493-498) ----- */
/* With profiling on (on = 1), every kernel launch of the batch is bracketed by hipEvents on the
 * batch's stream; hs_batch_profile gives, for each op label, the summed GPU nanoseconds, the
 * launch count and the algorithmic int8 operations (2 per multiply-accumulate of the GEMMs).
 * With on = 2 only each forward pass is bracketed (one pair from before its first input copy to
 * after its last launch, label "pass_span"), so the timed calls keep their launch rhythm and the
 * span gives their GPU time with the gaps between kernels. */
hs_status hs_batch_set_profiling(hs_batch *batch, int on);
/* Writes up to cap entries (labels are NUL-terminated in 32-byte slots); returns the number of
 * labels. Clears the counters when `clear` is nonzero. The event times of the calls since the
 * last read are gathered here (the calls themselves only record the events). */
size_t hs_batch_profile(hs_batch *batch, char *labels, uint64_t *ns, uint64_t *launches,
                        uint64_t *ops, size_t cap, int clear);

/* ---- Device memory (test and measurement plumbing; the reference's device buffers,
 * crates/hardshell-cuda/src/driver.rs:229-265, are crate-private, so these have no public
 * counterpart). All copies are synchronous on the device stream. ---------------------------- */
hs_status hs_device_alloc(hs_device *dev, size_t bytes, void **out);
void hs_device_free(hs_device *dev, void *ptr);
hs_status hs_device_upload(hs_device *dev, void *dst, const void *src, size_t bytes);
hs_status hs_device_download(hs_device *dev, void *dst, const void *src, size_t bytes);
hs_status hs_device_synchronize(hs_device *dev);
/* Device-to-device copy; also the known-size copy that calibrates HBM traffic counters. */
hs_status hs_device_copy(hs_device *dev, void *dst, const void *src, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* HARDSHELL_HIP_H */
