/*
 * The oracle: a CPU restatement of the reference HardShell engine (crates/hardshell), its
 * frequency tables and range coder (crates/taco-coder), the block payload
 * (crates/taco/src/codec.rs, payload.rs) and the seeded test builder
 * (crates/hardshell/tests/common).
 *
 * TEST INFRASTRUCTURE ONLY. It is the checker that the GPU path is compared with. Only the
 * tests, the smoke check and the CPU-baseline leg of the benchmark load it. The product
 * library (taco_amd/libhardshell_hip.so) never links, loads or calls it.
 *
 * Every function is pinned by a golden vector or a closed-form check in tests/:
 *   - integer rules: the unit vectors of crates/hardshell/src/int.rs:299-363 and exact
 *     big-integer arithmetic in Python;
 *   - builder + reference session: GOLDEN_MODEL / GOLDEN_OUTPUT (tests/gpt2.rs:203-226), the
 *     overlap hash (tests/context.rs:321-353) and the version 2 hashes (tests/wide.rs:259-277);
 *   - frequency tables + coder: TABLE_A_SHA256 / STREAM_SHA256 (taco-coder tests/golden.rs)
 *     and the unit vectors of taco-coder/src/freq.rs;
 *   - payload + container: the coded conformance/v2 vectors (decoded and re-encoded);
 *   - fast engine (the timed CPU baseline): equal to the reference session on every step.
 */
#ifndef HS_ORACLE_H
#define HS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- integer rules (crates/hardshell/src/int.rs) ---- */
/* rescale(x, m, s) as an i128, returned as (hi, lo) words. */
void or_rescale(int64_t x, int32_t m, uint8_t s, int64_t *hi, uint64_t *lo);
/* rescale_wide(x, m, s) with x = (xhi, xlo). */
void or_rescale_wide(int64_t xhi, uint64_t xlo, int32_t m, uint8_t s, int64_t *hi, uint64_t *lo);
int64_t or_rescale_clamp(int64_t x, int32_t m, uint8_t s, int64_t lo, int64_t hi);
int64_t or_floor_div(int64_t a, int64_t b);
/* isqrt_u128 of (xhi, xlo); the root fits in 64 bits. */
uint64_t or_isqrt_u128(uint64_t xhi, uint64_t xlo);
/* LayerNorm of one row: crates/hardshell/src/layernorm.rs:201-256. out is i8 (bits 8) or i16. */
int or_layernorm(const int32_t *x, size_t n, const int16_t *gamma, const int32_t *beta, int32_t m,
                 uint8_t s, uint8_t beta_frac, uint8_t k, uint8_t j, uint64_t eps, int bits,
                 void *out);
/* Integer softmax of one row: crates/hardshell/src/softmax.rs:78-104. */
int or_softmax(const int64_t *scores, size_t n, const int32_t *table, size_t len, uint8_t p,
               int64_t *out);
/* logits -> weights: crates/hardshell/src/logits.rs:62-72. */
int or_logits_to_weights(const int64_t *logits, size_t n, const uint64_t *table, size_t len,
                         uint64_t *out);

/* ---- model ---- */
typedef struct or_model or_model;
/* Loads a .hsm file (a well-formed file; the strict accept/reject rules live in the product
 * loader and are tested there). Returns NULL on a parse error. */
or_model *or_model_load(const uint8_t *bytes, size_t len);
void or_model_free(or_model *m);
/* dims[0..8] = n_layer, n_head, d_model, d_ff, vocab, n_ctx, eot, is_wide */
void or_model_dims(const or_model *m, uint32_t *dims);

/* ---- reference session (crates/hardshell/src/gpt2/reference.rs) ---- */
typedef struct or_session or_session;
or_session *or_session_new(const or_model *m, uint32_t overlap);
void or_session_free(or_session *s);
/* Weights (vocab values) of start_block / step. Returns 0, or -1 on a bad token/overlap. */
int or_session_start_block(or_session *s, uint64_t *weights);
int or_session_step(or_session *s, uint32_t token, uint64_t *weights);
uint32_t or_session_position(const or_session *s);
/* Intermediate tensors of the last forward row, for op-level parity tests. */
int or_session_probe(or_session *s, uint32_t token, int32_t *x_after_embed, int8_t *ln1_out,
                     int8_t *qkv_out, int8_t *att_out, int32_t *x_after_block0);

/* ---- fast engine: the timed CPU baseline (batched rows, AVX2 products, chunked prefill) ---- */
/* All rows of one window: EOT, tokens[0..n-1); the weights of row i code tokens[i]. Writes the
 * (symbol, start, freq) of tokens[i] in the table of from_weights(weights_i, 32). */
int or_fast_window_intervals(const or_model *m, const uint32_t *tokens, size_t n, size_t chunk,
                             uint64_t *intervals);
/* Weights of every row of one window (n rows, n * vocab values), fast path. */
int or_fast_window_weights(const or_model *m, const uint32_t *tokens, size_t n, size_t chunk,
                           uint64_t *weights);
/* The fold of `count` windows of `n` tokens each (tokens[w*n .. (w+1)*n)) with `threads`
 * threads; windows are dealt w, w+threads, ... . Writes the payload of each window into
 * out (window w at w*cap, its length in lens[w]). */
int or_fold_payloads(const or_model *m, const uint32_t *tokens, size_t count, size_t n,
                     size_t chunk, int threads, uint8_t *out, size_t cap, size_t *lens);
/* dot-product kernel check: out[r*rows + o] = w[o] . x[r] (AVX2 path). */
void or_matmul_i8(const int8_t *w, size_t rows, const int8_t *x, size_t n, size_t cols,
                  int32_t *out);

/* ---- coder (crates/taco-coder) ---- */
/* FreqTable::from_weights: writes the frequencies; returns 0 or a negative error. */
int or_freq_from_weights(const uint64_t *w, size_t n, uint32_t bits, uint64_t *freqs);
/* Interval of `symbol` in from_weights(w, bits): (start, freq). */
int or_freq_interval(const uint64_t *w, size_t n, uint32_t bits, uint32_t symbol, uint64_t *start,
                     uint64_t *freq);
/* Symbol whose interval holds target, in from_weights(w, bits). */
int or_freq_find(const uint64_t *w, size_t n, uint32_t bits, uint64_t target, uint32_t *symbol,
                 uint64_t *start, uint64_t *freq);
/* A scripted encoder run: ops[i] = kind (0 symbol with explicit interval, 1 bit), a, b, c.
 * kind 0: start=a, freq=b, bits=c. kind 1: p1=a, bit=b. Returns the output length. */
size_t or_encode_script(const uint64_t *ops, size_t nops, uint8_t *out, size_t cap);
/* The matching decoder: kind 0 entries give start/freq tables through (a, b, c) = (table id,
 * unused, bits); tables are passed as concatenated freqs. Used for the golden stream. */
typedef struct or_decoder or_decoder;
or_decoder *or_decoder_new(const uint8_t *bytes, size_t len);
void or_decoder_free(or_decoder *d);
uint64_t or_decoder_target(const or_decoder *d, uint32_t bits);
int or_decoder_decode_interval(or_decoder *d, uint64_t start, uint64_t freq, uint32_t bits);
int or_decoder_decode_bit(or_decoder *d, uint32_t p1);

/* ---- block payload (crates/taco/src/codec.rs) with the reference session ---- */
/* encode_block with the reference session and overlap K; stop = SIZE_MAX for no stop. Writes
 * the payload; returns its length, or (size_t)-1 if the encoder stopped (no payload). */
size_t or_encode_block(const or_model *m, uint32_t overlap, const uint32_t *tokens, size_t n,
                       size_t stop, uint8_t *out, size_t cap);
/* Decodes one coded payload: writes up to cap tokens; returns the token count or -1. */
long or_decode_block(const or_model *m, uint32_t overlap, const uint8_t *payload, size_t len,
                     uint32_t *tokens, size_t cap);

/* ---- seeded test builder (crates/hardshell/tests/common/builder.rs) ---- */
/* Writes the .hsm bytes of build(dims, seed, calib_len) (wide = build_wide) into out (if
 * cap is large enough); returns the length. dims = n_layer, n_head, d_model, d_ff, vocab,
 * n_ctx. */
size_t or_build_model(const uint32_t *dims, uint64_t seed, size_t calib_len, int wide,
                      uint8_t *out, size_t cap);

/* ---- op-level references for the GPU op tests ---- */
void or_linear_act_ref(const int8_t *w, const int8_t *a, const int32_t *bias, const int32_t *mult,
                       uint8_t s, size_t m, size_t n, size_t k, int8_t *out);
void or_attend_decode_ref(const int8_t *q, const int8_t *kc, const int8_t *vc, const uint32_t *ctx,
                          size_t b, size_t h, size_t hd, size_t ctx_cap, int32_t score_m,
                          uint8_t score_s, int32_t out_m, uint8_t out_s, const int32_t *table,
                          size_t len, uint8_t p, int8_t *out);

#ifdef __cplusplus
}
#endif
#endif
