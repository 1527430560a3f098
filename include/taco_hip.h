/*
 * taco_hip.h — the host harness above the HardShell C ABI (libtaco_hip.so). It plays the role of
 * the reference's `taco` crate on this path: it cuts blocks into context windows, drives a
 * batch of slots through hs_batch_run_coded (the `Lanes::coded` call of
 * crates/taco/src/lanes.rs:77 on CudaLanes), feeds the intervals to the host range coder,
 * writes the block payloads and builds the .taco container. Unfold decodes coded blocks with
 * Decode queries, one row per slot per call, as crates/taco/src/gpu_unfold.rs:143-160.
 *
 * The bytes are those of crates/taco/src/codec.rs (encode_block), crates/taco-coder (the
 * range coder) and crates/taco-format/src/writer.rs:245-288 (Container::build).
 *
 * Calls on different batches may run on different host threads at once (each batch has its own
 * stream; the range coders' worker pool takes their jobs one after another). One batch serves
 * one call at a time.
 */
#ifndef TACO_HIP_H
#define TACO_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "hardshell_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The number of bits of every frequency table total: T = 2^32 (crates/taco/src/codec.rs:35). */
#define TC_FREQ_BITS 32

/* Codes `count` blocks of tokens (block b is tokens[offsets[b] .. offsets[b + 1])) with the
 * context overlap `overlap` on `batch` (its slots run windows in waves; its overlap must equal
 * `overlap`). Writes the payload of block b (LEB128 count, then the range coder bytes) at
 * out + b * cap and its length in lens[b]; lens[b] = SIZE_MAX if the payload is not smaller
 * than stop[b] bytes (the encoder's stop rule, crates/taco/src/codec.rs:105-112; stop may be
 * NULL for no stop). The windows follow crates/taco/src/gpu_fold.rs:128-186. */
hs_status tc_fold_blocks(hs_batch *batch, uint32_t overlap, const uint32_t *tokens,
                         const size_t *offsets, size_t count, const size_t *stop, uint8_t *out,
                         size_t cap, size_t *lens);

/* Decodes `count` coded payloads (payload b is payloads[offsets[b] .. offsets[b + 1])) on
 * `batch` with the context overlap `overlap` (set on the batch, as hs_batch_set_overlap; a
 * value that does not fit the context is refused with its error). One slot per block: blocks
 * take the slots in order, and a slot whose block is complete takes the next waiting block
 * (crates/taco/src/gpu_unfold.rs:74-196). Block b's tokens go to tokens + b * cap; counts[b]
 * is its token count. */
hs_status tc_unfold_blocks(hs_batch *batch, uint32_t overlap, const uint8_t *payloads,
                           const size_t *offsets, size_t count, uint32_t *tokens, size_t cap,
                           size_t *counts);

/* ---- The tokenizer (crates/taco/src/tokenizer): GPT-2 byte-level BPE ---------------------- */
typedef struct tc_tokenizer tc_tokenizer;
/* Tokenizer::new (tokenizer/mod.rs:87-147): token i has the bytes token_bytes[token_offsets[i]
 * .. token_offsets[i + 1]) (count + 1 offsets); eot is the <|endoftext|> id (UINT32_MAX for
 * none); merges are `n_merges` (left, right) id pairs in rank order. The EOT token and tokens
 * with no bytes never appear in the output. Refused with HS_MODEL_ERROR (code
 * HS_MODEL_VOCABULARY) when a byte value has no single-byte token or two, or a merge is not
 * valid (a part out of range, EOT or empty; no token or two tokens with the joined bytes; a
 * pair given twice). */
hs_status tc_tokenizer_new(const uint8_t *token_bytes, const size_t *token_offsets, size_t count,
                           uint32_t eot, const uint32_t *merges, size_t n_merges,
                           tc_tokenizer **out);
/* Tokenizer::for_vocabulary (tokenizer/mod.rs:150-160): the vocabulary and merges of a model. */
hs_status tc_tokenizer_for_model(const hs_model *model, tc_tokenizer **out);
void tc_tokenizer_free(tc_tokenizer *tokenizer);
/* Tokenizer::encode (tokenizer/mod.rs:176-201): the token ids of data (maximal runs of
 * well-formed UTF-8 through the GPT-2 pre-tokenizer and the merges; any other byte as its
 * single-byte token). Writes up to cap ids; *count is the number of ids (HS_LENGTH_MISMATCH
 * when it exceeds cap). */
hs_status tc_tokenize(const tc_tokenizer *tokenizer, const uint8_t *data, size_t len, uint32_t *ids,
                      size_t cap, size_t *count);
/* The pieces of the GPT-2 pre-tokenizer (tokenizer/pretokenize.rs) of well-formed UTF-8 text:
 * writes the byte end of each piece (up to cap) and returns the number of pieces, or SIZE_MAX
 * when the text is not well-formed UTF-8. For tests. */
size_t tc_pretokenize(const uint8_t *text, size_t len, size_t *ends, size_t cap);

/* The byte-level fold of the text profile (crates/taco/src/fold.rs:502-565, code_segment):
 * `data` cut into blocks of block_size bytes, each block tokenized (its tokens must restore its
 * bytes), coded on `batch` with the context overlap, and each block stored as the smaller of
 * its coded payload and its raw bytes (Block::choose_smallest without a zstd candidate), in a
 * version-2 container. Writes the container to out when it fits cap; *out_len is its length. */
hs_status tc_fold_bytes(hs_batch *batch, const tc_tokenizer *tokenizer, const uint8_t *data,
                        size_t len, uint32_t block_size, uint32_t overlap, uint8_t *out, size_t cap,
                        size_t *out_len);

/* Container::build of format version 2 (crates/taco-format/src/writer.rs:245-288) for the text
 * profile: kinds[b] is 0 (raw) or 1 (coded); coded blocks are blocks[block_offsets[b] ..
 * block_offsets[b + 1]). Returns the container length (the bytes are written if cap allows),
 * or 0 on a refused input (a coded block that is not smaller than its original bytes). */
size_t tc_container_build(const uint8_t model_hash[32], const uint8_t *original, size_t len,
                          uint32_t block_size, uint32_t overlap, const uint8_t *kinds,
                          const uint8_t *blocks, const size_t *block_offsets, uint8_t *out,
                          size_t cap);

#ifdef __cplusplus
}
#endif
#endif /* TACO_HIP_H */
