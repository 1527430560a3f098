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
