/* TEST INFRASTRUCTURE — the CPU oracle, not the product.
 *
 * BLAKE3 written from its public specification (the BLAKE3 paper, section 2: compression
 * function, chunk chaining, binary tree, keyed mode, extendable output). The reference
 * (pacifai/pots-2.0) links BLAKE3's C library 1.8.7, fetched from GitHub at build time
 * (verification/commitment/native.py:51-54); that library is not in this container, so this
 * restatement stands in for it. It is an incremental hasher with a chaining-value stack, the
 * structure the specification describes for streaming input.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this code.
 */
#ifndef POTS_ORACLE_BLAKE3_SPEC_H
#define POTS_ORACLE_BLAKE3_SPEC_H

#include <stddef.h>
#include <stdint.h>

#define B3_OUT_LEN 32
#define B3_KEY_LEN 32
#define B3_BLOCK_LEN 64
#define B3_CHUNK_LEN 1024

typedef struct {
  uint32_t cv[8];
  uint64_t chunk_counter;
  uint8_t buf[B3_BLOCK_LEN];
  uint8_t buf_len;
  uint8_t blocks_compressed;
  uint8_t flags;
} b3_chunk_state;

typedef struct {
  uint32_t key[8];
  b3_chunk_state chunk;
  uint8_t cv_stack_len;
  uint32_t cv_stack[54][8]; /* 2^54 chunks is beyond any input this code sees */
} b3_hasher;

void b3_init(b3_hasher *h);
void b3_init_keyed(b3_hasher *h, const uint8_t key[B3_KEY_LEN]);
void b3_update(b3_hasher *h, const void *input, size_t len);
/* Extended output from byte offset `seek`; `out_len` bytes. */
void b3_finalize_seek(const b3_hasher *h, uint64_t seek, uint8_t *out, size_t out_len);
void b3_finalize(const b3_hasher *h, uint8_t *out, size_t out_len);

/* The compression function alone, exported for the known-answer tests. */
void b3_compress(const uint32_t cv[8], const uint8_t block[B3_BLOCK_LEN], uint64_t counter,
                 uint32_t block_len, uint32_t flags, uint32_t out[16]);

#endif
