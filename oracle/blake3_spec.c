/* TEST INFRASTRUCTURE — the CPU oracle, not the product.
 *
 * BLAKE3 from its public specification: the G function, seven rounds with the message
 * permutation between them, chunks of 1024 bytes chained block by block, parents over pairs
 * of chaining values, the ROOT flag on the last compression, and the extendable output read
 * by compressing the root node again with the output block counter. Keyed hashing replaces
 * the IV by the key words and sets KEYED_HASH on every compression.
 *
 * The tree is built incrementally: each finished chunk's chaining value is pushed on a stack
 * and merged with the stack top while the count of finished chunks is even; finalization folds
 * the stack right to left into the last chunk's output. This is a different algorithm from the
 * recursive split the product kernels and the Python twin (oracle/blake3_tree.py) use, so a
 * tree-shape mistake in either shows up as a disagreement.
 */
#include "blake3_spec.h"

#include <string.h>

enum {
  CHUNK_START = 1u << 0,
  CHUNK_END = 1u << 1,
  PARENT = 1u << 2,
  ROOT = 1u << 3,
  KEYED_HASH = 1u << 4,
};

static const uint32_t IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                               0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};

static const uint8_t PERM[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};

static inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static inline uint32_t load_le(const uint8_t *p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

static inline void store_le(uint8_t *p, uint32_t w) {
  p[0] = (uint8_t)w;
  p[1] = (uint8_t)(w >> 8);
  p[2] = (uint8_t)(w >> 16);
  p[3] = (uint8_t)(w >> 24);
}

static inline void g(uint32_t s[16], int a, int b, int c, int d, uint32_t mx, uint32_t my) {
  s[a] = s[a] + s[b] + mx;
  s[d] = rotr(s[d] ^ s[a], 16);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 12);
  s[a] = s[a] + s[b] + my;
  s[d] = rotr(s[d] ^ s[a], 8);
  s[c] = s[c] + s[d];
  s[b] = rotr(s[b] ^ s[c], 7);
}

void b3_compress(const uint32_t cv[8], const uint8_t block[B3_BLOCK_LEN], uint64_t counter,
                 uint32_t block_len, uint32_t flags, uint32_t out[16]) {
  uint32_t m[16], t[16], s[16];
  for (int i = 0; i < 16; i++) m[i] = load_le(block + 4 * i);
  for (int i = 0; i < 8; i++) s[i] = cv[i];
  for (int i = 0; i < 4; i++) s[8 + i] = IV[i];
  s[12] = (uint32_t)counter;
  s[13] = (uint32_t)(counter >> 32);
  s[14] = block_len;
  s[15] = flags;
  for (int r = 0; r < 7; r++) {
    g(s, 0, 4, 8, 12, m[0], m[1]);
    g(s, 1, 5, 9, 13, m[2], m[3]);
    g(s, 2, 6, 10, 14, m[4], m[5]);
    g(s, 3, 7, 11, 15, m[6], m[7]);
    g(s, 0, 5, 10, 15, m[8], m[9]);
    g(s, 1, 6, 11, 12, m[10], m[11]);
    g(s, 2, 7, 8, 13, m[12], m[13]);
    g(s, 3, 4, 9, 14, m[14], m[15]);
    if (r < 6) {
      for (int i = 0; i < 16; i++) t[i] = m[PERM[i]];
      memcpy(m, t, sizeof m);
    }
  }
  for (int i = 0; i < 8; i++) {
    out[i] = s[i] ^ s[i + 8];
    out[i + 8] = s[i + 8] ^ cv[i];
  }
}

/* A node's inputs before its final compression: what the root output or a chaining value is
 * computed from. */
typedef struct {
  uint32_t cv[8];
  uint8_t block[B3_BLOCK_LEN];
  uint64_t counter;
  uint8_t block_len;
  uint8_t flags;
} b3_output;

static void output_cv(const b3_output *o, uint32_t cv[8]) {
  uint32_t w[16];
  b3_compress(o->cv, o->block, o->counter, o->block_len, o->flags, w);
  memcpy(cv, w, 32);
}

static void chunk_init(b3_chunk_state *c, const uint32_t key[8], uint64_t counter,
                       uint8_t flags) {
  memcpy(c->cv, key, 32);
  c->chunk_counter = counter;
  memset(c->buf, 0, sizeof c->buf);
  c->buf_len = 0;
  c->blocks_compressed = 0;
  c->flags = flags;
}

static size_t chunk_len(const b3_chunk_state *c) {
  return (size_t)B3_BLOCK_LEN * c->blocks_compressed + c->buf_len;
}

static uint8_t chunk_start_flag(const b3_chunk_state *c) {
  return c->blocks_compressed == 0 ? CHUNK_START : 0;
}

static void chunk_update(b3_chunk_state *c, const uint8_t *in, size_t len) {
  while (len > 0) {
    if (c->buf_len == B3_BLOCK_LEN) {
      uint32_t w[16];
      b3_compress(c->cv, c->buf, c->chunk_counter, B3_BLOCK_LEN,
                  c->flags | chunk_start_flag(c), w);
      memcpy(c->cv, w, 32);
      c->blocks_compressed++;
      memset(c->buf, 0, sizeof c->buf);
      c->buf_len = 0;
    }
    size_t take = B3_BLOCK_LEN - c->buf_len;
    if (take > len) take = len;
    memcpy(c->buf + c->buf_len, in, take);
    c->buf_len += (uint8_t)take;
    in += take;
    len -= take;
  }
}

static b3_output chunk_output(const b3_chunk_state *c) {
  b3_output o;
  memcpy(o.cv, c->cv, 32);
  memcpy(o.block, c->buf, B3_BLOCK_LEN);
  o.counter = c->chunk_counter;
  o.block_len = c->buf_len;
  o.flags = c->flags | chunk_start_flag(c) | CHUNK_END;
  return o;
}

static b3_output parent_output(const uint32_t left[8], const uint32_t right[8],
                               const uint32_t key[8], uint8_t flags) {
  b3_output o;
  memcpy(o.cv, key, 32);
  for (int i = 0; i < 8; i++) store_le(o.block + 4 * i, left[i]);
  for (int i = 0; i < 8; i++) store_le(o.block + 32 + 4 * i, right[i]);
  o.counter = 0;
  o.block_len = B3_BLOCK_LEN;
  o.flags = flags | PARENT;
  return o;
}

static void hasher_init(b3_hasher *h, const uint32_t key[8], uint8_t flags) {
  memcpy(h->key, key, 32);
  chunk_init(&h->chunk, key, 0, flags);
  h->cv_stack_len = 0;
}

void b3_init(b3_hasher *h) { hasher_init(h, IV, 0); }

void b3_init_keyed(b3_hasher *h, const uint8_t key[B3_KEY_LEN]) {
  uint32_t k[8];
  for (int i = 0; i < 8; i++) k[i] = load_le(key + 4 * i);
  hasher_init(h, k, KEYED_HASH);
}

static void add_chunk_cv(b3_hasher *h, uint32_t cv[8], uint64_t total_chunks) {
  /* Each trailing zero bit of the finished-chunk count closes one complete subtree. */
  while ((total_chunks & 1) == 0) {
    b3_output p = parent_output(h->cv_stack[--h->cv_stack_len], cv, h->key, h->chunk.flags);
    output_cv(&p, cv);
    total_chunks >>= 1;
  }
  memcpy(h->cv_stack[h->cv_stack_len++], cv, 32);
}

void b3_update(b3_hasher *h, const void *input, size_t len) {
  const uint8_t *in = (const uint8_t *)input;
  while (len > 0) {
    if (chunk_len(&h->chunk) == B3_CHUNK_LEN) {
      uint32_t cv[8];
      b3_output o = chunk_output(&h->chunk);
      output_cv(&o, cv);
      uint64_t total = h->chunk.chunk_counter + 1;
      add_chunk_cv(h, cv, total);
      chunk_init(&h->chunk, h->key, total, h->chunk.flags);
    }
    size_t take = B3_CHUNK_LEN - chunk_len(&h->chunk);
    if (take > len) take = len;
    chunk_update(&h->chunk, in, take);
    in += take;
    len -= take;
  }
}

void b3_finalize_seek(const b3_hasher *h, uint64_t seek, uint8_t *out, size_t out_len) {
  b3_output o = chunk_output(&h->chunk);
  for (size_t i = h->cv_stack_len; i > 0; i--) {
    uint32_t right[8];
    output_cv(&o, right);
    o = parent_output(h->cv_stack[i - 1], right, h->key, h->chunk.flags);
  }
  uint64_t block = seek / 64;
  size_t skip = (size_t)(seek % 64);
  while (out_len > 0) {
    uint32_t w[16];
    uint8_t bytes[64];
    b3_compress(o.cv, o.block, block, o.block_len, o.flags | ROOT, w);
    for (int i = 0; i < 16; i++) store_le(bytes + 4 * i, w[i]);
    size_t take = 64 - skip;
    if (take > out_len) take = out_len;
    memcpy(out, bytes + skip, take);
    out += take;
    out_len -= take;
    skip = 0;
    block++;
  }
}

void b3_finalize(const b3_hasher *h, uint8_t *out, size_t out_len) {
  b3_finalize_seek(h, 0, out, out_len);
}
