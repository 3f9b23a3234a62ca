/* TEST INFRASTRUCTURE — the CPU oracle, not the product.
 *
 * A restatement of the reference's native batch (verification/commitment/native.c) over the
 * spec BLAKE3 of blake3_spec.c, with the same semantics entry point by entry point:
 *
 *   oracle_hash_leaves   native.c:243 pots_hash_leaves: leaf i's digest BLAKE3(0x00 || header
 *                        || payload), the payload tested for NaN/Inf 64 KiB at a time before
 *                        it is hashed (native.c:199-217), leaves handed to threads by an atomic
 *                        grab counter (native.c:219-234); returns the smallest index whose
 *                        payload is non-finite, or n.
 *   oracle_all_finite    native.c:299 pots_all_finite.
 *   oracle_merkle_tree   native.c:315-337 build_tree / pots_merkle_tree: the 2n - 1 node
 *                        hashes of the RFC 6962 tree in pre-order, H_node = BLAKE3(0x01||l||r).
 *   oracle_challenges    native.c:71-139 fill_rows / pots_challenges: keyed XOF of the label
 *                        0x10 || m (BE32) || j, entries (2(w >> 8) + 1 - 2^24) / 2^24, item i's
 *                        matrix [widths[i], k] row-major at out + offsets[i].
 *
 * It is also the bench's CPU baseline ("port"): scalar BLAKE3 on pthreads.
 */
#include <pthread.h>
#include <stdatomic.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "blake3_spec.h"

#define MAX_THREADS 256

static int run_threads(void *(*fn)(void *), void *arg, uint32_t t) {
  pthread_t tids[MAX_THREADS];
  uint32_t started = 0;
  int rc = 0;
  if (t > MAX_THREADS) t = MAX_THREADS;
  for (; started + 1 < t; started++)
    if (pthread_create(&tids[started], NULL, fn, arg) != 0) {
      rc = -2;
      break;
    }
  fn(arg);
  for (uint32_t i = 0; i < started; i++) pthread_join(tids[i], NULL);
  return rc;
}

/* ---- finiteness (native.c:146-169) ---- */

enum { KIND_NONE = 0, KIND_F32 = 1, KIND_BF16 = 2, KIND_F16 = 3 };

static int block_finite(const uint8_t *p, size_t nbytes, uint8_t kind) {
  uint32_t bad = 0;
  if (kind == KIND_F32) {
    for (size_t i = 0; i + 4 <= nbytes; i += 4) {
      uint32_t w;
      memcpy(&w, p + i, 4);
      bad |= (w & 0x7f800000u) == 0x7f800000u;
    }
  } else if (kind == KIND_BF16 || kind == KIND_F16) {
    uint16_t mask = kind == KIND_BF16 ? 0x7f80 : 0x7c00;
    for (size_t i = 0; i + 2 <= nbytes; i += 2) {
      uint16_t h;
      memcpy(&h, p + i, 2);
      bad |= (uint16_t)(h & mask) == mask;
    }
  }
  return !bad;
}

/* ---- leaf hashing (native.c:171-259) ---- */

#define BLOCK_BYTES (64 << 10)
#define GRAB_BYTES (1 << 20)
#define BYTES_PER_THREAD (1 << 20)

typedef struct {
  size_t n;
  const uint8_t *hdr_buf;
  const uint64_t *hdr_off;
  const uint32_t *hdr_len;
  const uint32_t *hdr_idx;
  const uint64_t *payload_ptr;
  const uint64_t *payload_len;
  const uint8_t *kind;
  uint8_t *out;
  size_t per_grab;
  atomic_size_t next;
  atomic_size_t bad;
} leaf_job_t;

static void note_bad(leaf_job_t *job, size_t i) {
  size_t cur = atomic_load(&job->bad);
  while (i < cur && !atomic_compare_exchange_weak(&job->bad, &cur, i)) {
  }
}

static int hash_one_leaf(const leaf_job_t *job, size_t i) {
  static const uint8_t prefix = 0x00;
  uint32_t u = job->hdr_idx[i];
  const uint8_t *p = (const uint8_t *)(uintptr_t)job->payload_ptr[i];
  uint64_t len = job->payload_len[i];
  uint8_t kind = job->kind[i];
  b3_hasher h;
  b3_init(&h);
  b3_update(&h, &prefix, 1);
  if (job->hdr_len[u]) b3_update(&h, job->hdr_buf + job->hdr_off[u], job->hdr_len[u]);
  for (uint64_t pos = 0; pos < len;) {
    size_t take = len - pos < BLOCK_BYTES ? (size_t)(len - pos) : BLOCK_BYTES;
    if (kind && !block_finite(p + pos, take, kind)) return 0;
    b3_update(&h, p + pos, take);
    pos += take;
  }
  b3_finalize(&h, job->out + 32 * i, 32);
  return 1;
}

static void *leaf_worker(void *arg) {
  leaf_job_t *job = arg;
  for (;;) {
    size_t lo = atomic_fetch_add(&job->next, job->per_grab);
    if (lo >= job->n) break;
    size_t hi = lo + job->per_grab < job->n ? lo + job->per_grab : job->n;
    for (size_t i = lo; i < hi; i++) {
      if (i > atomic_load(&job->bad)) break;
      if (!hash_one_leaf(job, i)) {
        note_bad(job, i);
        break;
      }
    }
  }
  return NULL;
}

size_t oracle_hash_leaves(size_t n, const uint8_t *hdr_buf, const uint64_t *hdr_off,
                          const uint32_t *hdr_len, const uint32_t *hdr_idx,
                          const uint64_t *payload_ptr, const uint64_t *payload_len,
                          const uint8_t *kind, uint8_t *out, uint32_t n_threads) {
  if (n == 0) return 0;
  uint64_t total = 0;
  for (size_t i = 0; i < n; i++) total += payload_len[i] + hdr_len[hdr_idx[i]];
  leaf_job_t job = {n, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len,
                    kind, out, 1, 0, n};
  uint64_t avg = total / n;
  job.per_grab = avg >= GRAB_BYTES ? 1 : (size_t)(GRAB_BYTES / (avg ? avg : 1));
  uint64_t useful = total / BYTES_PER_THREAD;
  uint32_t t = n_threads < 1 ? 1 : n_threads;
  if (useful < t) t = useful < 1 ? 1 : (uint32_t)useful;
  run_threads(leaf_worker, &job, t);
  return atomic_load(&job.bad);
}

int oracle_all_finite(const uint8_t *p, uint64_t nbytes, uint8_t kind) {
  if (nbytes == 0 || kind < KIND_F32 || kind > KIND_F16) return 1;
  for (uint64_t pos = 0; pos < nbytes;) {
    size_t take = nbytes - pos < BLOCK_BYTES ? (size_t)(nbytes - pos) : BLOCK_BYTES;
    if (!block_finite(p + pos, take, kind)) return 0;
    pos += take;
  }
  return 1;
}

/* One message hashed whole: the helper the Python side uses for hash_leaf / hash_node. */
void oracle_blake3(const uint8_t *msg, size_t len, const uint8_t *key, uint64_t seek,
                   uint8_t *out, size_t out_len) {
  b3_hasher h;
  if (key) b3_init_keyed(&h, key);
  else b3_init(&h);
  b3_update(&h, msg, len);
  b3_finalize_seek(&h, seek, out, out_len);
}

/* ---- Merkle tree (native.c:312-337) ---- */

static void build_tree(const uint8_t *leaves, size_t lo, size_t hi, uint8_t *nodes, size_t p) {
  if (hi - lo == 1) {
    memcpy(nodes + 32 * p, leaves + 32 * lo, 32);
    return;
  }
  size_t k = 1;
  while (k * 2 < hi - lo) k *= 2;
  build_tree(leaves, lo, lo + k, nodes, p + 1);
  build_tree(leaves, lo + k, hi, nodes, p + 2 * k);
  uint8_t buf[65];
  buf[0] = 0x01;
  memcpy(buf + 1, nodes + 32 * (p + 1), 32);
  memcpy(buf + 33, nodes + 32 * (p + 2 * k), 32);
  oracle_blake3(buf, sizeof buf, NULL, 0, nodes + 32 * p, 32);
}

void oracle_merkle_tree(size_t n, const uint8_t *leaves, uint8_t *nodes) {
  if (n >= 1) build_tree(leaves, 0, n, nodes, 0);
}

/* ---- challenges (native.c:50-139) ---- */

#define ROWS 256

typedef struct {
  const uint8_t *key;
  uint32_t k;
  size_t n;
  const uint32_t *ms;
  const uint32_t *widths;
  const uint64_t *offsets;
  float *out;
  const uint64_t *first;
  atomic_size_t next;
} ch_job_t;

static void fill_rows(const uint8_t *key, uint32_t m, uint32_t k, uint32_t e0, uint32_t e1,
                      float *mat) {
  uint8_t buf[4 * ROWS];
  size_t rows = e1 - e0;
  for (uint32_t j = 1; j <= k; j++) {
    uint8_t label[6] = {0x10, (uint8_t)(m >> 24), (uint8_t)(m >> 16), (uint8_t)(m >> 8),
                        (uint8_t)m, (uint8_t)j};
    oracle_blake3(label, sizeof label, key, 4 * (uint64_t)e0, buf, 4 * rows);
    float *col = mat + (size_t)e0 * k + (j - 1);
    for (size_t e = 0; e < rows; e++) {
      const uint8_t *b = buf + 4 * e;
      uint32_t w = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 |
                   (uint32_t)b[3] << 24;
      int32_t numerator = 2 * (int32_t)(w >> 8) + 1 - (1 << 24);
      col[e * k] = (float)numerator / 16777216.0f;
    }
  }
}

static void *challenge_worker(void *arg) {
  ch_job_t *job = arg;
  size_t total = job->first[job->n];
  for (;;) {
    size_t u = atomic_fetch_add(&job->next, 1);
    if (u >= total) break;
    size_t a = 0, b = job->n;
    while (b - a > 1) {
      size_t mid = a + (b - a) / 2;
      if (job->first[mid] <= u) a = mid;
      else b = mid;
    }
    uint32_t e0 = (uint32_t)(u - job->first[a]) * ROWS;
    uint32_t e1 = e0 + ROWS < job->widths[a] ? e0 + ROWS : job->widths[a];
    fill_rows(job->key, job->ms[a], job->k, e0, e1, job->out + job->offsets[a]);
  }
  return NULL;
}

int oracle_challenges(const uint8_t key[32], uint32_t k, size_t n, const uint32_t *ms,
                      const uint32_t *widths, const uint64_t *offsets, float *out,
                      uint32_t n_threads) {
  if (n == 0) return 0;
  uint64_t *first = malloc((n + 1) * sizeof *first);
  if (!first) return -1;
  first[0] = 0;
  for (size_t i = 0; i < n; i++) first[i + 1] = first[i] + (widths[i] + ROWS - 1) / ROWS;
  ch_job_t job = {key, k, n, ms, widths, offsets, out, first, 0};
  int rc = run_threads(challenge_worker, &job, n_threads < 1 ? 1 : n_threads);
  free(first);
  return rc;
}

void oracle_compress(const uint32_t cv[8], const uint8_t block[64], uint64_t counter,
                     uint32_t block_len, uint32_t flags, uint32_t out[16]) {
  b3_compress(cv, block, counter, block_len, flags, out);
}
