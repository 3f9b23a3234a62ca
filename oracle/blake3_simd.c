/* TEST INFRASTRUCTURE — the CPU oracle, not the product.
 *
 * The bench's CPU baseline at the speed of the reference's own CPU path. The reference hashes
 * each leaf on one thread with BLAKE3's C library (native.c:171-259), which compresses many
 * whole chunks at once with SIMD ("hash_many": one chunk per 32-bit vector lane); leaves go to
 * pthreads by an atomic grab counter. This file restates that with AVX-512, written from the
 * BLAKE3 specification (the paper, section 2, and its section 5.3 on SIMD over chunks):
 *
 *   - 16 whole chunks of a leaf are compressed together, one per lane: the 16 chunks' block b
 *     is loaded as 16 rows of 16 words and transposed, so vector w holds message word w of
 *     every chunk; the 7 rounds then run on 16-lane vectors;
 *   - a leaf's last, partial chunk and the parent nodes are compressed one at a time with the
 *     spec's compression function (b3_compress in blake3_spec.c);
 *   - the tree is BLAKE3's: the left subtree holds the largest power of two of chunks below
 *     the count, and only the top node carries ROOT;
 *   - the payload's NaN/Inf test runs on the whole payload before it is hashed, 64 bytes per
 *     vector comparison (native.c:152-169 tests each 64 KiB before hashing it; the first
 *     non-finite leaf and the digests before it are the same either way).
 *
 * oracle_hash_leaves_simd has oracle_hash_leaves's signature and results; the CPU tests check
 * it against the spec hasher on every chunk-count boundary. Without AVX-512 it reports a SIMD
 * degree of 1 and hashes with the spec hasher.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "blake3_spec.h"

enum { CHUNK_START = 1, CHUNK_END = 2, PARENT = 4, ROOT = 8 };
enum { KIND_NONE = 0, KIND_F32 = 1, KIND_BF16 = 2, KIND_F16 = 3 };

static const uint32_t IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                               0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};

static int have_avx512(void) {
  static int cached = -1;
  if (cached < 0) {
    __builtin_cpu_init();
    cached = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
  }
  return cached;
}

int oracle_simd_degree(void) { return have_avx512() ? 16 : 1; }

/* ---- 16 chunks at once ------------------------------------------------------------------ */

#define V __m512i
#define TGT __attribute__((target("avx512f,avx512bw")))

TGT static inline V add(V a, V b) { return _mm512_add_epi32(a, b); }
TGT static inline V xor_(V a, V b) { return _mm512_xor_si512(a, b); }

TGT static inline void g16(V *s, int a, int b, int c, int d, V mx, V my) {
  s[a] = add(add(s[a], s[b]), mx);
  s[d] = _mm512_ror_epi32(xor_(s[d], s[a]), 16);
  s[c] = add(s[c], s[d]);
  s[b] = _mm512_ror_epi32(xor_(s[b], s[c]), 12);
  s[a] = add(add(s[a], s[b]), my);
  s[d] = _mm512_ror_epi32(xor_(s[d], s[a]), 8);
  s[c] = add(s[c], s[d]);
  s[b] = _mm512_ror_epi32(xor_(s[b], s[c]), 7);
}

/* The message word order of round r: the permutation applied r times (the spec permutes the
 * message between rounds; here the schedule is a table). */
static const uint8_t SCHED[7][16] = {
    {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15},
    {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8},
    {3, 4, 10, 12, 13, 2, 7, 14, 6, 5, 9, 0, 11, 15, 8, 1},
    {10, 7, 12, 9, 14, 3, 13, 15, 4, 0, 11, 2, 5, 8, 1, 6},
    {12, 13, 9, 11, 15, 10, 14, 8, 7, 2, 5, 3, 0, 1, 6, 4},
    {9, 14, 11, 5, 8, 12, 15, 1, 13, 3, 0, 10, 2, 6, 4, 7},
    {11, 15, 5, 0, 1, 9, 8, 6, 14, 10, 2, 12, 3, 4, 7, 13},
};

/* cv ← the first half of compress(cv, m, counter, 64, flags), lane by lane. */
TGT static inline void compress16(V cv[8], const V m[16], V ctr_lo, V ctr_hi, uint32_t flags) {
  V s[16];
  for (int i = 0; i < 8; i++) s[i] = cv[i];
  for (int i = 0; i < 4; i++) s[8 + i] = _mm512_set1_epi32((int)IV[i]);
  s[12] = ctr_lo;
  s[13] = ctr_hi;
  s[14] = _mm512_set1_epi32(64);
  s[15] = _mm512_set1_epi32((int)flags);
  /* unrolled, so that the schedule's indices are constants and the message stays in registers */
#pragma GCC unroll 7
  for (int r = 0; r < 7; r++) {
    const uint8_t *p = SCHED[r];
    g16(s, 0, 4, 8, 12, m[p[0]], m[p[1]]);
    g16(s, 1, 5, 9, 13, m[p[2]], m[p[3]]);
    g16(s, 2, 6, 10, 14, m[p[4]], m[p[5]]);
    g16(s, 3, 7, 11, 15, m[p[6]], m[p[7]]);
    g16(s, 0, 5, 10, 15, m[p[8]], m[p[9]]);
    g16(s, 1, 6, 11, 12, m[p[10]], m[p[11]]);
    g16(s, 2, 7, 8, 13, m[p[12]], m[p[13]]);
    g16(s, 3, 4, 9, 14, m[p[14]], m[p[15]]);
  }
  for (int i = 0; i < 8; i++) cv[i] = xor_(s[i], s[i + 8]);
}

/* rows[i] = 16 words of lane i  →  rows[w] = word w of every lane. */
TGT static inline void transpose16(V r[16]) {
  V a[16], b[16];
  for (int i = 0; i < 16; i += 2) {
    a[i] = _mm512_unpacklo_epi32(r[i], r[i + 1]);
    a[i + 1] = _mm512_unpackhi_epi32(r[i], r[i + 1]);
  }
  /* b[4g + s], 128-bit lane L: word 4L + s of rows 4g .. 4g + 3 */
  for (int i = 0; i < 16; i += 4) {
    b[i] = _mm512_unpacklo_epi64(a[i], a[i + 2]);
    b[i + 1] = _mm512_unpackhi_epi64(a[i], a[i + 2]);
    b[i + 2] = _mm512_unpacklo_epi64(a[i + 1], a[i + 3]);
    b[i + 3] = _mm512_unpackhi_epi64(a[i + 1], a[i + 3]);
  }
  /* word 4L + s, 128-bit lane G = b[4G + s], lane L: a 4x4 transpose of 128-bit lanes */
  for (int s = 0; s < 4; s++) {
    V t0 = _mm512_shuffle_i32x4(b[s], b[4 + s], _MM_SHUFFLE(1, 0, 1, 0));
    V t1 = _mm512_shuffle_i32x4(b[s], b[4 + s], _MM_SHUFFLE(3, 2, 3, 2));
    V t2 = _mm512_shuffle_i32x4(b[8 + s], b[12 + s], _MM_SHUFFLE(1, 0, 1, 0));
    V t3 = _mm512_shuffle_i32x4(b[8 + s], b[12 + s], _MM_SHUFFLE(3, 2, 3, 2));
    r[s] = _mm512_shuffle_i32x4(t0, t2, _MM_SHUFFLE(2, 0, 2, 0));
    r[4 + s] = _mm512_shuffle_i32x4(t0, t2, _MM_SHUFFLE(3, 1, 3, 1));
    r[8 + s] = _mm512_shuffle_i32x4(t1, t3, _MM_SHUFFLE(2, 0, 2, 0));
    r[12 + s] = _mm512_shuffle_i32x4(t1, t3, _MM_SHUFFLE(3, 1, 3, 1));
  }
}

/* The chaining values of 16 whole chunks: lane i's chunk is the 1024 bytes at in[i], chunk
 * counter counter0 + i. */
TGT static void chunks16(const uint8_t *const in[16], uint64_t counter0, uint32_t out[16][8]) {
  V cv[8];
  for (int i = 0; i < 8; i++) cv[i] = _mm512_set1_epi32((int)IV[i]);
  const V lane = _mm512_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
  const V lo0 = _mm512_set1_epi32((int)(uint32_t)counter0);
  const V ctr_lo = add(lo0, lane);
  /* carry into the high word where the low word wrapped */
  const __mmask16 wrap = _mm512_cmplt_epu32_mask(ctr_lo, lo0);
  const V hi0 = _mm512_set1_epi32((int)(uint32_t)(counter0 >> 32));
  const V ctr_hi = _mm512_mask_add_epi32(hi0, wrap, hi0, _mm512_set1_epi32(1));
  for (int b = 0; b < 16; b++) {
    V m[16];
    for (int i = 0; i < 16; i++) m[i] = _mm512_loadu_si512((const void *)(in[i] + 64 * b));
    transpose16(m);
    const uint32_t flags = (b == 0 ? CHUNK_START : 0u) | (b == 15 ? CHUNK_END : 0u);
    compress16(cv, m, ctr_lo, ctr_hi, flags);
  }
  uint32_t w[8][16];
  for (int i = 0; i < 8; i++) _mm512_storeu_si512((void *)w[i], cv[i]);
  for (int l = 0; l < 16; l++)
    for (int i = 0; i < 8; i++) out[l][i] = w[i][l];
}

/* True when no value of the payload is NaN or Inf (its exponent field all ones). */
TGT static int finite_avx512(const uint8_t *p, uint64_t n, uint8_t kind) {
  if (kind == KIND_NONE) return 1;
  uint64_t i = 0;
  if (kind == KIND_F32) {
    const V mask = _mm512_set1_epi32(0x7f800000);
    for (; i + 64 <= n; i += 64) {
      V x = _mm512_and_si512(_mm512_loadu_si512((const void *)(p + i)), mask);
      if (_mm512_cmpeq_epi32_mask(x, mask)) return 0;
    }
    for (; i + 4 <= n; i += 4) {
      uint32_t w;
      memcpy(&w, p + i, 4);
      if ((w & 0x7f800000u) == 0x7f800000u) return 0;
    }
    return 1;
  }
  const uint16_t m16 = kind == KIND_BF16 ? 0x7f80 : 0x7c00;
  const V mask = _mm512_set1_epi16((short)m16);
  for (; i + 64 <= n; i += 64) {
    V x = _mm512_and_si512(_mm512_loadu_si512((const void *)(p + i)), mask);
    if (_mm512_cmpeq_epi16_mask(x, mask)) return 0;
  }
  for (; i + 2 <= n; i += 2) {
    uint16_t h;
    memcpy(&h, p + i, 2);
    if ((uint16_t)(h & m16) == m16) return 0;
  }
  return 1;
}

/* ---- one chunk, one parent, the tree ------------------------------------------------------ */

static void words_to_bytes(const uint32_t *w, int n, uint8_t *out) {
  for (int i = 0; i < n; i++) {
    out[4 * i] = (uint8_t)w[i];
    out[4 * i + 1] = (uint8_t)(w[i] >> 8);
    out[4 * i + 2] = (uint8_t)(w[i] >> 16);
    out[4 * i + 3] = (uint8_t)(w[i] >> 24);
  }
}

/* The chaining value of a chunk of len (1..1024) bytes, not the root. */
static void chunk_cv(const uint8_t *data, size_t len, uint64_t counter, uint32_t cv[8]) {
  uint32_t out[16];
  memcpy(cv, IV, sizeof IV);
  size_t nb = (len + 63) / 64;
  for (size_t b = 0; b < nb; b++) {
    uint8_t block[64] = {0};
    size_t take = len - 64 * b < 64 ? len - 64 * b : 64;
    memcpy(block, data + 64 * b, take);
    uint32_t flags = (b == 0 ? CHUNK_START : 0u) | (b + 1 == nb ? CHUNK_END : 0u);
    b3_compress(cv, block, counter, (uint32_t)take, flags, out);
    memcpy(cv, out, 32);
  }
}

static void parent(const uint32_t l[8], const uint32_t r[8], uint32_t flags, uint32_t out8[8]) {
  uint8_t block[64];
  uint32_t out[16];
  words_to_bytes(l, 8, block);
  words_to_bytes(r, 8, block + 32);
  b3_compress(IV, block, 0, 64, PARENT | flags, out);
  memcpy(out8, out, 32);
}

/* The node over cvs[0 .. n): the left subtree takes the largest power of two below n. */
static void subtree(const uint32_t (*cvs)[8], uint64_t n, uint32_t flags, uint32_t out[8]) {
  if (n == 1) {
    memcpy(out, cvs[0], 32);
    return;
  }
  uint64_t k = 1;
  while (2 * k < n) k *= 2;
  uint32_t l[8], r[8];
  subtree(cvs, k, 0, l);
  subtree(cvs + k, n - k, 0, r);
  parent(l, r, flags, out);
}

/* BLAKE3(head ‖ payload) into out (32 bytes), with the 16-lane chunk compressor. */
TGT static int leaf_digest(const uint8_t *head, size_t hl, const uint8_t *payload, uint64_t len,
                           uint8_t out[32]) {
  const uint64_t total = hl + len;
  if (total <= 1024) {  /* one chunk: it is the root */
    b3_hasher h;
    b3_init(&h);
    b3_update(&h, head, hl);
    if (len) b3_update(&h, payload, (size_t)len);
    b3_finalize(&h, out, 32);
    return 1;
  }
  const uint64_t n = (total + 1023) / 1024;
  const uint64_t full = total % 1024 ? n - 1 : n;
  uint32_t (*cvs)[8] = malloc(n * sizeof *cvs);
  if (!cvs) return 0;
  uint8_t first[1024];  /* chunk 0: head, then the payload's first bytes */
  memcpy(first, head, hl);
  memcpy(first + hl, payload, 1024 - hl);
  for (uint64_t c0 = 0; c0 < full; c0 += 16) {
    const uint8_t *in[16];
    for (int l = 0; l < 16; l++) {
      uint64_t c = c0 + (uint64_t)l;
      in[l] = c >= full ? first : c == 0 ? first : payload + 1024 * c - hl;
    }
    uint32_t got[16][8];
    chunks16(in, c0, got);
    for (int l = 0; l < 16 && c0 + (uint64_t)l < full; l++) memcpy(cvs[c0 + l], got[l], 32);
  }
  if (full < n)
    chunk_cv(payload + 1024 * full - hl, (size_t)(total - 1024 * full), full, cvs[full]);
  uint32_t root[8];
  subtree((const uint32_t(*)[8])cvs, n, ROOT, root);
  words_to_bytes(root, 8, out);
  free(cvs);
  return 1;
}

/* ---- leaves on pthreads (native.c:219-259) ------------------------------------------------ */

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
  atomic_int failed;
} simd_job_t;

static void note_bad(simd_job_t *job, size_t i) {
  size_t cur = atomic_load(&job->bad);
  while (i < cur && !atomic_compare_exchange_weak(&job->bad, &cur, i)) {
  }
}

TGT static int hash_leaf(simd_job_t *job, size_t i) {
  uint32_t u = job->hdr_idx[i];
  uint8_t head[1 + 1024];
  size_t hl = 1 + job->hdr_len[u];
  if (hl > sizeof head) return -1;
  head[0] = 0x00;
  memcpy(head + 1, job->hdr_buf + job->hdr_off[u], hl - 1);
  const uint8_t *p = (const uint8_t *)(uintptr_t)job->payload_ptr[i];
  uint64_t len = job->payload_len[i];
  if (!finite_avx512(p, len, job->kind[i])) return 0;
  return leaf_digest(head, hl, p, len, job->out + 32 * i) ? 1 : -1;
}

static void *simd_worker(void *arg) {
  simd_job_t *job = arg;
  for (;;) {
    size_t lo = atomic_fetch_add(&job->next, job->per_grab);
    if (lo >= job->n) break;
    size_t hi = lo + job->per_grab < job->n ? lo + job->per_grab : job->n;
    for (size_t i = lo; i < hi; i++) {
      if (i > atomic_load(&job->bad)) break;
      int rc = hash_leaf(job, i);
      if (rc < 0) atomic_store(&job->failed, 1);
      if (rc <= 0) {
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
                          const uint8_t *kind, uint8_t *out, uint32_t n_threads);

/* oracle_hash_leaves with the 16-lane chunk compressor; SIZE_MAX when a leaf's header is
 * longer than 1 KiB or memory ran out. */
size_t oracle_hash_leaves_simd(size_t n, const uint8_t *hdr_buf, const uint64_t *hdr_off,
                               const uint32_t *hdr_len, const uint32_t *hdr_idx,
                               const uint64_t *payload_ptr, const uint64_t *payload_len,
                               const uint8_t *kind, uint8_t *out, uint32_t n_threads) {
  if (!have_avx512())
    return oracle_hash_leaves(n, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len,
                              kind, out, n_threads);
  if (n == 0) return 0;
  uint64_t total = 0;
  for (size_t i = 0; i < n; i++) total += payload_len[i] + hdr_len[hdr_idx[i]];
  simd_job_t job = {n, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len,
                    kind, out, 1, 0, n, 0};
  uint64_t avg = total / n;
  job.per_grab = avg >= (1u << 20) ? 1 : (size_t)((1u << 20) / (avg ? avg : 1));
  uint32_t t = n_threads < 1 ? 1 : n_threads > 256 ? 256 : n_threads;
  pthread_t tids[256];
  uint32_t started = 0;
  for (; started + 1 < t; started++)
    if (pthread_create(&tids[started], NULL, simd_worker, &job) != 0) break;
  simd_worker(&job);
  for (uint32_t i = 0; i < started; i++) pthread_join(tids[i], NULL);
  if (atomic_load(&job.failed)) return SIZE_MAX;
  return atomic_load(&job.bad);
}
