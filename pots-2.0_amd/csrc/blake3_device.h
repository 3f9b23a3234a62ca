// BLAKE3 compression on gfx950, written from the BLAKE3 specification.
//
// One lane runs one compression at a time with the 16 state words and the 16 message words
// in VGPRs. The seven rounds are unrolled with the message permutation folded into the
// register names (the schedule below), so no word moves between rounds. Rotations compile to
// v_alignbit_b32 and the three-input adds to v_add3_u32: about 12 VALU ops per G, ~690 per
// 64-byte block, which makes hashing integer-VALU bound on this chip (~11 ops per byte).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pots {

enum : uint32_t {
  B3_CHUNK_START = 1u << 0,
  B3_CHUNK_END = 1u << 1,
  B3_PARENT = 1u << 2,
  B3_ROOT = 1u << 3,
  B3_KEYED_HASH = 1u << 4,
};

constexpr uint32_t B3_IV0 = 0x6A09E667u, B3_IV1 = 0xBB67AE85u, B3_IV2 = 0x3C6EF372u,
                   B3_IV3 = 0xA54FF53Au, B3_IV4 = 0x510E527Fu, B3_IV5 = 0x9B05688Cu,
                   B3_IV6 = 0x1F83D9ABu, B3_IV7 = 0x5BE0CD19u;

__device__ __forceinline__ uint32_t rotr32(uint32_t x, uint32_t n) {
  return (x >> n) | (x << (32u - n));
}

#define POTS_B3_G(a, b, c, d, mx, my) \
  do {                                \
    a = a + b + (mx);                 \
    d = rotr32(d ^ a, 16);            \
    c = c + d;                        \
    b = rotr32(b ^ c, 12);            \
    a = a + b + (my);                 \
    d = rotr32(d ^ a, 8);             \
    c = c + d;                        \
    b = rotr32(b ^ c, 7);             \
  } while (0)

// One round with message word order s0..s15 (the permutation applied r times).
#define POTS_B3_ROUND(m, s0, s1, s2, s3, s4, s5, s6, s7, s8, s9, s10, s11, s12, s13, s14, s15) \
  do {                                                                                         \
    POTS_B3_G(v0, v4, v8, v12, m[s0], m[s1]);                                                  \
    POTS_B3_G(v1, v5, v9, v13, m[s2], m[s3]);                                                  \
    POTS_B3_G(v2, v6, v10, v14, m[s4], m[s5]);                                                 \
    POTS_B3_G(v3, v7, v11, v15, m[s6], m[s7]);                                                 \
    POTS_B3_G(v0, v5, v10, v15, m[s8], m[s9]);                                                 \
    POTS_B3_G(v1, v6, v11, v12, m[s10], m[s11]);                                               \
    POTS_B3_G(v2, v7, v8, v13, m[s12], m[s13]);                                                \
    POTS_B3_G(v3, v4, v9, v14, m[s14], m[s15]);                                                \
  } while (0)

// The state after the seven rounds, before the output feed-forward: v[0..15].
__device__ __forceinline__ void b3_rounds(const uint32_t cv[8], const uint32_t m[16],
                                          uint32_t counter_lo, uint32_t counter_hi,
                                          uint32_t block_len, uint32_t flags,
                                          uint32_t v[16]) {
  uint32_t v0 = cv[0], v1 = cv[1], v2 = cv[2], v3 = cv[3];
  uint32_t v4 = cv[4], v5 = cv[5], v6 = cv[6], v7 = cv[7];
  uint32_t v8 = B3_IV0, v9 = B3_IV1, v10 = B3_IV2, v11 = B3_IV3;
  uint32_t v12 = counter_lo, v13 = counter_hi, v14 = block_len, v15 = flags;
  POTS_B3_ROUND(m, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
  POTS_B3_ROUND(m, 2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8);
  POTS_B3_ROUND(m, 3, 4, 10, 12, 13, 2, 7, 14, 6, 5, 9, 0, 11, 15, 8, 1);
  POTS_B3_ROUND(m, 10, 7, 12, 9, 14, 3, 13, 15, 4, 0, 11, 2, 5, 8, 1, 6);
  POTS_B3_ROUND(m, 12, 13, 9, 11, 15, 10, 14, 8, 7, 2, 5, 3, 0, 1, 6, 4);
  POTS_B3_ROUND(m, 9, 14, 11, 5, 8, 12, 15, 1, 13, 3, 0, 10, 2, 6, 4, 7);
  POTS_B3_ROUND(m, 11, 15, 5, 0, 1, 9, 8, 6, 14, 10, 2, 12, 3, 4, 7, 13);
  v[0] = v0; v[1] = v1; v[2] = v2; v[3] = v3; v[4] = v4; v[5] = v5; v[6] = v6; v[7] = v7;
  v[8] = v8; v[9] = v9; v[10] = v10; v[11] = v11; v[12] = v12; v[13] = v13; v[14] = v14;
  v[15] = v15;
}

// The chaining value (first 8 output words) of one compression; `cv` may alias `out`.
__device__ __forceinline__ void b3_compress_cv(const uint32_t cv[8], const uint32_t m[16],
                                               uint64_t counter, uint32_t block_len,
                                               uint32_t flags, uint32_t out[8]) {
  uint32_t v[16];
  b3_rounds(cv, m, (uint32_t)counter, (uint32_t)(counter >> 32), block_len, flags, v);
#pragma unroll
  for (int i = 0; i < 8; i++) out[i] = v[i] ^ v[i + 8];
}

// The same with a 32-bit counter (its high word a compile-time zero).
__device__ __forceinline__ void b3_compress_cv32(const uint32_t cv[8], const uint32_t m[16],
                                                 uint32_t counter, uint32_t block_len,
                                                 uint32_t flags, uint32_t out[8]) {
  uint32_t v[16];
  b3_rounds(cv, m, counter, 0u, block_len, flags, v);
#pragma unroll
  for (int i = 0; i < 8; i++) out[i] = v[i] ^ v[i + 8];
}

// All 16 output words (the extendable-output block of a root compression).
__device__ __forceinline__ void b3_compress_xof(const uint32_t cv[8], const uint32_t m[16],
                                                uint64_t counter, uint32_t block_len,
                                                uint32_t flags, uint32_t out[16]) {
  uint32_t v[16];
  b3_rounds(cv, m, (uint32_t)counter, (uint32_t)(counter >> 32), block_len, flags, v);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    out[i] = v[i] ^ v[i + 8];
    out[i + 8] = v[i + 8] ^ cv[i];
  }
}

__device__ __forceinline__ void b3_iv(uint32_t cv[8]) {
  cv[0] = B3_IV0; cv[1] = B3_IV1; cv[2] = B3_IV2; cv[3] = B3_IV3;
  cv[4] = B3_IV4; cv[5] = B3_IV5; cv[6] = B3_IV6; cv[7] = B3_IV7;
}

// Parent node of two chaining values under the unkeyed IV: the 64-byte block left || right.
__device__ __forceinline__ void b3_parent_cv(const uint32_t l[8], const uint32_t r[8],
                                             uint32_t flags, uint32_t out[8]) {
  uint32_t m[16], iv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    m[i] = l[i];
    m[i + 8] = r[i];
  }
  b3_iv(iv);
  b3_compress_cv(iv, m, 0, 64, B3_PARENT | flags, out);
}

}  // namespace pots
