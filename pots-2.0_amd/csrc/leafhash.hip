// Leaf hashing on gfx950: H_leaf = BLAKE3(0x00 || header || payload) for every leaf of a
// transcript in one pass over HBM, with the NaN/Inf test fused into the loads.
//
// Reference: verification/commitment/native.c:171-259 (pots_hash_leaves, hash_leaf,
// leaf_worker) and verification/commitment/leaves.py:312-437 (the batching around it).
//
// Decomposition. Every leaf's message is cut into BLAKE3's 1 KiB chunks; one lane compresses
// one chunk (up to 16 blocks) and writes its chaining value, or the digest itself when the
// leaf is a single chunk. The chunk CVs of a leaf form BLAKE3's tree, which has the RFC 6962
// shape (a run of n > 1 chunks splits at the largest power of two below n), so it is reduced
// level by level: level l+1 node j is the parent of level-l nodes 2j and 2j+1, or node 2j
// itself when it has no sibling. The node that covers the whole leaf gets the ROOT flag.
//
// Message layout in HBM. The 0x00 prefix and the tensor header are 4(1 + ndim) bytes, a whole
// number of words, so message word w of a leaf is payload word w - H/4 and no byte shifting is
// needed. A lane reads two 64-byte blocks at a time as 16-byte aligned loads and picks their
// 32 words out of the 36-word window with a shift SH (0..3) that is fixed per leaf; SH is a
// template parameter so the selection is register renaming. Blocks that touch the header, the end of
// the payload or a partial word take an edge path that patches header words in from a small
// table and masks bytes past the end. Leaves whose header length or payload address is not
// word aligned (records, odd views, host memory) are staged: their whole message is copied to
// an aligned device buffer first and hashed with an empty header.
//
// Finiteness. A value is NaN or Inf when its exponent field is all ones. Masking each payload
// word to its exponent fields and keeping a running per-16-bit-half maximum (one and, one
// packed max per word) reaches the all-ones pattern exactly when a non-finite value was seen.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <new>
#include <unordered_set>
#include <vector>

#include "blake3_device.h"
#include "common.h"
#include "freivalds.h"
#include "gmem.h"

namespace pots {

constexpr uint32_t kNoFuse = 0xFFFFFFFFu;

struct LeafDesc {
  uint64_t payload;    // device address of payload byte 0 (word aligned)
  uint64_t len;        // payload bytes
  uint32_t head_word;  // first word of this leaf's 0x00 || header in the head table
  uint32_t head_len;   // bytes of 0x00 || header, a multiple of 4 (0 for a staged leaf)
  uint32_t kind;       // POTS_KIND_*
  uint32_t fin_from;   // message byte where the payload (the NaN/Inf-tested bytes) begins
  uint64_t cv_first;   // where chunk 0's chaining value goes in the level-0 buffer
  uint32_t n_chunks;   // 1 KiB chunks of the message (at least 1)
  uint32_t fuse;       // index of its fused-product entry, or kNoFuse
};
static_assert(sizeof(LeafDesc) == 48, "LeafDesc layout");

// A leaf whose product's P-pass sums the chunk kernel takes (freivalds.h). Its first nf
// chunks are hashed in class order: class kappa = c mod T holds the chunks whose payload
// offset is the same modulo the row length. A lane hashes a run of consecutive chunks (of
// classes t0 .. t0 + RC − 1 of one period when T >= 4; of PG whole periods when T < 4), and
// the runs of one class range get Q lanes (Q a multiple of 64, padding lanes idle), so every
// wave is at one common column offset at each step of its runs: R is read with scalar loads,
// one copy for the wave. A last chunk with fewer than 128 bytes has no interior
// pair and no P-pass work; it is left out of the classes (nf = n_chunks - 1) and hashed by a
// wave of its own after them, so that the header's few bytes do not pad every class.
struct FuseDesc {
  uint64_t r;          // R [m][k] fp32, row-major
  uint64_t seg;        // run records [J][n_rows]
  uint32_t row_bytes;  // m · esz
  uint32_t n_rows;
  uint32_t J;          // record slots per row
  uint32_t T;          // classes
  uint32_t Q;          // lanes per class
  uint32_t esz;        // 2 (bf16) or 4 (fp32)
  uint32_t nf;         // chunks in class order
  uint32_t run;        // a lane's run: classes (low 16 bits) x periods (high 16 bits)
};
static_assert(sizeof(FuseDesc) == 48, "FuseDesc layout");

struct LevelEntry {     // one leaf with >= 2 nodes at the input level of one fold
  uint64_t in_off;      // its first node in the level's input buffer
  uint64_t out_off;     // its first node in the fold's output buffer
  uint64_t out_first;   // its first output, counted over the level's entries
  uint32_t n_in;        // its nodes at this level
  uint32_t leaf;
};
static_assert(sizeof(LevelEntry) == 32, "LevelEntry layout");

constexpr int kThreads = 256;
// Consecutive chunks one lane hashes in a row: each chunk after the first takes its first
// bytes from the unit its predecessor's last pair loaded, so the 128-byte line before a 1 KiB
// boundary is read once, not again by the next chunk.
#ifndef POTS_CHUNK_RUN
#define POTS_CHUNK_RUN 4
#endif
constexpr uint32_t kRun = POTS_CHUNK_RUN;
// Tree levels one launch of level_kernel reduces.
constexpr uint32_t kFold = 3;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// The NaN/Inf test of a chunk's payload words, one accumulator per lane: `mask` keeps each
// value's exponent field (fp32 0x7F800000, bf16 0x7F807F80, fp16 0x7C007C00, none 0), and the
// running per-half maximum of the masked words reaches the all-ones exponent (0x7F80 for fp32
// and bf16, 0x7C00 for fp16) exactly when a non-finite value was seen. Two VALU operations per
// word (and, packed 16-bit max). (A per-kind test with one v_dot2c_f32_bf16 per word measured
// slower: the chunk kernel's code doubles and its time went up by 5%.)
struct Fin {
  u16x2 acc = {0, 0};
  uint32_t mask;
  unsigned short thr;
  __device__ __forceinline__ explicit Fin(uint32_t kind)
      : mask(kind == POTS_KIND_F32    ? 0x7F800000u
             : kind == POTS_KIND_BF16 ? 0x7F807F80u
             : kind == POTS_KIND_F16  ? 0x7C007C00u
                                      : 0u),
        thr(kind == POTS_KIND_F16 ? 0x7C00 : 0x7F80) {}
  __device__ __forceinline__ void add(uint32_t w) {
    acc = __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, w & mask));
  }
  __device__ __forceinline__ bool bad() const {
    return mask != 0u && (acc.x >= thr || acc.y >= thr);
  }
};

// ---- P-pass sums of a fused product leaf ---------------------------------------------------
//
// A lane keeps one run at a time: Σ x·R[col][j] (j < 4) and Σ|x| in fp32 over the run, Σx² in
// fp32 over each 128-byte pair and in fp64 across pairs. A run ends where its row does (the
// row boundary is at the same offset in every lane of the wave, so the branch is uniform) and
// at the end of the chunk, and is written as one record.
//
// Σx² in fp32 is exact to rounding only while the squares are normal and their sum finite: a
// run with a pair whose largest biased exponent (from the NaN/Inf test's per-pair maximum) is
// outside [kSqLo, kSqHi] (|x| below 2^-50 or from 2^63 on) is marked in its record, and the
// P stage then takes that row's squares in fp64 from P, as the unfused P pass does.

constexpr uint32_t kSqLo = 127 - 50, kSqHi = 127 + 62;

typedef float v4f32 __attribute__((ext_vector_type(4)));
#define POTS_CONST __attribute__((address_space(4)))

struct PRun {
  float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f, s1 = 0.f;
  double s2 = 0.0;
  bool live = false;
  bool exact = false;  // a pair's exponents leave fp32 squares' range: the row is redone in fp64
};

// The elements t in [lo, hi) of a 128-byte pair (words w[0..31] of payload) into the run;
// element t's column is R row rcol + t (rcol: wave-uniform address of R's row for t = 0; a
// row is the plan's K challenges, K of 1, 2 or 4). Unmasked, every element of the pair is
// taken and the bounds are not read.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Elements t in [lo, hi) of a pair (its 32 payload words w) into the run. `emax`: the pair's
// largest biased exponent; outside [kSqLo, kSqHi] the run is marked for the exact squares.
typedef float v2f32 __attribute__((ext_vector_type(2)));

//
// `s1p`, `q2p`: an unmasked bf16 pair's Σ|x| and Σx², taken with the NaN/Inf test (unused
// otherwise). `zero`: every element of the pair is zero, whose squares are exact whatever the
// exponent test says.
template <int ESZ, bool MASKED, int K>
__device__ __forceinline__ void run_add(const uint32_t* w, float s1p, float q2p, uint64_t rcol,
                                        uint32_t lo, uint32_t hi, uint32_t emax, bool zero,
                                        PRun& a) {
  constexpr int NE = 128 / ESZ;
  static_assert(K == 1 || K == 2 || K == 4, "R rows of 1, 2 or 4 challenges");
  float q = 0.f;
#pragma unroll
  for (int t = 0; t < NE; t++) {
    if (MASKED && !((uint32_t)t >= lo && (uint32_t)t < hi)) continue;
    uint32_t wt = w[ESZ == 2 ? t >> 1 : t];
    // A masked pair is taken in two calls over the same words: an empty asm statement per
    // element keeps each conversion under its own bounds test, where the compiler would
    // otherwise convert all of the pair's elements once, ahead of both calls, and hold them.
    if (MASKED) asm volatile("" : "+v"(wt));
    float x;
    if (ESZ == 2) x = __uint_as_float((t & 1) ? (wt & 0xFFFF0000u) : (wt << 16));
    else x = __uint_as_float(wt);
    if constexpr (K == 4) {
      const v4f32 r = reinterpret_cast<const POTS_CONST v4f32*>(rcol)[t];
      a.d0 = fmaf(x, r[0], a.d0);
      a.d1 = fmaf(x, r[1], a.d1);
      a.d2 = fmaf(x, r[2], a.d2);
      a.d3 = fmaf(x, r[3], a.d3);
    } else if constexpr (K == 2) {
      const v2f32 r = reinterpret_cast<const POTS_CONST v2f32*>(rcol)[t];
      a.d0 = fmaf(x, r[0], a.d0);
      a.d1 = fmaf(x, r[1], a.d1);
    } else {
      a.d0 = fmaf(x, reinterpret_cast<const POTS_CONST float*>(rcol)[t], a.d0);
    }
    if (MASKED || ESZ == 4) {
      a.s1 += fabsf(x);
      q = fmaf(x, x, q);
    }
  }
  if (!MASKED && ESZ == 2) {
    a.s1 += s1p;
    q = q2p;
  }
  a.s2 += (double)q;
  a.exact |= (emax < kSqLo && !zero) || emax > kSqHi;
  a.live = true;
}

// Write the run of `row` in chunk c (message offset of the payload H) as its record: slot
// c − (chunk of the row's first element a chunk takes). Out-of-range indices are not written.
__device__ __forceinline__ void run_flush(const FuseDesc& f, uint64_t H, uint32_t row,
                                          uint64_t c, PRun& a) {
  if (a.live) {
    const uint64_t hc = (H + 127) & ~uint64_t(127);
    const uint64_t fs = max<uint64_t>(H + (uint64_t)row * f.row_bytes, hc);
    const uint64_t slot = c - (fs >> 10);
    if (row < f.n_rows && slot < f.J) {
      char* rec = reinterpret_cast<char*>(f.seg) +
                  (uint64_t)kRunBytes * (slot * f.n_rows + row);
      gstore<v4f32>(rec, v4f32{a.d0, a.d1, a.d2, a.d3});
      const uint64_t sb = (uint64_t)__double_as_longlong(a.s2);
      gstore<u32x4>(rec + 16, u32x4{__float_as_uint(a.s1), a.exact ? 1u : 0u, (uint32_t)sb,
                                    (uint32_t)(sb >> 32)});
    }
  }
  a = PRun();
}

// Message block b of chunk c for the general case: blocks that touch the header, the end of
// the payload or a partial word. Header words come from the head table (a staged leaf holds
// its header in the staged message instead); bytes past the end are zero; only payload words
// (from fin_from on) feed the NaN/Inf test.
template <int SH>
__device__ __forceinline__ void edge_block(const LeafDesc& d, const uint32_t* __restrict__ head,
                                           uint64_t o, uint32_t m[16], Fin& fin) {
  const uint64_t H = d.head_len, L = H + d.len;
  const uint64_t pbeg = d.payload, pend = d.payload + d.len;
  const uint64_t A = d.payload + o - H;  // address of message byte o, in payload terms
  const u32x4* A16 = reinterpret_cast<const u32x4*>(A & ~uint64_t(15));
  uint32_t w[20];
#pragma unroll
  for (int u = 0; u < 5; u++) {
    const uint64_t X = reinterpret_cast<uint64_t>(A16 + u);
    u32x4 q = u32x4{0, 0, 0, 0};
    if ((u < 4 || SH) && X + 16 > pbeg && X < pend) q = gload<u32x4>(A16 + u);
    w[4 * u] = q.x;
    w[4 * u + 1] = q.y;
    w[4 * u + 2] = q.z;
    w[4 * u + 3] = q.w;
  }
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint64_t at = o + 4u * j;  // message byte offset of this word
    uint32_t mw = w[j + SH];
    if (at < H) {
      mw = gload<uint32_t>(head + d.head_word + (uint32_t)(at >> 2));
    } else if (at >= L) {
      mw = 0;
    } else {
      const uint64_t rem = L - at;
      if (rem < 4) mw &= (1u << (8 * rem)) - 1u;
      if (at >= d.fin_from) fin.add(mw);
    }
    m[j] = mw;
  }
}

// One lane's chunk c of leaf d: its chaining value (or the leaf digest when `root`). Blocks
// go in pairs: a pair wholly inside the payload is read as one 144-byte aligned window (nine
// 16-byte loads), so each 128-byte line a lane touches is used up by one group of loads
// instead of being fetched again for the second half; other pairs take edge_block.
//
// ESZ != 0 (a fused product leaf, SH == 1): each interior pair's elements also go into the
// lane's P-pass run.
//
// `carry`, `have_carry`: with SH != 0, the last unit the previous pair loaded, kept across the
// chunks of a lane's run (the caller starts a run with have_carry false; chunk c + 1's first
// window begins with chunk c's last unit).
template <int SH, int ESZ, int K = 4>
__device__ __forceinline__ void hash_chunk(const LeafDesc& d, const uint32_t* __restrict__ head,
                                           uint64_t c, bool root, uint32_t cv[8], Fin& fin,
                                           const FuseDesc& f, u32x4& carry, bool& have_carry) {
  const uint64_t H = d.head_len;
  const uint64_t L = H + d.len;
  const uint64_t cstart = c * 1024u;
  const uint64_t cbytes = min<uint64_t>(1024u, L - cstart);
  uint32_t nb = (uint32_t)((cbytes + 63) / 64);
  if (nb == 0) nb = 1;  // the empty message: one empty block
  b3_iv(cv);
  // With SH != 0 a pair's window starts with the last 16 bytes of the previous pair's line;
  // they are carried over in registers rather than loaded again (a second load of a line
  // already streamed past is often an HBM refetch).
  PRun run;
  uint32_t prow = 0, prb = 0;  // row of the next pair and its byte offset in the row
  bool pinit = false;
#pragma unroll 1
  for (uint32_t b = 0; b < nb; b += 2) {
    const uint64_t o = cstart + 64u * b;
    uint32_t m0[16], m1[16];
    if (o >= d.fin_from && o + 128 <= L) {
      const u32x4* A16 =
          reinterpret_cast<const u32x4*>((d.payload + o - H) & ~uint64_t(15));
      u32x4 q[9];
      if (SH) {
        if (have_carry) q[0] = carry;
        else q[0] = gload<u32x4>(A16);
#pragma unroll
        for (int u = 1; u < 9; u++) q[u] = gload<u32x4>(A16 + u);
        carry = q[8];
        have_carry = true;
      } else {
#pragma unroll
        for (int u = 0; u < 8; u++) q[u] = gload<u32x4>(A16 + u);
        q[8] = u32x4{0, 0, 0, 0};
      }
      uint32_t w[36];
#pragma unroll
      for (int u = 0; u < 9; u++) {
        w[4 * u] = q[u].x;
        w[4 * u + 1] = q[u].y;
        w[4 * u + 2] = q[u].z;
        w[4 * u + 3] = q[u].w;
      }
#pragma unroll
      for (int j = 0; j < 16; j++) {
        m0[j] = w[j + SH];
        m1[j] = w[16 + j + SH];
      }
      // The NaN/Inf test's per-pair maximum (a tree, then one merge into the running one). A
      // fused bf16 leaf's words are masked to |x| (sign bits cleared) instead of to their
      // exponents: a half reaches 0x7F80 for the same values, and the pair's Σ|x| takes the
      // masked words two elements per v_dot2 against (1, 1), beside Σx² from each word
      // against itself (products of bf16 values are exact in fp32).
      const uint32_t pmask = ESZ == 2 ? 0x7FFF7FFFu : fin.mask;
      u16x2 pm[8];
      float s1p = 0.f, q2p = 0.f;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        uint32_t aw[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t wu = w[4 * j + e + SH];
          aw[e] = wu & pmask;
          if constexpr (ESZ == 2) {
            s1p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, aw[e]),
                                                  __builtin_bit_cast(bf16x2, 0x3F803F80u), s1p,
                                                  false);
            q2p = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wu),
                                                  __builtin_bit_cast(bf16x2, wu), q2p, false);
          }
        }
        pm[j] = __builtin_elementwise_max(
            __builtin_elementwise_max(__builtin_bit_cast(u16x2, aw[0]),
                                      __builtin_bit_cast(u16x2, aw[1])),
            __builtin_elementwise_max(__builtin_bit_cast(u16x2, aw[2]),
                                      __builtin_bit_cast(u16x2, aw[3])));
      }
#pragma unroll
      for (int j = 0; j < 4; j++) pm[j] = __builtin_elementwise_max(pm[j], pm[j + 4]);
      pm[0] = __builtin_elementwise_max(__builtin_elementwise_max(pm[0], pm[1]),
                                        __builtin_elementwise_max(pm[2], pm[3]));
      fin.acc = __builtin_elementwise_max(fin.acc, pm[0]);
      if constexpr (ESZ != 0) {
        // the pair's largest biased exponent: bf16 halves hold it at bit 7, fp32 at bit 23
        const uint32_t pmax = ESZ == 2 ? (uint32_t)max(pm[0].x, pm[0].y) : (uint32_t)pm[0].y;
        const uint32_t emax = pmax >> 7;
        // an all-zero pair, whose squares are exact (bf16; fp32's test keeps only exponents,
        // which do not tell zeros from subnormals)
        const bool zero = ESZ == 2 && pmax == 0;
        if (!pinit) {  // the chunk's first interior pair
          const uint64_t po = o - H;
          prow = (uint32_t)(po / f.row_bytes);
          prb = (uint32_t)(po - (uint64_t)prow * f.row_bytes);
          pinit = true;
        }
        // Every active lane holds the same offset (the class order), so these are scalars.
        // (readfirstlane returns int: each word goes through uint32_t before widening.)
        const uint32_t rb = (uint32_t)__builtin_amdgcn_readfirstlane(prb);
        const uint64_t rbase =
            (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(f.r >> 32)) << 32 |
            (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)f.r);
        if (rb + 128 <= f.row_bytes) {
          run_add<ESZ, false, K>(w + SH, s1p, q2p, rbase + (uint64_t)(rb / ESZ) * (4 * K), 0,
                                 128 / ESZ, emax, zero, run);
          prb = rb + 128;
          if (prb == f.row_bytes) {
            run_flush(f, H, prow, c, run);
            prow++;
            prb = 0;
          }
        } else {  // the pair ends row prow at element tb and starts row prow + 1
          const uint32_t tb = (f.row_bytes - rb) / ESZ;
          run_add<ESZ, true, K>(w + SH, 0.f, 0.f, rbase + (uint64_t)(rb / ESZ) * (4 * K), 0,
                                tb, emax, zero, run);
          run_flush(f, H, prow, c, run);
          prow++;
          run_add<ESZ, true, K>(w + SH, 0.f, 0.f, rbase - (uint64_t)tb * (4 * K), tb,
                                128 / ESZ, emax, zero, run);
          prb = rb + 128 - f.row_bytes;
        }
      }
      // Two whole 64-byte blocks of which the first never ends the chunk: the block lengths
      // are constant, and the chunk counter fits 32 bits (plan creation refuses a leaf of
      // 4 TiB or more).
      b3_compress_cv32(cv, m0, (uint32_t)c, 64u, b == 0 ? B3_CHUNK_START : 0u, cv);
      b3_compress_cv32(cv, m1, (uint32_t)c, 64u,
                       b + 2 == nb ? (B3_CHUNK_END | (root ? B3_ROOT : 0u)) : 0u, cv);
      continue;
    }
    edge_block<SH>(d, head, o, m0, fin);
    if (b + 1 < nb) edge_block<SH>(d, head, o + 64, m1, fin);
    have_carry = false;
    const uint32_t blen0 = (uint32_t)min<uint64_t>(64u, L > o ? L - o : 0u);
    uint32_t f0 = b == 0 ? B3_CHUNK_START : 0u;
    if (b + 1 == nb) f0 |= B3_CHUNK_END | (root ? B3_ROOT : 0u);
    b3_compress_cv(cv, m0, c, blen0, f0, cv);
    if (b + 1 < nb) {
      const uint32_t blen1 = (uint32_t)min<uint64_t>(64u, L - o - 64);
      const uint32_t f1 = b + 2 == nb ? (B3_CHUNK_END | (root ? B3_ROOT : 0u)) : 0u;
      b3_compress_cv(cv, m1, c, blen1, f1, cv);
    }
  }
  if constexpr (ESZ != 0) run_flush(f, H, prow, c, run);
}

// A chunk order: entry e covers slots first[e] .. first[e + 1] of leaf leaf[e], and the
// entries of block b's slots (kThreads of them) lie in blk_ent[b] .. blk_ent[b + 1].
struct Order {
  const uint64_t* __restrict__ first;
  const uint32_t* __restrict__ leaf;
  const uint32_t* __restrict__ blk_ent;
  uint64_t n_slots;   // slots of the order
  uint32_t n_blocks;  // ceil(n_slots / kThreads)
};

__device__ __forceinline__ uint32_t order_entry(const Order& od, uint64_t g, uint32_t blk) {
  uint32_t lo = od.blk_ent[blk], hi = od.blk_ent[blk + 1];
  while (lo < hi) {  // the last entry whose first slot is <= g
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (od.first[mid] <= g) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

__device__ __forceinline__ void store_cv(uint32_t* p, const uint32_t cv[8]) {
  u32x4* dst = reinterpret_cast<u32x4*>(p);
  gstore<u32x4>(dst, u32x4{cv[0], cv[1], cv[2], cv[3]});
  gstore<u32x4>(dst + 1, u32x4{cv[4], cv[5], cv[6], cv[7]});
}

// Chunks c0 .. c1 − 1 of leaf i, one after another on one lane, each chaining value to cv_out
// (or the leaf digest itself for a one-chunk leaf).
template <int SH>
__device__ __forceinline__ void hash_run(const LeafDesc& d, const uint32_t* __restrict__ head,
                                         uint32_t i, uint64_t c0, uint64_t c1, Fin& fin,
                                         uint32_t* __restrict__ cv_out,
                                         uint32_t* __restrict__ digests) {
  const FuseDesc none{};
  const bool root = d.n_chunks == 1;
  u32x4 carry = u32x4{0, 0, 0, 0};
  bool have_carry = false;
#pragma unroll 1
  for (uint64_t c = c0; c < c1; c++) {
    uint32_t cv[8];
    hash_chunk<SH, 0>(d, head, c, root, cv, fin, none, carry, have_carry);
    store_cv(root ? digests + 8ull * i : cv_out + 8ull * (d.cv_first + c), cv);
  }
}

// Every chunk of the unfused leaves: slot g of the plain order is run g − first[e] of leaf
// leaf[e], its chunks kRun·(g − first[e]) onwards (slots past a leaf's runs are idle). Block b
// hashes slot blocks b, b + gridDim.x, ... so a grid smaller than the order holds a bounded
// share of the GPU and leaves the rest to kernels on other streams.
__global__ __launch_bounds__(kThreads) void chunk_kernel(
    const LeafDesc* __restrict__ leaves, Order od, const uint32_t* __restrict__ head,
    uint32_t* __restrict__ cv_out, uint32_t* __restrict__ digests,
    uint32_t* __restrict__ first_bad) {
  for (uint32_t blk = blockIdx.x; blk < od.n_blocks; blk += gridDim.x) {
    const uint64_t g = (uint64_t)blk * kThreads + threadIdx.x;
    if (g >= od.n_slots) continue;
    const uint32_t e = order_entry(od, g, blk);
    const uint32_t i = od.leaf[e];
    const LeafDesc d = leaves[i];
    const uint64_t c0 = (g - od.first[e]) * kRun;
    if (c0 >= d.n_chunks) continue;
    const uint64_t c1 = min<uint64_t>(c0 + kRun, d.n_chunks);
    Fin fin(d.kind);
    switch ((uint32_t)((d.payload - d.head_len) >> 2) & 3u) {
      case 0: hash_run<0>(d, head, i, c0, c1, fin, cv_out, digests); break;
      case 1: hash_run<1>(d, head, i, c0, c1, fin, cv_out, digests); break;
      case 2: hash_run<2>(d, head, i, c0, c1, fin, cv_out, digests); break;
      default: hash_run<3>(d, head, i, c0, c1, fin, cv_out, digests); break;
    }
    if (fin.bad()) atomicMin(first_bad, i);
  }
}

// With a block per order block, block b takes order block xcd_block(b, n) (gmem.h): each XCD
// hashes a contiguous range of the fused order, and neighbouring slots read the same rows of
// R, which one L2 then holds (the kernel's reads went from 1.12x to 1.05x its message bytes).
// The plain order has no R and keeps the hardware's interleave.
//
// The fused leaves (FuseDesc), each starting at a multiple of 64 slots in the fused order and
// holding a multiple of 64: a wave's slots are one leaf's and one class range's, so the entry,
// the leaf's descriptors and, at each step of the runs, R's rows are wave-uniform and live in
// scalar registers. Local slot l < NR·Q (NR = ceil(T / RC) class ranges) is the run of class
// range l / Q in period group l mod Q: chunks t0 + T·PG·(l mod Q) onwards (t0 = RC·(l / Q)),
// RC·PG of them, which are consecutive; the short last chunk follows.
template <int K>
__global__ __launch_bounds__(kThreads) void chunk_kernel_fused(
    const LeafDesc* __restrict__ leaves, const FuseDesc* __restrict__ fuses, Order od,
    const uint32_t* __restrict__ head, uint32_t* __restrict__ cv_out,
    uint32_t* __restrict__ first_bad) {
  const uint32_t wave_lane0 = threadIdx.x & ~63u;
  for (uint32_t b = blockIdx.x; b < od.n_blocks; b += gridDim.x) {
    const uint32_t blk = gridDim.x >= od.n_blocks ? xcd_block(b, od.n_blocks) : b;
    const uint64_t g0 = (uint64_t)blk * kThreads + wave_lane0;  // the wave's first slot
    if (g0 >= od.n_slots) continue;  // n_slots is a multiple of 64: whole waves
    const uint32_t e = (uint32_t)__builtin_amdgcn_readfirstlane(order_entry(od, g0, blk));
    const uint32_t i = od.leaf[e];
    const LeafDesc d = leaves[i];
    const FuseDesc f = fuses[d.fuse];
    const uint32_t rc = f.run & 0xFFFFu, pg = f.run >> 16;
    const uint32_t tq = (f.T + rc - 1) / rc * f.Q;
    const uint32_t l32 = (uint32_t)(g0 - od.first[e]) + (threadIdx.x & 63u);  // < tq + 64
    Fin fin(d.kind);
    uint32_t cv[8];
    if (l32 < tq) {
      const uint32_t t0 = l32 / f.Q * rc;
      const uint64_t cs = (uint64_t)t0 + (uint64_t)f.T * pg * (l32 % f.Q);
      const uint64_t ce = min<uint64_t>(cs + (uint64_t)min(rc, f.T - t0) * pg, f.nf);
      u32x4 carry = u32x4{0, 0, 0, 0};
      bool have_carry = false;
#pragma unroll 1
      for (uint64_t c = cs; c < ce; c++) {
        if (f.esz == 2) hash_chunk<1, 2, K>(d, head, c, false, cv, fin, f, carry, have_carry);
        else hash_chunk<1, 4, K>(d, head, c, false, cv, fin, f, carry, have_carry);
        store_cv(cv_out + 8ull * (d.cv_first + c), cv);
      }
      if (cs >= ce) continue;
    } else {  // the short last chunk, if any
      const uint64_t c = (uint64_t)f.nf + (l32 - tq);
      if (c >= d.n_chunks) continue;
      u32x4 carry = u32x4{0, 0, 0, 0};
      bool have_carry = false;
      hash_chunk<1, 0>(d, head, c, false, cv, fin, f, carry, have_carry);
      store_cv(cv_out + 8ull * (d.cv_first + c), cv);
    }
    if (fin.bad()) atomicMin(first_bad, i);
  }
}

// Levels kFold at a time: thread t makes output node o of its leaf at level l + kFold from the
// (at most 2^kFold) nodes o·2^kFold .. of level l, level by level in registers with
// BLAKE3's rule (pairs are hashed, a last odd node is promoted). A leaf whose tree closes
// inside the fold writes its digest (the compression that makes the single top node carries
// ROOT). Block b's outputs lie in entries blk_ent[b] .. blk_ent[b + 1].
__global__ __launch_bounds__(kThreads) void level_kernel(
    const LevelEntry* __restrict__ ents, const uint32_t* __restrict__ blk_ent, uint64_t n_out,
    const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
    uint32_t* __restrict__ digests) {
  const uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= n_out) return;
  uint32_t lo = blk_ent[blockIdx.x], hi = blk_ent[blockIdx.x + 1];
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (ents[mid].out_first <= t) lo = mid;
    else hi = mid - 1;
  }
  const LevelEntry e = ents[lo];
  const uint64_t o = t - e.out_first;
  constexpr uint32_t W = 1u << kFold;
  const uint64_t first = o * W;
  const uint32_t cnt = (uint32_t)min<uint64_t>(W, e.n_in - first);
  uint32_t cv[W][8];
  const uint4* src = reinterpret_cast<const uint4*>(in + 8ull * (e.in_off + first));
#pragma unroll
  for (uint32_t a = 0; a < W; a++) {
    uint4 x = make_uint4(0, 0, 0, 0), y = make_uint4(0, 0, 0, 0);
    if (a < cnt) {
      x = src[2 * a];
      y = src[2 * a + 1];
    }
    cv[a][0] = x.x; cv[a][1] = x.y; cv[a][2] = x.z; cv[a][3] = x.w;
    cv[a][4] = y.x; cv[a][5] = y.y; cv[a][6] = y.z; cv[a][7] = y.w;
  }
  // m: this thread's nodes at the current level; n: the leaf's nodes at the current level.
  uint32_t m = cnt;
  uint64_t n = e.n_in;
#pragma unroll
  for (uint32_t lvl = 0; lvl < kFold; lvl++) {
    const uint64_t n_next = (n + 1) / 2;
    const uint32_t flags = n_next == 1 ? B3_ROOT : 0u;
#pragma unroll
    for (uint32_t a = 0; a < (W >> (lvl + 1)); a++) {
      if (2 * a + 1 < m) {
        b3_parent_cv(cv[2 * a], cv[2 * a + 1], flags, cv[a]);
      } else if (2 * a < m) {
#pragma unroll
        for (int q = 0; q < 8; q++) cv[a][q] = cv[2 * a][q];
      }
    }
    m = (m + 1) / 2;
    n = n_next;
  }
  uint4* dst = reinterpret_cast<uint4*>(n == 1 ? digests + 8ull * e.leaf
                                               : out + 8ull * (e.out_off + o));
  dst[0] = make_uint4(cv[0][0], cv[0][1], cv[0][2], cv[0][3]);
  dst[1] = make_uint4(cv[0][4], cv[0][5], cv[0][6], cv[0][7]);
}

__global__ void fill_u32(uint32_t* p, uint32_t v) { *p = v; }

// ---- host side ----------------------------------------------------------------------------

struct StageCopy {  // a staged leaf: its head bytes, then its payload, into one aligned buffer
  uint64_t dst;         // device address of the staged message
  uint64_t head_src;    // device address of the head bytes in the metadata region
  uint64_t head_bytes;
  uint64_t payload_src; // payload address (host or device)
  uint64_t payload_bytes;
  bool host;            // payload in host memory
};

struct LevelInfo {
  uint64_t ent_first;  // index of the fold's first entry in the entry array
  uint32_t n_ents;
  uint64_t n_out;
  uint64_t blk_first;  // index of the fold's block -> entry table in blk_ent
  int in_buf, out_buf;  // 0 = cv0, 1 = cv1
};

struct LeafPlan {
  size_t n = 0;
  uint64_t n_chunks = 0, bytes = 0;
  uint32_t n_fused = 0;  // product leaves whose P-pass sums the chunk kernel takes
  uint32_t fuse_k = 4;   // the fused plan's challenges per product (1, 2 or 4)
  uint64_t fused_msg = 0, fused_chunks = 0, fused_records = 0;  // per run of the fused kernel
  FuseDesc* d_fuse = nullptr;
  Order plain{}, fused{};  // the two kernels' chunk orders (device tables)
  bool owned = false;
  char* base = nullptr;  // one device allocation: metadata, then workspace
  size_t total = 0;
  // device views
  LeafDesc* d_leaves = nullptr;
  uint32_t* d_head = nullptr;
  LevelEntry* d_levels = nullptr;
  uint32_t* d_blk_ent = nullptr;
  uint32_t* d_cv[2] = {nullptr, nullptr};
  uint32_t max_grid = 0;  // chunk kernel's grid limit; 0 = one block per slot
  std::vector<LevelInfo> levels;
  std::vector<StageCopy> stages;
};

// Build the plan's host image and sizes. `device_only` refuses host payloads.
// A chunk order on the host: entries (first slot, leaf) and the block -> entry table.
struct OrderHost {
  std::vector<uint64_t> first;  // n_ents + 1 (closing bound = n_slots)
  std::vector<uint32_t> leaf;
  std::vector<uint32_t> blk_ent;
  uint64_t n_slots = 0;
  uint32_t n_blocks = 0;
  void add(uint32_t i, uint64_t slots) {
    first.push_back(n_slots);
    leaf.push_back(i);
    n_slots += slots;
  }
  bool finish() {
    first.push_back(n_slots);
    const uint64_t nb = (n_slots + kThreads - 1) / kThreads;
    if (nb >= 0x7FFFFFFFull || leaf.size() >= 0xFFFFFFFFull) return false;
    n_blocks = (uint32_t)nb;
    blk_ent.assign(n_blocks + 1, 0);
    size_t e = 0;
    for (uint32_t b = 0; b < n_blocks; b++) {
      const uint64_t g = (uint64_t)b * kThreads;
      while (first[e + 1] <= g) e++;
      blk_ent[b] = (uint32_t)e;
    }
    blk_ent[n_blocks] = leaf.empty() ? 0 : (uint32_t)(leaf.size() - 1);
    return true;
  }
};

// A fused leaf's chunk order: T classes (chunk c in class c mod T, T = lcm(row bytes, 1024) /
// 1024, so a class's chunks start at one offset in the row). A lane's run is RC = min(T, kRun)
// consecutive classes of one period, or, when T < kRun, PG = kRun / T whole periods; the runs
// of one class range get Q lanes, the number of runs rounded up to 64. Fusing is declined when
// the padding would exceed 1/16 of the chunks even with runs of one chunk.
static bool fuse_shape(uint64_t msg_bytes, uint32_t row_bytes, uint32_t* T, uint32_t* Q,
                       uint32_t* run, uint32_t* nf, uint64_t* slots) {
  const uint64_t n_chunks = (msg_bytes + 1023) / 1024;
  const uint64_t f = msg_bytes % 1024 != 0 && msg_bytes % 1024 < 128 ? n_chunks - 1 : n_chunks;
  uint64_t a = row_bytes, b = 1024;
  while (b) {
    const uint64_t t = a % b;
    a = b;
    b = t;
  }
  const uint64_t t = (uint64_t)row_bytes / a;  // lcm / 1024
  const uint64_t periods = (f + t - 1) / t;
  // Runs of kRun chunks, or, where rounding their count up to 64 pads too much (a leaf of
  // few periods with T < kRun), runs of one chunk.
  const uint64_t shapes[2][2] = {{std::min<uint64_t>(t, kRun), t >= kRun ? 1 : kRun / t},
                                 {1, 1}};
  for (const auto& sh : shapes) {
    const uint64_t rc = sh[0], pg = sh[1];
    const uint64_t q = ((periods + pg - 1) / pg + 63) / 64 * 64;
    const uint64_t total = (t + rc - 1) / rc * q + (f < n_chunks ? 64 : 0);
    if (total >= 0xFFFFFFFFull || (t * pg * q - f) * 16 > f) continue;
    *T = (uint32_t)t;
    *Q = (uint32_t)q;
    *run = (uint32_t)(rc | pg << 16);
    *nf = (uint32_t)f;
    *slots = total;
    return true;
  }
  return false;
}

static int plan_build(size_t n, const uint8_t* hdr_buf, const uint64_t* hdr_off,
                      const uint32_t* hdr_len, const uint32_t* hdr_idx,
                      const uint64_t* payload_ptr, const uint64_t* payload_len,
                      const uint8_t* kind, bool device_only, bool owned, void* fv,
                      LeafPlan** out, char* ext_base = nullptr, size_t ext_cap = 0) {
  if (n == 0 || n >= 0xFFFFFFFFull) return POTS_E_ARG;
  for (size_t i = 0; i < n; i++)
    if (kind[i] > POTS_KIND_F16) return POTS_E_ARG;
  LeafPlan* P = new (std::nothrow) LeafPlan;
  if (!P) return POTS_E_NOMEM;
  P->n = n;
  P->owned = owned;

  // Per leaf: its head bytes (0x00 || header) and whether it must be staged.
  std::vector<LeafDesc> desc(n);
  std::vector<uint8_t> headbytes;  // word-aligned heads of direct leaves, then staged heads
  OrderHost plain, fused;
  std::vector<int64_t> stage_head_at(n, -1);
  uint64_t stage_bytes = 0;
  std::vector<uint64_t> stage_off(n, 0);
  std::vector<FuseDesc> fdesc;                 // per fused leaf
  std::vector<uint32_t> fprod, fhead;          // its product and head bytes
  std::unordered_set<uint32_t> fused_prods;
  uint64_t nc = 0;
  for (size_t i = 0; i < n; i++) {
    const uint32_t u = hdr_idx[i];
    const uint64_t hl = 1 + (uint64_t)hdr_len[u];
    const uint64_t len = payload_len[i];
    const uint64_t ptr = payload_ptr[i];
    bool host = false;
    if (len > 0) host = !is_device_pointer(reinterpret_cast<const void*>(ptr));
    if (host && device_only) {
      delete P;
      return POTS_E_ARG;
    }
    const bool stage = host || (hl % 4) != 0 || (ptr % 4) != 0;
    LeafDesc& d = desc[i];
    d.kind = kind[i];
    const uint64_t at = headbytes.size();
    headbytes.push_back(0x00);
    headbytes.insert(headbytes.end(), hdr_buf + hdr_off[u], hdr_buf + hdr_off[u] + hdr_len[u]);
    while (headbytes.size() % 4) headbytes.push_back(0);
    d.fin_from = (uint32_t)hl;  // the 0x00 || header bytes are never NaN/Inf-tested
    if (!stage) {
      d.payload = ptr;
      d.len = len;
      d.head_word = (uint32_t)(at / 4);
      d.head_len = (uint32_t)hl;
    } else {
      stage_head_at[i] = (int64_t)at;
      stage_off[i] = stage_bytes;
      stage_bytes += align_up(hl + len, 16);
      d.payload = 0;  // filled once the workspace address is known
      d.len = hl + len;
      d.head_word = 0;
      d.head_len = 0;
      P->stages.push_back(StageCopy{stage_off[i], at, hl, ptr, len, host});
    }
    const uint64_t L = hl + len;
    if (L >> 42) {  // 2^32 chunks: the chunk kernel's 32-bit counter
      delete P;
      return POTS_E_ARG;
    }
    const uint64_t nck = std::max<uint64_t>(1, (L + 1023) / 1024);
    d.cv_first = nc;
    d.n_chunks = (uint32_t)nck;
    d.fuse = kNoFuse;
    FusedProduct fp;
    uint32_t T = 0, Q = 0, run = 0, nf = 0;
    uint64_t slots = 0;
    if (fv && !stage && (kind[i] == POTS_KIND_BF16 || kind[i] == POTS_KIND_F32) &&
        (ptr - hl) % 16 == 4 && fv_fuse_candidate(fv, ptr, len, kind[i], &fp) &&
        !fused_prods.count(fp.prod) && fuse_shape(L, fp.w * fp.esz, &T, &Q, &run, &nf, &slots)) {
      fused_prods.insert(fp.prod);
      P->fuse_k = fp.k;  // one Freivalds plan: every fused product has the plan's k
      FuseDesc f;
      memset(&f, 0, sizeof f);
      f.r = fp.r;
      f.row_bytes = fp.w * fp.esz;
      f.n_rows = fp.n;
      f.J = (f.row_bytes + 1023) / 1024 + 1;
      f.T = T;
      f.Q = Q;
      f.esz = fp.esz;
      f.nf = nf;
      f.run = run;
      d.fuse = (uint32_t)fdesc.size();
      fdesc.push_back(f);
      fprod.push_back(fp.prod);
      fhead.push_back((uint32_t)hl);
      fused.add((uint32_t)i, slots);  // slots: a multiple of 64, so every entry is aligned
      P->fused_msg += L;
      P->fused_chunks += nck;
      {  // run records: one per (row, chunk) with elements of the row in the chunk's pairs
        const uint64_t hc = (hl + 127) & ~uint64_t(127), lf = L & ~uint64_t(127);
        for (uint64_t r = 0; r < fp.n; r++) {
          const uint64_t fs = std::max<uint64_t>(hl + r * f.row_bytes, hc);
          const uint64_t fe = std::min<uint64_t>(hl + (r + 1) * f.row_bytes, lf);
          if (fs < fe) P->fused_records += ((fe - 1) >> 10) - (fs >> 10) + 1;
        }
      }
    } else {
      plain.add((uint32_t)i, (nck + kRun - 1) / kRun);
    }
    nc += nck;
    P->bytes += L;
  }
  P->n_chunks = nc;
  P->n_fused = (uint32_t)fdesc.size();
  if (headbytes.size() / 4 >= 0xFFFFFFFFull) {
    delete P;
    return POTS_E_ARG;
  }

  if (!plain.finish() || !fused.finish()) {
    delete P;
    return POTS_E_ARG;
  }

  // Reduction folds of kFold levels each. Level 0 nodes of leaf i sit at desc[i].cv_first in
  // cv0; a fold takes a leaf's n nodes to ceil(n / 2^kFold) (BLAKE3's halving with a
  // promoted odd node, kFold times, composes to that ceiling).
  std::vector<LevelEntry> ents;
  std::vector<uint32_t> blk_ent;
  std::vector<uint64_t> n_nodes(n), off(n);
  for (size_t i = 0; i < n; i++) {
    n_nodes[i] = desc[i].n_chunks;
    off[i] = desc[i].cv_first;
  }
  uint64_t cv1_need = 0;
  int in_buf = 0;
  for (;;) {
    LevelInfo li{ents.size(), 0, 0, blk_ent.size(), in_buf, 1 - in_buf};
    uint64_t out_next = 0;
    for (size_t i = 0; i < n; i++) {
      if (n_nodes[i] < 2) continue;
      const uint64_t nout = (n_nodes[i] + (1u << kFold) - 1) >> kFold;
      LevelEntry e;
      e.in_off = off[i];
      e.out_off = out_next;
      e.out_first = li.n_out;
      e.n_in = (uint32_t)n_nodes[i];
      e.leaf = (uint32_t)i;
      ents.push_back(e);
      li.n_out += nout;
      li.n_ents++;
      off[i] = out_next;
      n_nodes[i] = nout;
      out_next += nout;
    }
    if (li.n_ents == 0) break;
    // Per block of kThreads outputs: the fold-relative index of the entry holding its first
    // output, and a closing bound.
    const uint64_t nb = (li.n_out + kThreads - 1) / kThreads;
    uint32_t k = 0;
    for (uint64_t b = 0; b < nb; b++) {
      const uint64_t first_out = b * kThreads;
      while (k + 1 < li.n_ents && ents[li.ent_first + k + 1].out_first <= first_out) k++;
      blk_ent.push_back(k);
    }
    blk_ent.push_back(li.n_ents - 1);
    if (li.out_buf == 1) cv1_need = std::max(cv1_need, out_next);
    P->levels.push_back(li);
    in_buf = 1 - in_buf;
  }

  // One allocation: [metadata | head table | cv0 | cv1 | staging].
  size_t at = 0;
  auto place = [&](size_t bytes) {
    size_t a = at;
    at = align_up(at + bytes, 256);
    return a;
  };
  const size_t o_leaves = place(n * sizeof(LeafDesc));
  const size_t o_fuse = place(std::max<size_t>(fdesc.size(), 1) * sizeof(FuseDesc));
  size_t o_ord[2][3];
  OrderHost* ords[2] = {&plain, &fused};
  for (int k = 0; k < 2; k++) {
    o_ord[k][0] = place(ords[k]->first.size() * sizeof(uint64_t));
    o_ord[k][1] = place(std::max<size_t>(ords[k]->leaf.size(), 1) * sizeof(uint32_t));
    o_ord[k][2] = place(ords[k]->blk_ent.size() * sizeof(uint32_t));
  }
  const size_t o_head = place(std::max<size_t>(headbytes.size(), 4));
  const size_t o_lev = place(std::max<size_t>(ents.size(), 1) * sizeof(LevelEntry));
  const size_t o_blk_ent = place(std::max<size_t>(blk_ent.size(), 1) * sizeof(uint32_t));
  const size_t meta_bytes = at;
  const size_t o_cv0 = place(nc * 32);
  const size_t o_cv1 = place(std::max<uint64_t>(cv1_need, 1) * 32);
  const size_t o_stage = place(std::max<uint64_t>(stage_bytes, 16));
  P->total = at;

  int rc;
  if (ext_base) {  // memory the caller holds (the allocation-free entry point's scratch)
    if (P->total > ext_cap) {
      note_error("leaf hashing needs " + std::to_string(P->total) + " bytes of device scratch "
                 "for these leaves; the allocation-free entry point holds " +
                 std::to_string(ext_cap));
      delete P;
      return POTS_E_ARG;
    }
    P->owned = false;
    P->base = ext_base;
  } else if (owned) {
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&P->base), P->total);
    if (e != hipSuccess) {
      note_hip_error(e, "hipMalloc(leaf plan)", __FILE__, __LINE__);
      delete P;
      return e == hipErrorOutOfMemory ? POTS_E_NOMEM : POTS_E_HIP;
    }
  } else {
    void* p = nullptr;
    if ((rc = arena_get(0, P->total, &p)) != POTS_E_OK) {
      delete P;
      return rc;
    }
    P->base = static_cast<char*>(p);
  }
  const uint64_t B = reinterpret_cast<uint64_t>(P->base);
  for (size_t i = 0, s = 0; i < n; i++) {
    if (stage_head_at[i] >= 0) {
      desc[i].payload = B + o_stage + stage_off[i];
      StageCopy& sc = P->stages[s++];
      sc.dst = B + o_stage + sc.dst;
      sc.head_src = B + o_head + sc.head_src;
    }
  }
  P->d_leaves = reinterpret_cast<LeafDesc*>(P->base + o_leaves);
  P->d_fuse = reinterpret_cast<FuseDesc*>(P->base + o_fuse);
  Order* dords[2] = {&P->plain, &P->fused};
  for (int k = 0; k < 2; k++) {
    dords[k]->first = reinterpret_cast<const uint64_t*>(P->base + o_ord[k][0]);
    dords[k]->leaf = reinterpret_cast<const uint32_t*>(P->base + o_ord[k][1]);
    dords[k]->blk_ent = reinterpret_cast<const uint32_t*>(P->base + o_ord[k][2]);
    dords[k]->n_slots = ords[k]->n_slots;
    dords[k]->n_blocks = ords[k]->n_blocks;
  }
  P->d_head = reinterpret_cast<uint32_t*>(P->base + o_head);
  P->d_levels = reinterpret_cast<LevelEntry*>(P->base + o_lev);
  P->d_blk_ent = reinterpret_cast<uint32_t*>(P->base + o_blk_ent);
  P->d_cv[0] = reinterpret_cast<uint32_t*>(P->base + o_cv0);
  P->d_cv[1] = reinterpret_cast<uint32_t*>(P->base + o_cv1);

  // The fused products' run records, allocated by the Freivalds plan.
  if (!fdesc.empty()) {
    std::vector<uint64_t> segs;
    const int frc = fv_fuse_commit(fv, fprod, fhead, &segs);
    if (frc != POTS_E_OK) {
      if (owned) (void)hipFree(P->base);
      delete P;
      return frc;
    }
    for (size_t f = 0; f < fdesc.size(); f++) fdesc[f].seg = segs[f];
  }

  // Upload the metadata in one copy.
  std::vector<char> img(meta_bytes, 0);
  memcpy(img.data() + o_leaves, desc.data(), n * sizeof(LeafDesc));
  if (!fdesc.empty()) memcpy(img.data() + o_fuse, fdesc.data(), fdesc.size() * sizeof(FuseDesc));
  for (int k = 0; k < 2; k++) {
    memcpy(img.data() + o_ord[k][0], ords[k]->first.data(),
           ords[k]->first.size() * sizeof(uint64_t));
    if (!ords[k]->leaf.empty())
      memcpy(img.data() + o_ord[k][1], ords[k]->leaf.data(),
             ords[k]->leaf.size() * sizeof(uint32_t));
    memcpy(img.data() + o_ord[k][2], ords[k]->blk_ent.data(),
           ords[k]->blk_ent.size() * sizeof(uint32_t));
  }
  if (!headbytes.empty()) memcpy(img.data() + o_head, headbytes.data(), headbytes.size());
  if (!ents.empty()) memcpy(img.data() + o_lev, ents.data(), ents.size() * sizeof(LevelEntry));
  if (!blk_ent.empty())
    memcpy(img.data() + o_blk_ent, blk_ent.data(), blk_ent.size() * sizeof(uint32_t));
  hipError_t e = hipMemcpy(P->base, img.data(), meta_bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    note_hip_error(e, "hipMemcpy(leaf plan metadata)", __FILE__, __LINE__);
    if (owned) (void)hipFree(P->base);
    delete P;
    return POTS_E_HIP;
  }
  *out = P;
  return POTS_E_OK;
}

// One stage of a plan's run: 0 staging copies and the first-bad reset, 1 the chunk kernel,
// 2 the per-leaf tree levels.
static int plan_stage(LeafPlan* P, int stage, uint32_t* d_digests, uint32_t* d_first_bad,
                      hipStream_t stream) {
  int rc;
  switch (stage) {
    case 0:
      for (const StageCopy& s : P->stages) {
        POTS_HIP(hipMemcpyAsync(reinterpret_cast<void*>(s.dst),
                                reinterpret_cast<const void*>(s.head_src), s.head_bytes,
                                hipMemcpyDeviceToDevice, stream));
        if (s.payload_bytes)
          POTS_HIP(hipMemcpyAsync(reinterpret_cast<void*>(s.dst + s.head_bytes),
                                  reinterpret_cast<const void*>(s.payload_src), s.payload_bytes,
                                  s.host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice,
                                  stream));
      }
      hipLaunchKernelGGL(fill_u32, dim3(1), dim3(1), 0, stream, d_first_bad, (uint32_t)P->n);
      POTS_HIP(hipGetLastError());
      return POTS_E_OK;
    case 1:  // both chunk kernels: the fused leaves' (3), then the others' (4)
      if ((rc = plan_stage(P, POTS_LEAF_STAGE_FUSED_CHUNKS, d_digests, d_first_bad, stream)) !=
          POTS_E_OK)
        return rc;
      return plan_stage(P, POTS_LEAF_STAGE_PLAIN_CHUNKS, d_digests, d_first_bad, stream);
    case POTS_LEAF_STAGE_FUSED_CHUNKS:
      if (P->fused.n_blocks) {
        const dim3 grid(P->max_grid ? std::min(P->max_grid, P->fused.n_blocks)
                                    : P->fused.n_blocks);
        switch (P->fuse_k) {
          case 1:
            hipLaunchKernelGGL(chunk_kernel_fused<1>, grid, dim3(kThreads), 0, stream,
                               P->d_leaves, P->d_fuse, P->fused, P->d_head, P->d_cv[0],
                               d_first_bad);
            break;
          case 2:
            hipLaunchKernelGGL(chunk_kernel_fused<2>, grid, dim3(kThreads), 0, stream,
                               P->d_leaves, P->d_fuse, P->fused, P->d_head, P->d_cv[0],
                               d_first_bad);
            break;
          case 4:
            hipLaunchKernelGGL(chunk_kernel_fused<4>, grid, dim3(kThreads), 0, stream,
                               P->d_leaves, P->d_fuse, P->fused, P->d_head, P->d_cv[0],
                               d_first_bad);
            break;
          default:
            return POTS_E_ARG;
        }
        POTS_HIP(hipGetLastError());
      }
      return POTS_E_OK;
    case POTS_LEAF_STAGE_PLAIN_CHUNKS:
      if (P->plain.n_blocks) {
        hipLaunchKernelGGL(chunk_kernel,
                           dim3(P->max_grid ? std::min(P->max_grid, P->plain.n_blocks)
                                            : P->plain.n_blocks),
                           dim3(kThreads), 0, stream, P->d_leaves, P->plain, P->d_head,
                           P->d_cv[0], d_digests, d_first_bad);
        POTS_HIP(hipGetLastError());
      }
      return POTS_E_OK;
    case 2:
      for (const LevelInfo& li : P->levels) {
        const uint64_t blocks = (li.n_out + kThreads - 1) / kThreads;
        hipLaunchKernelGGL(level_kernel, dim3((uint32_t)blocks), dim3(kThreads), 0, stream,
                           P->d_levels + li.ent_first, P->d_blk_ent + li.blk_first, li.n_out,
                           P->d_cv[li.in_buf], P->d_cv[li.out_buf], d_digests);
        POTS_HIP(hipGetLastError());
      }
      return POTS_E_OK;
    default:
      return POTS_E_ARG;
  }
}

static int plan_run(LeafPlan* P, uint32_t* d_digests, uint32_t* d_first_bad,
                    hipStream_t stream) {
  for (int stage = 0; stage < POTS_LEAF_STAGES; stage++) {
    const int rc = plan_stage(P, stage, d_digests, d_first_bad, stream);
    if (rc != POTS_E_OK) return rc;
  }
  return POTS_E_OK;
}

static void plan_free(LeafPlan* P) {
  if (!P) return;
  if (P->owned && P->base) (void)hipFree(P->base);
  delete P;
}

}  // namespace pots

using namespace pots;

extern "C" size_t pots_hash_leaves(size_t n, const uint8_t* hdr_buf, const uint64_t* hdr_off,
                                   const uint32_t* hdr_len, const uint32_t* hdr_idx,
                                   const uint64_t* payload_ptr, const uint64_t* payload_len,
                                   const uint8_t* kind, uint8_t* out, uint32_t n_threads) {
  (void)n_threads;
  if (n == 0) return 0;
  LeafPlan* P = nullptr;
  if (plan_build(n, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len, kind,
                 /*device_only=*/false, /*owned=*/false, nullptr, &P) != POTS_E_OK)
    return SIZE_MAX;
  void* res = nullptr;
  size_t bad = SIZE_MAX;
  if (arena_get(1, 32 * n + 16, &res) == POTS_E_OK) {
    uint32_t* d_dig = static_cast<uint32_t*>(res);
    uint32_t* d_bad = reinterpret_cast<uint32_t*>(static_cast<char*>(res) + 32 * n);
    uint32_t h_bad = 0;
    if (plan_run(P, d_dig, d_bad, 0) == POTS_E_OK) {
      hipError_t e = hipMemcpy(out, d_dig, 32 * n, hipMemcpyDeviceToHost);
      if (e == hipSuccess) e = hipMemcpy(&h_bad, d_bad, 4, hipMemcpyDeviceToHost);
      if (e == hipSuccess) bad = h_bad;
      else note_hip_error(e, "hipMemcpy(digests)", __FILE__, __LINE__);
    }
  }
  plan_free(P);
  return bad;
}

// ---- the allocation-free variant of pots_hash_leaves ----------------------------------------

// Device scratch of pots_hash_leaves_noalloc: the results (32 B per leaf and the first-bad
// word), then the plan (leaf descriptors, chaining values, staged messages). Each GPU the
// library runs on holds its own copy until the process ends.
constexpr size_t kNoallocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {
std::mutex g_scratch_mu;  // one call at a time per process: every call shares the array
char* g_scratch_ptr[64] = {};

// The array's device address on the current GPU, looked up once per device with that device
// current. Host code passes this address, never the symbol itself.
int scratch_address(char** out) {
  int dev = 0;
  POTS_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return POTS_E_ARG;
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      note_hip_error(e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
      return POTS_E_HIP;
    }
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  *out = g_scratch_ptr[dev];
  return POTS_E_OK;
}
}  // namespace

extern "C" size_t pots_hash_leaves_noalloc(size_t n, const uint8_t* hdr_buf,
                                           const uint64_t* hdr_off, const uint32_t* hdr_len,
                                           const uint32_t* hdr_idx, const uint64_t* payload_ptr,
                                           const uint64_t* payload_len, const uint8_t* kind,
                                           uint8_t* out, uint32_t n_threads) {
  (void)n_threads;
  if (n == 0) return 0;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  char* base = nullptr;
  if (scratch_address(&base) != POTS_E_OK) return SIZE_MAX;
  const size_t res_bytes = align_up(32 * n + 16, 256);
  if (res_bytes >= kNoallocScratchBytes) {
    note_error(std::to_string(n) + " leaves need " + std::to_string(res_bytes) + " bytes of "
               "results; the allocation-free entry point's scratch holds " +
               std::to_string(kNoallocScratchBytes));
    return SIZE_MAX;
  }
  LeafPlan* P = nullptr;
  if (plan_build(n, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len, kind,
                 /*device_only=*/false, /*owned=*/false, nullptr, &P, base + res_bytes,
                 kNoallocScratchBytes - res_bytes) != POTS_E_OK)
    return SIZE_MAX;
  uint32_t* d_dig = reinterpret_cast<uint32_t*>(base);
  uint32_t* d_bad = reinterpret_cast<uint32_t*>(base + 32 * n);
  size_t bad = SIZE_MAX;
  uint32_t h_bad = 0;
  if (plan_run(P, d_dig, d_bad, 0) == POTS_E_OK) {
    hipError_t e = hipMemcpy(out, d_dig, 32 * n, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(&h_bad, d_bad, 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess) bad = h_bad;
    else note_hip_error(e, "hipMemcpy(digests)", __FILE__, __LINE__);
  }
  plan_free(P);  // host bookkeeping only: the plan's memory is the scratch
  return bad;
}

extern "C" int pots_leaf_plan_create(size_t n, const uint8_t* hdr_buf, const uint64_t* hdr_off,
                                     const uint32_t* hdr_len, const uint32_t* hdr_idx,
                                     const uint64_t* payload_ptr, const uint64_t* payload_len,
                                     const uint8_t* kind, void** plan) {
  if (!plan) return POTS_E_ARG;
  LeafPlan* P = nullptr;
  int rc = plan_build(n, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len, kind,
                      /*device_only=*/true, /*owned=*/true, nullptr, &P);
  if (rc == POTS_E_OK) *plan = P;
  return rc;
}

extern "C" int pots_leaf_plan_create_fused(size_t n, const uint8_t* hdr_buf,
                                           const uint64_t* hdr_off, const uint32_t* hdr_len,
                                           const uint32_t* hdr_idx, const uint64_t* payload_ptr,
                                           const uint64_t* payload_len, const uint8_t* kind,
                                           void* fv_plan, void** plan) {
  if (!plan || !fv_plan) return POTS_E_ARG;
  LeafPlan* P = nullptr;
  int rc = plan_build(n, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len, kind,
                      /*device_only=*/true, /*owned=*/true, fv_plan, &P);
  if (rc == POTS_E_OK) *plan = P;
  return rc;
}

extern "C" uint32_t pots_leaf_plan_fused(const void* plan) {
  return plan ? static_cast<const LeafPlan*>(plan)->n_fused : 0;
}

extern "C" int pots_leaf_plan_fused_stats(const void* plan, uint64_t* msg_bytes,
                                          uint64_t* chunks, uint64_t* records) {
  if (!plan || !msg_bytes || !chunks || !records) return POTS_E_ARG;
  const LeafPlan* P = static_cast<const LeafPlan*>(plan);
  *msg_bytes = P->fused_msg;
  *chunks = P->fused_chunks;
  *records = P->fused_records;
  return POTS_E_OK;
}

extern "C" int pots_step_run(void* leaf_plan, void* fv_plan, const uint8_t* d_key,
                             uint8_t* d_digests, uint32_t* d_first_bad, double* d_rows,
                             void* stream) {
  if (!leaf_plan || !fv_plan || !d_key || !d_digests || !d_first_bad || !d_rows)
    return POTS_E_ARG;
  int rc;
  if ((rc = pots_fv_plan_run_stage(fv_plan, 0, d_key, d_rows, stream)) != POTS_E_OK) return rc;
  for (int st = 0; st < POTS_LEAF_STAGES; st++)
    if ((rc = pots_leaf_plan_run_stage(leaf_plan, st, d_digests, d_first_bad, stream)) !=
        POTS_E_OK)
      return rc;
  for (int st = 1; st < POTS_FV_STAGES; st++)
    if ((rc = pots_fv_plan_run_stage(fv_plan, st, d_key, d_rows, stream)) != POTS_E_OK)
      return rc;
  return POTS_E_OK;
}

extern "C" int pots_leaf_plan_run(void* plan, uint8_t* d_out, uint32_t* d_first_bad,
                                  void* stream) {
  if (!plan || !d_out || !d_first_bad) return POTS_E_ARG;
  return plan_run(static_cast<LeafPlan*>(plan), reinterpret_cast<uint32_t*>(d_out),
                  d_first_bad, static_cast<hipStream_t>(stream));
}

extern "C" int pots_leaf_plan_run_stage(void* plan, int stage, uint8_t* d_out,
                                        uint32_t* d_first_bad, void* stream) {
  if (!plan || !d_out || !d_first_bad || stage < 0 ||
      stage > POTS_LEAF_STAGE_PLAIN_CHUNKS)
    return POTS_E_ARG;
  return plan_stage(static_cast<LeafPlan*>(plan), stage, reinterpret_cast<uint32_t*>(d_out),
                    d_first_bad, static_cast<hipStream_t>(stream));
}

extern "C" int pots_leaf_plan_set_grid(void* plan, uint32_t max_blocks) {
  if (!plan) return POTS_E_ARG;
  static_cast<LeafPlan*>(plan)->max_grid = max_blocks;
  return POTS_E_OK;
}

extern "C" uint64_t pots_leaf_plan_chunks(const void* plan) {
  return plan ? static_cast<const LeafPlan*>(plan)->n_chunks : 0;
}

extern "C" uint64_t pots_leaf_plan_bytes(const void* plan) {
  return plan ? static_cast<const LeafPlan*>(plan)->bytes : 0;
}

extern "C" void pots_leaf_plan_destroy(void* plan) { plan_free(static_cast<LeafPlan*>(plan)); }
