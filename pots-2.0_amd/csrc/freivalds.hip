// Batched Freivalds measurement of every captured matmul on gfx950.
//
// Reference: verification/verifier/matmul_check/freivalds.py:255-321 (ROW, measure_product_row)
// and :384-410 (measure_products_rows). For each product P = A·B (+ 1·bᵀ), k challenge columns
// R [w, k] keyed on the claimed root, the row is
//   [ ‖|A|(|B|1) (+‖b‖₁)‖, ‖|P|1‖, ‖P‖_F, Σ_i (A²(B²1))_i, ‖b‖², ‖A(BR_j) (+bᵀR_j) − PR_j‖_j ]
// in fp64, the matvec and matmul outputs being fp32 as in the reference and every norm summed
// in fp64 (squares of fp32 values neither overflow nor underflow in fp64, which gives the
// reference's scaled-norm semantics without the scaling).
//
// Three streaming passes read each operand once from HBM. Each pass is the same kernel,
// "row pass": for a matrix X [rows, cols] and V [cols, k] it computes, per row,
//   dot = X·V (k values), s1 = Σ|x|·u, s2 = Σ x²·w     (u, w per-column weights, or ones)
//   B pass: X = B, V = R      -> B·R, |B|·1, B²·1
//   A pass: X = A, V = B·R    -> A·(B·R), |A|·(|B|·1), A²·(B²·1)
//   P pass: X = P, V = R      -> P·R, |P|·1, P²·1 (fp64)
//
// Work split. A block is 4 waves over 64 consecutive rows (16 per wave) and one column chunk
// of at most 4096 columns; consecutive blocks take consecutive row groups of the same chunk,
// so the chunk's V stays in each XCD's L2 while its row groups stream. Each lane (g, i) of a
// wave reads row i: 16 contiguous bytes at columns c + PER·g of every K-step c (PER = 8 bf16
// or 4 fp32), KU = 4 K-steps per pipeline stage, so a stage reads 256 contiguous bytes of
// each of the wave's 16 rows, and the loads of stage s+1 are in flight while stage s is
// multiplied.
//
// X·V runs on the matrix cores. The lane's K index inside a K-step is a permutation of the
// MFMA's, applied identically to V. bf16 X uses v_mfma_f32_16x16x16_bf16 with V as three
// exact bf16 terms (hi + mid + lo == the fp32 value) placed in separate output columns: a
// group of 16 MFMA columns holds 5 challenge columns x 3 terms (slot 3·jl + term), and the
// three terms' fp32 results are added after the loop. fp32 X uses v_mfma_f32_16x16x4_f32
// with V in fp32, 16 challenge columns per group. A block computes NJG groups at once, so X
// is read once for k <= 5·NJG (bf16) or 16·NJG (fp32).
//
// V, packed per K-group of PER columns: the 16 slots of group jg for K-group G occupy 256
// bytes at ((G · n_jg + jg) · 16 + slot) · 16, each slot holding PER consecutive rows of V
// (bf16 terms, or fp32). Rows past the matrix and unused slots are zero.
//
// The two sums are VALU work on the loaded registers; the A pass's weights u, w are staged in
// LDS once per block. Columns are split into chunks whose partial sums are reduced in a fixed
// order later, so every product yields enough blocks and no result depends on timing.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "freivalds.h"
#include "gmem.h"

namespace pots {

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef float v4f32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

enum : uint32_t { DT_F32 = 0, DT_BF16 = 1 };

constexpr uint32_t kRowsPerBlock = 64;  // 4 waves x 16 rows

// K-steps per pipeline stage of the row pass.
#ifndef POTS_FV_KU
#define POTS_FV_KU 4
#endif
constexpr uint32_t KU = POTS_FV_KU;

template <uint32_t XT>
struct Geo;
// CHUNK: columns per chunk at most. A chunk's dot products accumulate in fp32 on the matrix
// cores, one K-step after another, and chunks are added in fp64; 1024 fp32 columns keep that
// rounding below the reference's own fp32 matvec error (about one band unit at q ~ 8000).
// The A pass's weights of a chunk sit in LDS (2 x 4 x CHUNK bytes).
template <>
struct Geo<DT_BF16> {
  static constexpr uint32_t KSTEP = 32, PER = 8, ESZ = 2, CHUNK = 4096;
};
template <>
struct Geo<DT_F32> {
  static constexpr uint32_t KSTEP = 16, PER = 4, ESZ = 4, CHUNK = 1024;
};

// One matrix of one pass.
struct PassJob {
  uint64_t x;           // X[0][0]
  uint64_t ld;          // row stride in elements
  uint64_t v;           // packed V of this job
  uint64_t u, w;        // per-column weights (fp32 [cols]) or 0 for ones
  uint64_t pdot;        // partial X·V: float [n_chunks][rows_pad][k]
  uint64_t pabs;        // partial Σ|x|u: float [n_chunks][rows_pad]
  uint64_t psq;         // partial Σx²w: double [n_chunks][rows_pad]
  uint32_t rows, cols;
  uint32_t rows_pad, chunk_cols;
  uint32_t n_chunks, n_rg;  // column chunks; 64-row groups
  uint32_t n_jg, n_jt;      // 16-slot column groups; blocks per (row group, chunk)
  uint64_t block_first;     // prefix of blocks over the launch's jobs before it
  uint32_t aligned;         // 16-byte aligned rows and base
  uint32_t pack;            // a B-pass job of one column chunk for a bf16 A pass: bit 0, the
                            // pass writes the reduction's outputs itself (vout, uo, wo) in
                            // place of partials; bit 1, also b1's terms in slots 12..14
  uint64_t vout, uo, wo;    // with pack: packed B·R for the A pass, b1 = |B|·1, b2 = B²·1
};
static_assert(sizeof(PassJob) == 136, "PassJob layout");

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Lane i + N's value within lane i's row of 16 lanes (a DPP row shift on the VALU, no LDS
// round trip); lanes whose i + N leaves the row read their own value, and no caller uses them.
template <int N>
__device__ __forceinline__ float row_next(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                               __builtin_bit_cast(int, v),
                                                               0x100 + N, 0xF, 0xF, false));
}

template <bool SQ64>
struct SqAcc;
template <>
struct SqAcc<true> {
  double v = 0.0;
  __device__ void add(float x, float w) { v = fma((double)x * (double)x, (double)w, v); }
  __device__ void add1(float x) { v = fma((double)x, (double)x, v); }
  __device__ double get() const { return v; }
};
template <>
struct SqAcc<false> {
  float v = 0.0f;
  __device__ void add(float x, float w) { v = fmaf(x * x, w, v); }
  __device__ void add1(float x) { v = fmaf(x, x, v); }
  __device__ double get() const { return (double)v; }
};

// ---- the row pass ---------------------------------------------------------------------------

// A stage of a wave's X: KU K-steps, lane (g, i) holding row i's 8 (bf16) or 4 (fp32) columns
// of K-group g of each; and, unless the block shares V (VS), the lane's own V: slot i of
// K-group g of each K-step, for each of the NJG groups.
template <uint32_t NJG, bool VS>
struct StageRegs {
  u32x4 x[KU];
  u32x4 v[VS ? 1 : KU][VS ? 1 : NJG];
};

// Sharing V (VS): the block's four waves multiply the same columns by the same V, so each
// stage's V (NJG groups of 16 slots for each of the stage's 4·KU K-groups) is loaded once per
// block, every thread taking kPer of its 16-byte units, and written to one of two LDS stage
// buffers, from which each wave reads its lanes' slots. Loaded by every wave, V was four times
// the block's X traffic through L2 at k = 16, and the row passes ran at 37% of HBM. It costs
// a barrier per stage, which holds the four waves together: a pass with a full grid (a block
// per tile, many blocks on each CU) shares V; a pass limited to a block or two per CU, beside
// the hashing kernels, loads it per lane (measured at C4: the B pass 3.56 → 3.25 ms sharing;
// the A row pass at one block per CU 2.4-2.8 → 4.15 ms sharing, so it does not).
template <uint32_t NJG>
struct VStage {
  static constexpr uint32_t kUnits = 64 * KU * NJG;  // 16-byte units of one stage's V
  static constexpr uint32_t kPer = (kUnits + 255) / 256;
  u32x4 v[kPer];
};

// The per-lane view of one tile: X row, weights and bounds. The full stages' X loads address
// memory as a wave-uniform base, advanced in scalar registers from K-step to K-step, plus a
// per-lane 32-bit offset fixed for the tile, so most of the per-K-step address arithmetic is
// scalar work.
struct Lane {
  const char* xrow;   // this lane's X row (clamped to the matrix)
  const char* vlane;  // V slot of this lane for K-group g of group jt·NJG
  const char* xbase;  // wave-uniform: the wave's first X row, column 0
  const char* vjt;    // wave-uniform: V of K-group 0, group jt·NJG, slot 0
  uint64_t vstep;     // bytes of V per K-group
  uint32_t xoff;      // this lane's X bytes past xbase (its row, its 8 or 4 columns)
  uint32_t voff;      // this lane's V bytes past vjt (its K-group, its slot)
  uint32_t g, c1;
  uint32_t nvalid;    // groups of this block that exist (the last block of a row may hold fewer)
  bool kaligned;      // an aligned job whose chunk ends on a K-step: its last partial stage
                      // takes load_partial
  brsrc xr, vr;       // buffer resources at xbase and vjt (the full and partial stages' and
                      // the V staging's loads)
};

// A whole stage of an aligned job, every column inside the chunk: plain 16-byte loads.
template <uint32_t XT, uint32_t NJG, bool VS>
__device__ __forceinline__ void load_full(StageRegs<NJG, VS>& r, const Lane& L, uint32_t cs) {
  using G = Geo<XT>;
#pragma unroll
  for (uint32_t u = 0; u < KU; u++) {
    const uint32_t cu = cs + u * G::KSTEP;
    r.x[u] = bload128(L.xr, L.xoff, cu * G::ESZ);
    if constexpr (!VS) {
      const uint32_t vb = (cu / G::PER) * (uint32_t)L.vstep;  // uniform
      // Every load is unconditional, so the compiler's wait counts stay exact across the
      // pipeline: a group past n_jg (only in a row's last column-group block) rereads the
      // last valid group, and its results are not stored.
#pragma unroll
      for (uint32_t q = 0; q < NJG; q++)
        r.v[u][q] = bload128(L.vr, L.voff, vb + (q < L.nvalid ? q : L.nvalid - 1) * 256);
    }
  }
}

// The last, partial stage of an aligned job's chunk whose columns end on a K-step (a narrow
// X, such as an attention head's 64 columns, is one such stage per row): K-steps inside the
// chunk take one 16-byte load per lane, the rest read as zero, and so does the lane's own V
// of K-steps past c1 (V rows past the matrix are zero in memory).
template <uint32_t XT, uint32_t NJG, bool VS>
__device__ __forceinline__ void load_partial(StageRegs<NJG, VS>& r, const Lane& L,
                                             uint32_t cs) {
  using G = Geo<XT>;
#pragma unroll
  for (uint32_t u = 0; u < KU; u++) {
    const uint32_t cu = cs + u * G::KSTEP;
    r.x[u] = cu < L.c1 ? bload128(L.xr, L.xoff, cu * G::ESZ) : u32x4{0, 0, 0, 0};
    if constexpr (!VS) {
      const uint32_t vb = (cu / G::PER) * (uint32_t)L.vstep;  // uniform
#pragma unroll
      for (uint32_t q = 0; q < NJG; q++)
        r.v[u][q] = (q < L.nvalid && cu < L.c1) ? bload128(L.vr, L.voff, vb + q * 256)
                                                : u32x4{0, 0, 0, 0};
    }
  }
  // Wait for these loads here (s_waitcnt vmcnt(0)). Left in flight, they would reach the
  // merge with load_full's path, whose loads into the same registers the compiler would then
  // hold behind every earlier load (stage V's included) in every full stage, which is the
  // whole software pipeline.
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

// A stage that may run past the chunk's end across a K-step, or of an unaligned job: element
// loads with a column guard; columns past c1 read as zero, and so does the lane's own V of
// K-steps past c1 (V rows past the matrix are zero in memory).
template <uint32_t XT, uint32_t NJG, bool VS>
__device__ __forceinline__ void load_guarded(StageRegs<NJG, VS>& r, const Lane& L,
                                             uint32_t cs) {
  using G = Geo<XT>;
#pragma unroll
  for (uint32_t u = 0; u < KU; u++) {
    const uint32_t cu = cs + u * G::KSTEP;
    const uint32_t cl = cu + G::PER * L.g;
    if (XT == DT_BF16) {
      const uint16_t* p = reinterpret_cast<const uint16_t*>(L.xrow);
      uint32_t e[8];
#pragma unroll
      for (uint32_t t = 0; t < 8; t++) e[t] = cl + t < L.c1 ? gload<uint16_t>(p + cl + t) : 0u;
      r.x[u] = u32x4{e[0] | e[1] << 16, e[2] | e[3] << 16, e[4] | e[5] << 16, e[6] | e[7] << 16};
    } else {
      const uint32_t* p = reinterpret_cast<const uint32_t*>(L.xrow);
      uint32_t e[4];
#pragma unroll
      for (uint32_t t = 0; t < 4; t++) e[t] = cl + t < L.c1 ? gload<uint32_t>(p + cl + t) : 0u;
      r.x[u] = u32x4{e[0], e[1], e[2], e[3]};
    }
    if constexpr (!VS) {
      const char* vp = L.vlane + (uint64_t)(cu / G::PER) * L.vstep;
#pragma unroll
      for (uint32_t q = 0; q < NJG; q++)
        r.v[u][q] = (q < L.nvalid && cu < L.c1) ? gload<u32x4>(vp + q * 256) : u32x4{0, 0, 0, 0};
    }
  }
  // Waited for here, as in load_partial (the element loads above already wait one by one for
  // their guards' merges), so that no register of this loader stays pending past it.
  __builtin_amdgcn_s_waitcnt(0x0F70);
}

// This thread's units of the stage at column cs: unit n is slot n mod 16 of group
// (n / 16) mod NJG of the stage's K-group n / (16·NJG). A group past n_jg (only in a row's last
// column-group block) rereads the last valid group; its results are not stored. A K-step that
// starts past c1 (only in a partial stage) reads as zero, and V rows past the matrix are zero
// in memory.
template <uint32_t XT, uint32_t NJG>
__device__ __forceinline__ void vstage_load(VStage<NJG>& vs, const Lane& L, uint32_t cs) {
  using G = Geo<XT>;
  constexpr uint32_t GPS = G::KSTEP / G::PER;  // K-groups per K-step (4)
  const uint32_t v0 = (cs / G::PER) * (uint32_t)L.vstep;  // uniform
#pragma unroll
  for (uint32_t e = 0; e < VStage<NJG>::kPer; e++) {
    const uint32_t n = threadIdx.x + 256 * e;
    const uint32_t kg = n / (16 * NJG), q = (n / 16) % NJG, slot = n % 16;
    const uint32_t qv = q < L.nvalid ? q : L.nvalid - 1;
    const bool in = n < VStage<NJG>::kUnits && cs + (kg / GPS) * G::KSTEP < L.c1;
    vs.v[e] = in ? bload128(L.vr, kg * (uint32_t)L.vstep + qv * 256 + slot * 16, v0)
                 : u32x4{0, 0, 0, 0};
  }
}

template <uint32_t NJG>
__device__ __forceinline__ void vstage_store(const VStage<NJG>& vs, u32x4* sv) {
  // kUnits is a multiple of the block's 256 threads: every thread stores every one of its
  // units, with no lane mask (a masked store would let the staging loads reach the loop's back
  // edge unwaited on the path that skips it, and the compiler would then wait for every load
  // before the next stage's staging loads)
  static_assert(VStage<NJG>::kUnits % 256 == 0, "whole units per thread");
#pragma unroll
  for (uint32_t e = 0; e < VStage<NJG>::kPer; e++) sv[threadIdx.x + 256 * e] = vs.v[e];
}

// One stage: X from the wave's registers; V from the lanes' registers, or (VS) from the
// block's LDS stage buffer `sv`, where lane (g, i) finds K-group g of K-step u, group q, slot i
// at unit (4u + g)·16·NJG + 16q + i.
template <uint32_t XT, bool WEIGHTED, bool SQ64, uint32_t NJG, bool VS>
__device__ __forceinline__ void compute_stage(const StageRegs<NJG, VS>& r, const u32x4* sv,
                                              v4f32 acc[NJG], float& s1, SqAcc<SQ64>& s2,
                                              bool sums, const float* wu, const float* ww,
                                              uint32_t off, uint32_t g, uint32_t i) {
  using G = Geo<XT>;
#pragma unroll
  for (uint32_t u = 0; u < KU; u++) {
    u32x4 v[NJG];
#pragma unroll
    for (uint32_t q = 0; q < NJG; q++)
      v[q] = VS ? sv[((4 * u + g) * NJG + q) * 16 + i] : r.v[VS ? 0 : u][VS ? 0 : q];
    if (XT == DT_BF16) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const v4i16 a = __builtin_bit_cast(v4i16, v2u32{r.x[u][2 * h], r.x[u][2 * h + 1]});
#pragma unroll
        for (uint32_t q = 0; q < NJG; q++) {
          const v4i16 b = __builtin_bit_cast(v4i16, v2u32{v[q][2 * h], v[q][2 * h + 1]});
          acc[q] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc[q], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) {
#pragma unroll
        for (uint32_t q = 0; q < NJG; q++)
          acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(r.x[u][e]),
                                                        __uint_as_float(v[q][e]), acc[q],
                                                        0, 0, 0);
      }
    }
    if (sums) {
      float xs[G::PER];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if (XT == DT_BF16) {
          xs[2 * e] = bf_lo(r.x[u][e]);
          xs[2 * e + 1] = bf_hi(r.x[u][e]);
        } else {
          xs[e] = __uint_as_float(r.x[u][e]);
        }
      }
      if (WEIGHTED) {
        const uint32_t o = off + u * G::KSTEP;
        float uc[G::PER], wc[G::PER];
#pragma unroll
        for (uint32_t t = 0; t < G::PER; t += 4) {
          const v4f32 a = *reinterpret_cast<const v4f32*>(wu + o + t);
          const v4f32 b = *reinterpret_cast<const v4f32*>(ww + o + t);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            uc[t + e] = a[e];
            wc[t + e] = b[e];
          }
        }
#pragma unroll
        for (uint32_t t = 0; t < G::PER; t++) {
          s1 = fmaf(fabsf(xs[t]), uc[t], s1);
          s2.add(xs[t], wc[t]);
        }
      } else {
#pragma unroll
        for (uint32_t t = 0; t < G::PER; t++) {
          s1 += fabsf(xs[t]);
          s2.add1(xs[t]);
        }
      }
    }
  }
}

// The A pass's weights u, w of columns c0 .. c1 − 1 into LDS (zero up to chunk_cols): 16-byte
// loads, every one issued before the first store, so a tile waits for one load's latency
// here, not one per element. Chunk starts are whole pipeline stages (multiples of 64 columns)
// and the weights 256-byte aligned, so the vector loads are aligned.
template <uint32_t CHUNK>
__device__ __forceinline__ void stage_weights(uint64_t u, uint64_t w, uint32_t c0, uint32_t c1,
                                              uint32_t chunk_cols, float* s_u, float* s_w) {
  constexpr uint32_t NV = (CHUNK + 1023) / 1024;  // 4-column groups per thread
  const float* up = reinterpret_cast<const float*>(u) + c0;
  const float* wp = reinterpret_cast<const float*>(w) + c0;
  const uint32_t n = c1 - c0;
  v4f32 ua[NV], wa[NV];
#pragma unroll
  for (uint32_t v = 0; v < NV; v++) {
    const uint32_t t = 4 * (threadIdx.x + 256 * v);
    if (t + 4 <= n) {
      ua[v] = gload<v4f32>(up + t);
      wa[v] = gload<v4f32>(wp + t);
    } else {
#pragma unroll
      for (uint32_t e = 0; e < 4; e++) {
        ua[v][e] = t + e < n ? gload<float>(up + t + e) : 0.f;
        wa[v][e] = t + e < n ? gload<float>(wp + t + e) : 0.f;
      }
    }
  }
#pragma unroll
  for (uint32_t v = 0; v < NV; v++) {
    const uint32_t t = 4 * (threadIdx.x + 256 * v);
    if (t < chunk_cols) {
      *reinterpret_cast<v4f32*>(s_u + t) = ua[v];
      *reinterpret_cast<v4f32*>(s_w + t) = wa[v];
    }
  }
}

// The twin pass's one weight w of columns c0 .. c1 − 1 into LDS, as stage_weights stages two
// (c1 − c0 ≤ CHUNK; the twin pass reads no column past c1).
template <uint32_t CHUNK>
__device__ __forceinline__ void stage_weight(uint64_t w, uint32_t c0, uint32_t c1, float* s_w) {
  constexpr uint32_t NV = (CHUNK + 1023) / 1024;  // 4-column groups per thread
  const float* wp = reinterpret_cast<const float*>(w) + c0;
  const uint32_t n = c1 - c0;
  v4f32 wa[NV];
#pragma unroll
  for (uint32_t v = 0; v < NV; v++) {
    const uint32_t t = 4 * (threadIdx.x + 256 * v);
    if (t + 4 <= n) {
      wa[v] = gload<v4f32>(wp + t);
    } else {
#pragma unroll
      for (uint32_t e = 0; e < 4; e++) wa[v][e] = t + e < n ? gload<float>(wp + t + e) : 0.f;
    }
  }
#pragma unroll
  for (uint32_t v = 0; v < NV; v++) {
    const uint32_t t = 4 * (threadIdx.x + 256 * v);
    if (t < CHUNK) *reinterpret_cast<v4f32*>(s_w + t) = wa[v];
  }
}

// One tile: job blk_job[bidx], 64-row group, column chunk and column-group block decoded
// from its index within the job (row group fastest). Every wave of the block calls it with the
// same tile and reaches its barrier.
// A B-pass job of one column chunk writes what the reduction (reduce_b) would make of its one
// chunk of partials, the same values bit for bit: for each 8-row group and challenge j, B·R's
// three exact bf16 terms in slots 3(j mod 5) .. of the group's column group j / 5 (rows past
// the matrix zero; groups wholly past it are never written, and the plan zeroed them when it
// was built), and from the first column-group block, b1 = Σ|x| and b2 = Σx² per row (b1's
// terms in slots 12..14 too, for a twin's A pass). Lane (g, i) holds rows 4g + e (e < 4) of the
// wave's 16 rows; a lane with g even takes rows 4g + 4 .. from lane + 16.
template <uint32_t NJG>
__device__ __forceinline__ void pack_b_rows(const PassJob& J, const v4f32 (&acc)[NJG],
                                            uint32_t jt, uint32_t k, uint32_t r0,
                                            uint32_t lane, uint32_t g, uint32_t i,
                                            uint32_t nvalid, float s1, double s2, bool sums) {
  uint16_t* vo = reinterpret_cast<uint16_t*>(J.vout);
  const uint32_t g3 = groups_b3(k);
  const uint32_t rb = r0 + 4 * g;  // the first of a lane's 8 rows when g is even
  auto put = [&](uint16_t* dst, const float (&x)[8]) {
    uint16_t pl[3][8];
#pragma unroll
    for (int t = 0; t < 8; t++) split_bf16x3(x[t], pl[0][t], pl[1][t], pl[2][t]);
#pragma unroll
    for (int p = 0; p < 3; p++)
      gstore<u32x4>(dst + 8 * p, u32x4{pl[p][0] | (uint32_t)pl[p][1] << 16,
                                       pl[p][2] | (uint32_t)pl[p][3] << 16,
                                       pl[p][4] | (uint32_t)pl[p][5] << 16,
                                       pl[p][6] | (uint32_t)pl[p][7] << 16});
  };
#pragma unroll
  for (uint32_t q = 0; q < NJG; q++) {
    const uint32_t jg = jt * NJG + q;
    float val[4], oth[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float v0 = acc[q][e];
      const float v1 = __shfl(v0, (int)lane + 1);
      const float v2 = __shfl(v0, (int)lane + 2);
      val[e] = (v0 + v1) + v2;  // the partial the reduction would read, as the pass makes it
    }
#pragma unroll
    for (int e = 0; e < 4; e++) oth[e] = __shfl(val[e], (int)lane + 16);
    const uint32_t j = 5 * jg + i / 3;
    if ((g & 1) == 0 && i % 3 == 0 && i < 15 && q < nvalid && j < k && rb < J.rows) {
      float x[8];
#pragma unroll
      for (int t = 0; t < 8; t++)
        x[t] = rb + t < J.rows ? (t < 4 ? val[t] : oth[t - 4]) : 0.f;
      put(vo + (((uint64_t)(rb / 8) * g3 + j / 5) * 16 + 3 * (j % 5)) * 8, x);
    }
  }
  if (!sums) return;
  float a = s1;
  float qf = (float)s2;  // the B pass takes Σx² in fp32 (SqAcc<false>)
  qf += __shfl_xor(qf, 16);
  qf += __shfl_xor(qf, 32);
  a += __shfl_xor(a, 16);
  a += __shfl_xor(a, 32);
  const uint32_t row = r0 + i;
  if (g == 0 && row < J.rows) {
    gstore<float>(reinterpret_cast<float*>(J.uo) + row, a);
    gstore<float>(reinterpret_cast<float*>(J.wo) + row, qf);
  }
  if (J.pack & 2) {
    float x[8];
#pragma unroll
    for (int t = 0; t < 8; t++) x[t] = __shfl(a, (int)(lane & ~7u) + t);
    if (g == 0 && (i & 7) == 0 && row < J.rows) {
#pragma unroll
      for (int t = 0; t < 8; t++)
        if (row + t >= J.rows) x[t] = 0.f;
      put(vo + ((uint64_t)(row / 8) * 16 + 12) * 8, x);
    }
  }
}

template <uint32_t XT, bool WEIGHTED, bool SQ64, uint32_t NJG, bool VS>
__device__ __forceinline__ void row_tile(const PassJob* __restrict__ jobs,
                                         const uint32_t* __restrict__ blk_job, uint32_t k,
                                         uint32_t bidx, float* s_u, float* s_w, u32x4* s_v) {
  using G = Geo<XT>;
  constexpr uint32_t SSTEP = G::KSTEP * KU;
  // The wave index is uniform; readfirstlane lets the compiler keep everything derived from
  // it in scalar registers, so the loop has no divergent branches.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  const PassJob J = jobs[blk_job[bidx]];
  uint32_t local = bidx - (uint32_t)J.block_first;
  const uint32_t rg = local % J.n_rg;
  local /= J.n_rg;
  const uint32_t chunk = local % J.n_chunks;
  const uint32_t jt = local / J.n_chunks;
  const uint32_t c0 = chunk * J.chunk_cols;
  const uint32_t c1 = min(c0 + J.chunk_cols, J.cols);
  const bool sums = jt == 0;  // the two sums are taken once, by the first column-group block
  const uint32_t r0 = rg * kRowsPerBlock + wave * 16;
  const bool active = r0 < J.rows;  // waves past the matrix only take part in the staging
  const uint32_t g = lane >> 4, i = lane & 15;
  const uint32_t row = r0 + i;
  Lane L;
  // Rows past the matrix read its last row; their results are never written.
  const uint32_t rowc = row < J.rows ? row : J.rows - 1;
  L.xrow = reinterpret_cast<const char*>(J.x) + (uint64_t)rowc * J.ld * G::ESZ;
  L.vstep = (uint64_t)J.n_jg * 256;
  L.vjt = reinterpret_cast<const char*>(J.v) + (uint64_t)jt * NJG * 256;
  L.voff = (uint32_t)((uint64_t)g * L.vstep) + i * 16;
  L.vlane = L.vjt + L.voff;
  // the same addresses as uniform bases and 32-bit lane offsets (plan creation keeps 16 rows
  // of an aligned job's X below 2^31 bytes; 4 K-groups of V are far below)
  L.xbase = reinterpret_cast<const char*>(J.x) + (uint64_t)r0 * J.ld * G::ESZ;
  L.xoff = (uint32_t)((uint64_t)(rowc - r0) * J.ld * G::ESZ) + G::PER * g * G::ESZ;
  L.g = g;
  L.c1 = c1;
  L.nvalid = min(NJG, J.n_jg - jt * NJG);
  L.kaligned = J.aligned != 0 && (c1 - c0) % G::KSTEP == 0;
  L.xr = make_rsrc(L.xbase);
  L.vr = make_rsrc(L.vjt);
  // The chunk's stages: the first nfull of an aligned job are whole (plain 16-byte loads);
  // an aligned chunk's last partial stage takes load_partial when the chunk ends on a K-step,
  // else the guarded loads, which every stage of an unaligned job takes.
  const uint32_t nfull = J.aligned ? (c1 - c0) / SSTEP : 0;
  const uint32_t nst = (c1 - c0 + SSTEP - 1) / SSTEP;
  u32x4* const sv0 = s_v;
  u32x4* const sv1 = s_v + VStage<NJG>::kUnits;

  // The first stage's X and V loads go out before the weights are staged, so the latencies
  // overlap. Waves past the matrix take part in the staging and the barriers only.
  StageRegs<NJG, VS> ra, rb;
  VStage<NJG> vs;
  if constexpr (VS) vstage_load<XT, NJG>(vs, L, c0);
  if (active) {
    if (nfull > 0) load_full<XT, NJG, VS>(ra, L, c0);
    else if (L.kaligned) load_partial<XT, NJG, VS>(ra, L, c0);
    else load_guarded<XT, NJG, VS>(ra, L, c0);
  }
  if (WEIGHTED && sums) stage_weights<G::CHUNK>(J.u, J.w, c0, c1, J.chunk_cols, s_u, s_w);
  if constexpr (VS) vstage_store<NJG>(vs, sv0);
  if (WEIGHTED || VS) __syncthreads();
  if (!VS && !active) return;

  v4f32 acc[NJG];
#pragma unroll
  for (uint32_t q = 0; q < NJG; q++) acc[q] = v4f32{0.f, 0.f, 0.f, 0.f};
  float s1 = 0.f;
  SqAcc<SQ64> s2;
  const uint32_t woff = G::PER * g - c0;  // LDS weight index = column - c0

  // Stage s is multiplied while stage s + 1's loads are in flight (a two-buffer software
  // pipeline). Sharing V, stage s reads LDS buffer s mod 2, stage s + 1's V goes to the other
  // buffer once stage s is computed, and one barrier per stage keeps each buffer's writers and
  // readers apart.
  auto step = [&](const StageRegs<NJG, VS>& cur, StageRegs<NJG, VS>& nxt, uint32_t s) {
    const uint32_t cs = c0 + s * SSTEP;
    const bool more = s + 1 < nst;
    // A path that issues no next-stage loads (the last stage; a wave past the matrix) waits
    // for its own loads at once: nothing else is in flight there, so it costs nothing, and
    // no registers of this stage stay pending into the next step's merge.
    if (more) {
      if constexpr (VS) vstage_load<XT, NJG>(vs, L, cs + SSTEP);
      if (active) {
        if (s + 1 < nfull) load_full<XT, NJG, VS>(nxt, L, cs + SSTEP);
        else if (L.kaligned) load_partial<XT, NJG, VS>(nxt, L, cs + SSTEP);
        else load_guarded<XT, NJG, VS>(nxt, L, cs + SSTEP);
      } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);
      }
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    if (active)
      compute_stage<XT, WEIGHTED, SQ64, NJG, VS>(cur, (s & 1) ? sv1 : sv0, acc, s1, s2, sums,
                                                 s_u, s_w, cs + woff, g, i);
    if constexpr (VS) {
      // Stored whether or not a next stage was loaded (after the last stage the registers are
      // stale and the buffer is not read again in this tile), for the same reason as the
      // unmasked stores in vstage_store.
      vstage_store<NJG>(vs, (s & 1) ? sv0 : sv1);
      __syncthreads();
    }
  };
  // With V per lane, pairs of stages whose next stage is whole run first, in a loop with no
  // branch around their loads. The compiler's wait counts ignore which way a branch went: in
  // the general step, its control flow for the choice of loader has a path (never taken) from
  // the loop header to the MFMAs that skips every load, along which this stage's own loads
  // are the newest, and every stage then waited for the next stage's first loads. (Sharing V,
  // the barrier between stages orders them already; the extra loop there cost registers and
  // occupancy, measured slower.)
  uint32_t s0 = 0;
  if constexpr (!VS) {
    auto step_full = [&](const StageRegs<NJG, VS>& cur, StageRegs<NJG, VS>& nxt, uint32_t s) {
      const uint32_t cs = c0 + s * SSTEP;
      load_full<XT, NJG, VS>(nxt, L, cs + SSTEP);
      compute_stage<XT, WEIGHTED, SQ64, NJG, VS>(cur, sv0, acc, s1, s2, sums, s_u, s_w,
                                                 cs + woff, g, i);
    };
    for (; s0 + 2 < nfull; s0 += 2) {
      step_full(ra, rb, s0);
      step_full(rb, ra, s0 + 1);
    }
  }
  for (uint32_t s = s0; s < nst; s += 2) {
    step(ra, rb, s);
    if (s + 1 < nst) step(rb, ra, s + 1);
  }
  if (!active) return;

  // X·V: lane (g, i) holds rows 4g + e of the wave's 16 and slot i of each group.
  float* pdot = reinterpret_cast<float*>(J.pdot);
  const uint64_t cbase = (uint64_t)chunk * J.rows_pad;
  if (XT == DT_BF16 && J.pack) {
    pack_b_rows<NJG>(J, acc, jt, k, r0, lane, g, i, L.nvalid, s1, s2.get(), sums);
    return;
  }
#pragma unroll
  for (uint32_t q = 0; q < NJG; q++) {
    const uint32_t jg = jt * NJG + q;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t orow = r0 + 4 * g + e;
      if (XT == DT_BF16) {
        // The three terms of challenge column jl sit in slots 3jl, 3jl + 1, 3jl + 2.
        const float v0 = acc[q][e];
        const float v1 = __shfl(v0, (int)lane + 1);
        const float v2 = __shfl(v0, (int)lane + 2);
        const uint32_t j = 5 * jg + i / 3;
        if (i % 3 == 0 && i < 15 && q < L.nvalid && j < k && orow < J.rows)
          gstore<float>(pdot + (cbase + orow) * k + j, (v0 + v1) + v2);
      } else {
        const uint32_t j = 16 * jg + i;
        if (q < L.nvalid && j < k && orow < J.rows)
          gstore<float>(pdot + (cbase + orow) * k + j, acc[q][e]);
      }
    }
  }
  if (sums) {
    float* pabs = reinterpret_cast<float*>(J.pabs);
    double* psq = reinterpret_cast<double*>(J.psq);
    float a = s1;
    double q = s2.get();
    if (!SQ64) {  // combine in the accumulation precision
      float qf = (float)q;
      qf += __shfl_xor(qf, 16);
      qf += __shfl_xor(qf, 32);
      q = qf;
    } else {
      q += __shfl_xor(q, 16);
      q += __shfl_xor(q, 32);
    }
    a += __shfl_xor(a, 16);
    a += __shfl_xor(a, 32);
    if (g == 0 && row < J.rows) {
      gstore<float>(pabs + cbase + row, a);
      gstore<double>(psq + cbase + row, q);
    }
  }
}

// One tile queue per XCD: queue x holds tiles [n·x/8, n·(x+1)/8), a contiguous range, so the
// tiles that share a column chunk's B·R and weights run on one XCD and find them in its L2
// (the GPU's 8 XCDs each have their own). A block works from its own XCD's queue, then from
// the others in turn.
constexpr uint32_t kQueues = 8;

__device__ __forceinline__ uint32_t queue_lo(uint32_t n, uint32_t x) {
  return (uint32_t)((uint64_t)n * x / kQueues);
}

// The XCD this wave runs on (hardware register XCC_ID); only a locality hint.
__device__ __forceinline__ uint32_t xcd_id() {
  return (uint32_t)__builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) % kQueues;
}

// The tiles of a launch, from the tile queues when the grid is limited, else one block per
// tile. With a smaller grid, the pass holds a bounded share of each CU (a block holds 4 waves
// and its LDS) so that a kernel on another stream (the leaf hasher) keeps the rest, and the
// blocks take tiles from the queues: counters (zero at launch) that each block's first thread
// advances by one per tile, a tile ahead of the one the block works on, moving to the next
// queue when one runs out. A block that lands on a CU shared with more hashing waves then
// takes fewer tiles, where a fixed split would leave it the last to finish. Every thread of a
// block reads the same tile index, so all of its waves leave the loop together once every
// queue is empty; each counter value below its range hands out one tile, so every tile is
// taken exactly once. `body(t)` is called by every thread of the block with the same t.
template <typename F>
__device__ __forceinline__ void tile_loop(uint32_t n_tiles, uint32_t* __restrict__ queue,
                                          uint32_t* s_tile, F&& body) {
  if (queue == nullptr) {
    if (blockIdx.x < n_tiles) body(blockIdx.x);
    return;
  }
  // Thread 0's state: the queues tried so far, from this XCD's own.
  const uint32_t home = xcd_id();
  uint32_t qi = 0;
  auto take = [&]() -> uint32_t {  // the next tile, or n_tiles once every queue is empty
    for (; qi < kQueues; qi++) {
      const uint32_t x = (home + qi) % kQueues;
      const uint32_t lo = queue_lo(n_tiles, x);
      const uint32_t t = atomicInc(queue + x, 0xFFFFFFFFu);
      if (t < queue_lo(n_tiles, x + 1) - lo) return lo + t;
    }
    return n_tiles;
  };
  if (threadIdx.x == 0) *s_tile = take();
  __syncthreads();
  uint32_t b = *s_tile;
  while (b < n_tiles) {
    // The next tile's counter value is taken now; its latency passes under this tile. (An
    // increment that wraps only at 2^32 − 1 is an add of one; written as atomicInc, the
    // compiler does not rewrite it into a wave-level add whose result it must wait for.)
    uint32_t next = 0;
    if (threadIdx.x == 0 && qi < kQueues)
      next = atomicInc(queue + (home + qi) % kQueues, 0xFFFFFFFFu);
    body(b);
    __syncthreads();  // every wave is done with this tile's LDS and has read s_tile
    if (threadIdx.x == 0) {
      uint32_t nb = n_tiles;
      if (qi < kQueues) {
        const uint32_t x = (home + qi) % kQueues;
        const uint32_t lo = queue_lo(n_tiles, x);
        if (next < queue_lo(n_tiles, x + 1) - lo) {
          nb = lo + next;
        } else {
          qi++;
          nb = take();
        }
      }
      *s_tile = nb;
    }
    __syncthreads();
    b = *s_tile;
  }
}

// The row pass over n_tiles tiles. With a block per tile (queue null), block b takes tile b
// (mapping blocks XCD by XCD, as the fused chunk kernel does, cut the B pass's reads 1.08x ->
// 1.02x but made it slower: with no stealing, XCDs given equal tile counts of unequal tiles
// finish apart). With a smaller grid the blocks take tiles from the queues (tile_loop).
template <uint32_t XT, bool WEIGHTED, bool SQ64, uint32_t NJG, bool VS>
__global__ __launch_bounds__(256) void row_pass(const PassJob* __restrict__ jobs,
                                                const uint32_t* __restrict__ blk_job,
                                                uint32_t k, uint32_t n_tiles,
                                                uint32_t* __restrict__ queue) {
  using G = Geo<XT>;
  __shared__ __align__(16) float s_u[WEIGHTED ? G::CHUNK : 4];
  __shared__ __align__(16) float s_w[WEIGHTED ? G::CHUNK : 4];
  __shared__ __align__(16) u32x4 s_v[VS ? 2 * VStage<NJG>::kUnits : 1];  // two stages of V
  __shared__ uint32_t s_tile;
  tile_loop(n_tiles, queue, &s_tile, [&](uint32_t b) {
    row_tile<XT, WEIGHTED, SQ64, NJG, VS>(jobs, blk_job, k, b, s_u, s_w, s_v);
  });
}

__global__ void queue_reset(uint32_t* q) {
  if (threadIdx.x < kQueues) q[threadIdx.x] = 0u;
}

// ---- twin pass: one read of an operand shared as A and Aᵀ ------------------------------
//
// Two products of a training step often share their A operand as X and Xᵀ: the attention
// probabilities are O's A and, transposed, dV's; δS is dQ's A and dK's; a linear layer's
// output gradient is its input gradient's A and its weight gradient's; the logits' gradient is
// dF's A and G_head's. The twin pass reads X once for both products: X·V₁ row by row (the A
// pass of m₁, A₁ = X) and Xᵀ·V₂ column by column (the A pass of m₂, A₂ = Xᵀ), with the sums
// of both, in one pass over X's tiles:
//   - the dot products X·V₁ and Xᵀ·V₂ on the matrix cores as in the row pass (V as three exact
//     bf16 terms);
//   - ν₂ = |Xᵀ|·u₂ on the matrix cores too, into m₂'s accumulators: u₂'s three exact bf16
//     terms sit in slots 12..14 of m₂'s packed operand (k ≤ 4 leaves them free);
//   - ν₁ = |X|·u₁ and Σx²w₁ per row on the VALU, from u₁ and w₁ staged in LDS;
//   - U₂ = Σ_r w₂(r)·Σ_c x_rc² from each lane's row sums of squares (v_dot2 on bf16 pairs,
//     exact in fp32). Only U's total enters the row, so each tile writes its total as one
//     partial and zeros for the rest.
//
// A tile is kTwinRows rows by kTwinCols columns of X (bf16, rows a multiple of 16 and columns
// of 128). Wave w takes the tile's strips (KU K-steps of 32 columns) w, w + 4, … and walks
// each strip down the tile's rows, 16 rows (one stage) at a time:
//   - m₁: X·V₁ on the matrix cores as in the row pass (V₁ of the strip loaded once), Σ|x|u₁
//     and Σx²w₁ on the VALU; a stage's row values are added into the wave's own LDS
//     accumulator, and the four waves' accumulators are summed in wave order when the tile
//     ends, so no address has two writers and the result does not depend on timing.
//   - m₂: each K-step's 16 × 32 block is written to the wave's LDS slab and read back four
//     rows of one column per lane, the A operand of Xᵀ·V₂ (a 16 × 16 × 16 MFMA whose K is the
//     16 rows). |Xᵀ|·u₂ runs on the matrix cores too, into the same accumulators: u₂'s three
//     exact bf16 terms sit in slots 12..14 of m₂'s packed operand (k ≤ 4 leaves them free),
//     each MFMA seeing only its own slots. The strip's column results accumulate down all
//     the tile's rows in registers and are written when the strip ends, one partial per
//     column and tile row.
//   - Σx²w₂: each lane's row sum of squares (products of bf16 values are exact in fp32) times
//     w₂ of that row, summed per lane in fp64; the tile's total is m₂'s only nonzero Σx²w
//     partial of the tile (the finish adds partials in fp64, so where the total sits does
//     not matter).
constexpr uint32_t kTwinRows = 512;
constexpr uint32_t kTwinCols = 1024;
constexpr uint32_t kTwinStrip = 32 * KU;  // columns per stage: KU K-steps of 32
constexpr uint32_t kTwinColStep = 128;    // a twin's X has columns in multiples of this
static_assert(kTwinColStep % kTwinStrip == 0 && kTwinCols % kTwinColStep == 0, "twin tiles");
constexpr uint32_t kTwinSlots = 5;  // a row's m₁ values in a wave's LDS: X·V₁'s (k ≤ 4), ν₁
constexpr uint32_t kSlabRow = 36;     // bf16 per slab row: 32 columns and 4 of padding, so
                                      // the four row groups a read touches sit 8 banks apart

struct TwinJob {
  uint64_t x, ld;             // X[0][0] (bf16), row stride in elements
  uint64_t v1, u1, w1;        // m₁: packed B₁·R₁ over X's columns, |B₁|·1, B₁²·1 (fp32)
  uint64_t v2, w2;            // m₂: packed B₂·R₂ with |B₂|·1's terms, over X's rows; B₂²·1
  uint64_t dot1, abs1, sq1;   // m₁ partials: [n_ct][rows_pad1] (dot: × k)
  uint64_t dot2, abs2, sq2;   // m₂ partials: [n_rt][rows_pad2], rows of m₂ = columns of X
  uint64_t tile_first;        // prefix of tiles over the twins before this one
  uint32_t rows, cols;
  uint32_t rows_pad1, rows_pad2;
  uint32_t n_rt, n_ct;        // tile rows and tile columns
  uint32_t pad0, pad1;
};
static_assert(sizeof(TwinJob) == 144, "TwinJob layout");

struct TwinStage {
  u32x4 x[KU];   // 16 rows × one strip: lane (g, i) row i, columns 32u + 8g .. + 7
  v2u32 v2;     // m₂'s packed operand: rows 4g .. 4g + 3 of the group, slot i
  float w2;     // B₂²·1 of row i
};

// A tile's buffer resources and this lane's offsets into them: X from the tile's first row
// (a tile's 512 rows stay far below 4 GiB), m₂'s packed operand and B₂²·1 from their starts.
struct TwinBuf {
  brsrc x, v2, w2;
  uint32_t ld2;           // X's row stride in bytes
  uint32_t xl, v2l, w2l;  // lane offsets: row i, columns 8g..; slot i of rows 4g..; row i
};

__device__ __forceinline__ TwinBuf twin_buf(const TwinJob& J, uint32_t r0, uint32_t g,
                                            uint32_t i) {
  TwinBuf b;
  b.x = make_rsrc(reinterpret_cast<const char*>(J.x) + (uint64_t)r0 * J.ld * 2);
  b.v2 = make_rsrc(reinterpret_cast<const void*>(J.v2));
  b.w2 = make_rsrc(reinterpret_cast<const void*>(J.w2));
  b.ld2 = (uint32_t)J.ld * 2;
  b.xl = i * b.ld2 + 16 * g;
  b.v2l = (((g >> 1) * 16 + i) * 8 + 4 * (g & 1)) * 2;
  b.w2l = i * 4;
  return b;
}

// Row group rr (a multiple of 16, rows of the tile from r0) of the strip at column cs.
__device__ __forceinline__ void twin_load(TwinStage& st, const TwinBuf& B, uint32_t r0,
                                          uint32_t rr, uint32_t cs) {
  const uint32_t xs = (rr - r0) * B.ld2 + cs * 2;  // uniform
#pragma unroll
  for (uint32_t u = 0; u < KU; u++) st.x[u] = bload128(B.x, B.xl, xs + 64 * u);
  // K-group (rr + 4g) / 8 of 8 rows, slot i, the half of it holding rows 4g .. 4g + 3: rows
  // rr .. (two K-groups of 16 slots of 8 bf16) from 32·rr bytes on
  st.v2 = __builtin_bit_cast(v2u32, __builtin_amdgcn_raw_buffer_load_b64(B.v2, B.v2l, rr * 32, 0));
  st.w2 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(B.w2, B.w2l, rr * 4, 0));
}

__device__ __forceinline__ void twin_stage(const TwinStage& st, const u32x4 (&bv1)[KU],
                                           const u32x4 (&bu1)[KU], v4f32 (&acc2)[2 * KU],
                                           float (&colsq)[2 * KU], double& u2sum, float* acc_w,
                                           uint16_t* slab, uint32_t row0, uint32_t k,
                                           uint32_t lane, uint32_t g, uint32_t i) {
  // m₁: X·V₁ and |X|·u₁ for the stage's 16 rows on the matrix cores (bv1: V₁'s slots 0..11,
  // bu1: u₁'s terms in slots 12..14), and row i's sum of squares for U₂
  v4f32 acc1 = {0.f, 0.f, 0.f, 0.f};
  float q2 = 0.f;
#pragma unroll
  for (uint32_t u = 0; u < KU; u++) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const v2u32 xa = {st.x[u][2 * h], st.x[u][2 * h + 1]};
      acc1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
          __builtin_bit_cast(v4i16, xa),
          __builtin_bit_cast(v4i16, v2u32{bv1[u][2 * h], bv1[u][2 * h + 1]}), acc1, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
          __builtin_bit_cast(v4i16, v2u32{xa.x & 0x7FFF7FFFu, xa.y & 0x7FFF7FFFu}),
          __builtin_bit_cast(v4i16, v2u32{bu1[u][2 * h], bu1[u][2 * h + 1]}), acc1, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
      // (a bit_cast straight from the vector element compiled to the first element every
      // time; through a scalar it does not)
      const uint32_t wv = st.x[u][e];
      const bf16x2 b = __builtin_bit_cast(bf16x2, wv);
      q2 = __builtin_amdgcn_fdot2_f32_bf16(b, b, q2, false);
    }
  }
  u2sum = fma((double)q2, (double)st.w2, u2sum);

  // m₂: Xᵀ·V₂ and |Xᵀ|·u₂ through the slab, one K-step at a time; the same reads give each
  // lane's column sums of squares for U₁ (two rows of one column per word)
  const v2u32 zero = {0u, 0u};
  const v4i16 bv = __builtin_bit_cast(v4i16, i < 12 ? st.v2 : zero);
  const v4i16 bu = __builtin_bit_cast(v4i16, i >= 12 ? st.v2 : zero);
#pragma unroll
  for (uint32_t u = 0; u < KU; u++) {
    uint16_t* wr = slab + i * kSlabRow + 8 * g;  // row i, columns 8g .. 8g + 7
    *reinterpret_cast<v2u32*>(wr) = v2u32{st.x[u][0], st.x[u][1]};
    *reinterpret_cast<v2u32*>(wr + 4) = v2u32{st.x[u][2], st.x[u][3]};
#pragma unroll
    for (uint32_t cb = 0; cb < 2; cb++) {
      // Rows 4g .. 4g + 3 of column 16cb + i in one transposing LDS read (ds_read_b64_tr_b16):
      // within each 16 lanes, lane m reads the 4 values of row 4g + m / 4 at columns
      // 16cb + 4(m mod 4) .., and lane i receives, as 16-bit element e, the value lane
      // 4e + i / 4 read at position i mod 4, which is row 4g + e of column 16cb + i.
      const uint16_t* rd = slab + (4 * g + i / 4) * kSlabRow + 16 * cb + 4 * (i % 4);
      const v2u32 t = __builtin_bit_cast(
          v2u32, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                     (__attribute__((address_space(3))) v4i16*)(rd)));
      const uint32_t lo = t.x, hi = t.y;
      v4f32& a = acc2[2 * u + cb];
      a = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4i16, v2u32{lo, hi}),
                                                    bv, a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
          __builtin_bit_cast(v4i16, v2u32{lo & 0x7FFF7FFFu, hi & 0x7FFF7FFFu}), bu, a, 0, 0,
          0);
      float& cq = colsq[2 * u + cb];
      cq = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, lo),
                                           __builtin_bit_cast(bf16x2, lo), cq, false);
      cq = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, hi),
                                           __builtin_bit_cast(bf16x2, hi), cq, false);
    }
  }

  // m₁: the stage's row values into the wave's accumulator. Lane (g, i) holds rows 4g + e and
  // slot i; challenge j's three terms are slots 3j .. 3j + 2, u₁'s are slots 12 .. 14.
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float v0 = acc1[e];
    const float va = row_next<1>(v0);
    const float vb = row_next<2>(v0);
    const uint32_t slot = i == 12 ? 4u : i / 3;
    if (i % 3 == 0 && (i / 3 < k || i == 12))
      acc_w[(row0 + 4 * g + e) * kTwinSlots + slot] += (v0 + va) + vb;
  }
}

__device__ __forceinline__ void twin_tile(const TwinJob* __restrict__ jobs,
                                          const uint32_t* __restrict__ tile_job, uint32_t k,
                                          uint32_t tidx, float* s_w, float* s_acc,
                                          uint16_t* s_slab, double* s_red) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63, g = lane >> 4, i = lane & 15;
  const TwinJob J = jobs[tile_job[tidx]];
  const uint32_t local = tidx - (uint32_t)J.tile_first;
  const uint32_t rt = local % J.n_rt, ct = local / J.n_rt;
  const uint32_t r0 = rt * kTwinRows, r1 = min(r0 + kTwinRows, J.rows);
  const uint32_t c0 = ct * kTwinCols, c1 = min(c0 + kTwinCols, J.cols);
  const uint32_t nrg = (r1 - r0) / 16, nstrip = (c1 - c0) / kTwinStrip;
  float* acc_w = s_acc + wave * kTwinRows * kTwinSlots;
  const TwinBuf TB = twin_buf(J, r0, g, i);
  uint16_t* slab = s_slab + wave * 16 * kSlabRow;
  stage_weight<kTwinCols>(J.w1, c0, c1, s_w);
  for (uint32_t t = lane; t < kTwinRows * kTwinSlots; t += 64) acc_w[t] = 0.f;
  __syncthreads();

  double u1sum = 0.0, u2sum = 0.0;
  for (uint32_t s = wave; s < nstrip; s += 4) {
    const uint32_t cs = c0 + s * kTwinStrip;
    // V₁ of the strip's K-steps, the same for every row group: its challenge terms (slots
    // 0..11) for X·V₁ and its u₁ terms (slots 12..14) for |X|·u₁
    u32x4 bv1[KU], bu1[KU];
#pragma unroll
    for (uint32_t u = 0; u < KU; u++) {
      const u32x4 v = gload<u32x4>(reinterpret_cast<const char*>(J.v1) +
                                   ((uint64_t)((cs + 32 * u) / 8 + g) * 16 + i) * 16);
      const u32x4 z = {0u, 0u, 0u, 0u};
      bv1[u] = i < 12 ? v : z;
      bu1[u] = i < 12 ? z : v;
    }
    v4f32 acc2[2 * KU];
    float colsq[2 * KU];
#pragma unroll
    for (uint32_t q = 0; q < 2 * KU; q++) {
      acc2[q] = v4f32{0.f, 0.f, 0.f, 0.f};
      colsq[q] = 0.f;
    }
    // Three stages in flight: the loads of the next two row groups go out before this one is
    // computed (past the last group they reread it, so every load is unconditional). Beside
    // the hashing kernels the pass waits on memory, not on issue: a third stage buffer took
    // the C4 step from 39.45 to 39.1 ms on one box (217 VGPRs, still two hashing waves per
    // SIMD beside it).
    TwinStage sa, sb, sc;
    twin_load(sa, TB, r0, r0, cs);
    twin_load(sb, TB, r0, r0 + 16 * min(1u, nrg - 1), cs);
    // Wait for the strip's first two stages here (s_waitcnt vmcnt(0)), once per strip: with
    // them in flight at the loop's entry, the compiler would wait for every load at the top of
    // each pass through the loop instead of only for the stage it computes.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    for (uint32_t rg = 0; rg < nrg; rg += 3) {
      twin_load(sc, TB, r0, r0 + 16 * min(rg + 2, nrg - 1), cs);
      twin_stage(sa, bv1, bu1, acc2, colsq, u2sum, acc_w, slab, 16 * rg, k, lane, g, i);
      twin_load(sa, TB, r0, r0 + 16 * min(rg + 3, nrg - 1), cs);
      if (rg + 1 < nrg)
        twin_stage(sb, bv1, bu1, acc2, colsq, u2sum, acc_w, slab, 16 * (rg + 1), k, lane, g,
                   i);
      twin_load(sb, TB, r0, r0 + 16 * min(rg + 4, nrg - 1), cs);
      if (rg + 2 < nrg)
        twin_stage(sc, bv1, bu1, acc2, colsq, u2sum, acc_w, slab, 16 * (rg + 2), k, lane, g,
                   i);
    }
    // U₁ of the strip: lane (g, i)'s squares of column 32u + 16cb + i (rows 4g .. 4g + 3 of
    // every row group) times w₁ of that column
#pragma unroll
    for (uint32_t u = 0; u < KU; u++)
#pragma unroll
      for (uint32_t cb = 0; cb < 2; cb++)
        u1sum = fma((double)colsq[2 * u + cb], (double)s_w[cs - c0 + 32 * u + 16 * cb + i],
                    u1sum);
    // m₂'s partials of the strip's columns: lane (g, i) of block q holds columns
    // 16q + 4g + e and slot i.
    float* dot2 = reinterpret_cast<float*>(J.dot2);
    float* abs2 = reinterpret_cast<float*>(J.abs2);
    const uint64_t cbase = (uint64_t)rt * J.rows_pad2;
#pragma unroll
    for (uint32_t q = 0; q < 2 * KU; q++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float v0 = acc2[q][e];
        const float va = row_next<1>(v0);
        const float vb = row_next<2>(v0);
        const float t = (v0 + va) + vb;
        const uint32_t col = cs + 16 * q + 4 * g + e;
        if (i % 3 == 0 && i / 3 < k) gstore<float>(dot2 + (cbase + col) * k + i / 3, t);
        if (i == 12) gstore<float>(abs2 + cbase + col, t);
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    u1sum += __shfl_xor(u1sum, o);
    u2sum += __shfl_xor(u2sum, o);
  }
  if (lane == 0) {
    s_red[wave] = u2sum;
    s_red[4 + wave] = u1sum;
  }
  __syncthreads();
  // m₁'s partials of the tile's rows: the four waves' accumulators in wave order, and the
  // tile's Σx²w₁ total at its first row
  float* dot1 = reinterpret_cast<float*>(J.dot1);
  float* abs1 = reinterpret_cast<float*>(J.abs1);
  double* sq1 = reinterpret_cast<double*>(J.sq1);
  const uint64_t rbase = (uint64_t)ct * J.rows_pad1;
  const double tot1 = ((s_red[4] + s_red[5]) + s_red[6]) + s_red[7];
  for (uint32_t row = threadIdx.x; row < r1 - r0; row += blockDim.x) {
    float d[kTwinSlots];
#pragma unroll
    for (uint32_t t = 0; t < kTwinSlots; t++) d[t] = s_acc[row * kTwinSlots + t];
#pragma unroll
    for (uint32_t w = 1; w < 4; w++)
#pragma unroll
      for (uint32_t t = 0; t < kTwinSlots; t++)
        d[t] += s_acc[(w * kTwinRows + row) * kTwinSlots + t];
    for (uint32_t j = 0; j < k; j++) gstore<float>(dot1 + (rbase + r0 + row) * k + j, d[j]);
    gstore<float>(abs1 + rbase + r0 + row, d[4]);
    gstore<double>(sq1 + rbase + r0 + row, row == 0 ? tot1 : 0.0);
  }
  // m₂'s Σx²w₂ partials of the tile's columns: the tile's total at its first column
  const double tot = ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
  double* sq2 = reinterpret_cast<double*>(J.sq2);
  for (uint32_t c = c0 + threadIdx.x; c < c1; c += blockDim.x)
    gstore<double>(sq2 + (uint64_t)rt * J.rows_pad2 + c, c == c0 ? tot : 0.0);
}

// The tiles of every twin, from the tile queues when the grid is limited (as the row pass
// takes them), else one block per tile.
__global__ __launch_bounds__(256) void twin_pass(const TwinJob* __restrict__ jobs,
                                                 const uint32_t* __restrict__ tile_job,
                                                 uint32_t k, uint32_t n_tiles,
                                                 uint32_t* __restrict__ queue) {
  __shared__ __align__(16) float s_w[kTwinCols];
  __shared__ __align__(16) float s_acc[4 * kTwinRows * kTwinSlots];
  __shared__ __align__(16) uint16_t s_slab[4 * 16 * kSlabRow];
  __shared__ double s_red[8];
  __shared__ uint32_t s_tile;
  tile_loop(n_tiles, queue, &s_tile, [&](uint32_t t) {
    twin_tile(jobs, tile_job, k, t, s_w, s_acc, s_slab, s_red);
  });
}

// ---- B-pass reduction: B·R, |B|·1, B²·1 per row of B, packed for the A pass -------------

struct RedJob {
  uint64_t pdot, pabs, psq;  // the B job's partials
  uint64_t vout;             // packed B·R for the A pass
  uint64_t u, w;             // b1 = |B|·1 and b2 = B²·1, fp32 [q]
  uint64_t group_first;      // prefix of (8-row groups x k) over the jobs before it
  uint32_t rows, rows_pad;   // q and its padding
  uint32_t n_chunks, a_dt;   // the A pass's dtype decides the packing
  uint32_t u_slots, pad;     // 1: also pack b1's three bf16 terms into slots 12..14 (a
                             // twin product, whose |A|·b1 runs on the matrix cores)
};
static_assert(sizeof(RedJob) == 80, "RedJob layout");

__global__ __launch_bounds__(256) void reduce_b(const RedJob* __restrict__ jobs, uint32_t n_jobs,
                                                uint64_t n_threads, uint32_t k) {
  const uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= n_threads) return;
  uint32_t lo = 0, hi = n_jobs - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (jobs[mid].group_first <= g) lo = mid;
    else hi = mid - 1;
  }
  const RedJob J = jobs[lo];
  const uint64_t local = g - J.group_first;
  const uint32_t grp = (uint32_t)(local / k), j = (uint32_t)(local % k);
  const float* pdot = reinterpret_cast<const float*>(J.pdot);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const uint32_t row = 8 * grp + e;
    double s = 0.0;
    if (row < J.rows)
      for (uint32_t c = 0; c < J.n_chunks; c++)
        s += (double)gload<float>(pdot + ((uint64_t)c * J.rows_pad + row) * k + j);
    v[e] = (float)s;
  }
  if (J.a_dt == DT_BF16) {
    uint16_t pl[3][8];
#pragma unroll
    for (int e = 0; e < 8; e++) split_bf16x3(v[e], pl[0][e], pl[1][e], pl[2][e]);
    uint16_t* dst = reinterpret_cast<uint16_t*>(J.vout) +
                    (((uint64_t)grp * groups_b3(k) + j / 5) * 16 + 3 * (j % 5)) * 8;
#pragma unroll
    for (int p = 0; p < 3; p++)
      gstore<u32x4>(dst + 8 * p, u32x4{pl[p][0] | (uint32_t)pl[p][1] << 16,
                                       pl[p][2] | (uint32_t)pl[p][3] << 16,
                                       pl[p][4] | (uint32_t)pl[p][5] << 16,
                                       pl[p][6] | (uint32_t)pl[p][7] << 16});
  } else {
    float* base = reinterpret_cast<float*>(J.vout);
    const uint32_t njg = groups_f4(k);
#pragma unroll
    for (int h = 0; h < 2; h++)
      gstore<u32x4>(base + (((uint64_t)(2 * grp + h) * njg + j / 16) * 16 + j % 16) * 4,
                    u32x4{__float_as_uint(v[4 * h]), __float_as_uint(v[4 * h + 1]),
                          __float_as_uint(v[4 * h + 2]), __float_as_uint(v[4 * h + 3])});
  }
  if (j == 0) {
    const float* pabs = reinterpret_cast<const float*>(J.pabs);
    const double* psq = reinterpret_cast<const double*>(J.psq);
    float* u = reinterpret_cast<float*>(J.u);
    float* w = reinterpret_cast<float*>(J.w);
    float ua[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // rows past the matrix: zero
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t row = 8 * grp + e;
      if (row >= J.rows) continue;
      double a = 0.0, q = 0.0;
      for (uint32_t c = 0; c < J.n_chunks; c++) {
        a += (double)gload<float>(pabs + (uint64_t)c * J.rows_pad + row);
        q += gload<double>(psq + (uint64_t)c * J.rows_pad + row);
      }
      gstore<float>(u + row, (float)a);
      gstore<float>(w + row, (float)q);
      ua[e] = (float)a;
    }
    if (J.u_slots) {
      uint16_t pl[3][8];
#pragma unroll
      for (int e = 0; e < 8; e++) split_bf16x3(ua[e], pl[0][e], pl[1][e], pl[2][e]);
      uint16_t* dst = reinterpret_cast<uint16_t*>(J.vout) + ((uint64_t)grp * 16 + 12) * 8;
#pragma unroll
      for (int p = 0; p < 3; p++)
        gstore<u32x4>(dst + 8 * p, u32x4{pl[p][0] | (uint32_t)pl[p][1] << 16,
                                         pl[p][2] | (uint32_t)pl[p][3] << 16,
                                         pl[p][4] | (uint32_t)pl[p][5] << 16,
                                         pl[p][6] | (uint32_t)pl[p][7] << 16});
    }
  }
}

// ---- finish: one product's row ------------------------------------------------------------
//
// Three kernels. bias_terms: per biased product, ‖b‖₁, ‖b‖² and bᵀR_j. finish_slices: per
// slice of at most kSliceRows rows of a product, the fp64 sums over its rows of ν_i², |P|1_i²,
// ‖P_i‖², (A²(B²1))_i and d_ij², written as one record. finish_final: per product, the slices'
// records added in slice order, then the square roots. Every sum has a fixed order, so the
// row does not depend on timing; slicing keeps the largest products (150k rows) from running
// on one block.

constexpr uint32_t kSliceRows = 2048;

struct FinJob {
  uint64_t a_dot, a_abs, a_sq;  // A-pass partials (rows n)
  uint64_t p_dot, p_abs, p_sq;  // P-pass partials (rows n)
  uint64_t r;                   // canonical R [w][k] (for the bias term)
  uint64_t bias;                // fp32 [w] or 0
  uint32_t n, w;
  uint32_t a_rows_pad, a_chunks;
  uint32_t p_rows_pad, p_chunks;
  uint32_t slice_first, n_slices;  // this product's slice records
};
static_assert(sizeof(FinJob) == 96, "FinJob layout");

struct SliceJob {
  uint32_t prod, r0, r1, pad;
};
static_assert(sizeof(SliceJob) == 16, "SliceJob layout");

// Per product: ‖b‖₁ (fp32, as the reference adds it to each ν_i), ‖b‖² and bᵀR_j (fp32).
struct BiasOut {
  uint64_t babs;  // float bits in the low word
  double bsq;
};

__device__ __forceinline__ double block_sum(double v, double* sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
  __syncthreads();
  if (ln == 0) sh[wv] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += sh[i];
  __syncthreads();
  return t;
}

// One block per biased product (index list `which`).
__global__ __launch_bounds__(256) void bias_terms(const FinJob* __restrict__ jobs,
                                                  const uint32_t* __restrict__ which, uint32_t k,
                                                  BiasOut* __restrict__ bout,
                                                  float* __restrict__ br) {
  __shared__ double sh[4];
  const uint32_t pi = which[blockIdx.x];
  const FinJob J = jobs[pi];
  const float* bias = reinterpret_cast<const float*>(J.bias);
  const float* R = reinterpret_cast<const float*>(J.r);
  double a = 0.0, q = 0.0;
  for (uint32_t c = threadIdx.x; c < J.w; c += blockDim.x) {
    const double b = gload<float>(bias + c);
    a += fabs(b);
    q += b * b;
  }
  a = block_sum(a, sh);
  q = block_sum(q, sh);
  if (threadIdx.x == 0) {
    BiasOut o;
    o.babs = __float_as_uint((float)a);
    o.bsq = q;
    bout[pi] = o;
  }
  for (uint32_t j = 0; j < k; j++) {
    double t = 0.0;
    for (uint32_t c = threadIdx.x; c < J.w; c += blockDim.x)
      t += (double)gload<float>(bias + c) * (double)gload<float>(R + (uint64_t)c * k + j);
    t = block_sum(t, sh);
    if (threadIdx.x == 0) br[(uint64_t)pi * k + j] = (float)t;
  }
}

// block_sum of N values at once: each value's additions are block_sum's, in the same order.
template <int N>
__device__ __forceinline__ void block_sums(double (&v)[N], double* sh) {
#pragma unroll
  for (int n = 0; n < N; n++)
    for (int o = 32; o > 0; o >>= 1) v[n] += __shfl_xor(v[n], o);
  const int wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
  __syncthreads();
  if (ln == 0) {
#pragma unroll
    for (int n = 0; n < N; n++) sh[n * 4 + wv] = v[n];
  }
  __syncthreads();
#pragma unroll
  for (int n = 0; n < N; n++) {
    double t = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += sh[n * 4 + i];
    v[n] = t;
  }
  __syncthreads();
}

// Adds a row's partial dot products X·V_j, j = j0 .. j0 + nj − 1, over its column chunks in
// chunk order; 16-byte loads when every row's k values start 16-byte aligned.
__device__ __forceinline__ void chunk_dots(const float* __restrict__ dot, uint32_t rows_pad,
                                           uint32_t chunks, uint32_t r, uint32_t k,
                                           uint32_t j0, uint32_t nj, bool vec, double (&acc)[8]) {
  // Four chunks' loads go out before their sums, which are taken in chunk order (a chunk past
  // the last rereads the last and is not added).
  for (uint32_t c0 = 0; c0 < chunks; c0 += 4) {
    if (vec) {
      v4f32 x[4][2];
#pragma unroll
      for (uint32_t t = 0; t < 4; t++) {
        const uint32_t c = min(c0 + t, chunks - 1);
        const float* src = dot + ((uint64_t)c * rows_pad + r) * k + j0;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++)
          x[t][h] = 4 * h < nj ? gload<v4f32>(src + 4 * h) : v4f32{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (uint32_t t = 0; t < 4; t++)
        if (c0 + t < chunks)
#pragma unroll
          for (uint32_t h = 0; h < 2; h++)
            if (4 * h < nj)
#pragma unroll
              for (int e = 0; e < 4; e++) acc[4 * h + e] += (double)x[t][h][e];
    } else {
      float x[4][8];
#pragma unroll
      for (uint32_t t = 0; t < 4; t++) {
        const uint32_t c = min(c0 + t, chunks - 1);
        const float* src = dot + ((uint64_t)c * rows_pad + r) * k + j0;
#pragma unroll
        for (uint32_t jj = 0; jj < 8; jj++) x[t][jj] = jj < nj ? gload<float>(src + jj) : 0.f;
      }
#pragma unroll
      for (uint32_t t = 0; t < 4; t++)
        if (c0 + t < chunks)
#pragma unroll
          for (uint32_t jj = 0; jj < 8; jj++)
            if (jj < nj) acc[jj] += (double)x[t][jj];
    }
  }
}

// A row's |·| and squares partials over the chunks, four chunks' loads before their sums.
__device__ __forceinline__ void chunk_sums(const float* __restrict__ abs_,
                                           const double* __restrict__ sq, uint32_t rows_pad,
                                           uint32_t chunks, uint32_t r, double& s1, double& s2) {
  for (uint32_t c0 = 0; c0 < chunks; c0 += 4) {
    float a[4];
    double q[4];
#pragma unroll
    for (uint32_t t = 0; t < 4; t++) {
      const uint64_t at = (uint64_t)min(c0 + t, chunks - 1) * rows_pad + r;
      a[t] = gload<float>(abs_ + at);
      q[t] = gload<double>(sq + at);
    }
#pragma unroll
    for (uint32_t t = 0; t < 4; t++)
      if (c0 + t < chunks) {
        s1 += (double)a[t];
        s2 += q[t];
      }
  }
}

// One block per slice. Record layout: [Σν², Σ|P|1², Σ‖P_i‖², Σ(A²(B²1))_i, Σd_1², ..., Σd_k²].
// One sweep over the slice's rows takes the four sums and the residuals of challenges 1..8;
// each further 8 challenges take a sweep of their own.
__global__ __launch_bounds__(256) void finish_slices(const FinJob* __restrict__ jobs,
                                                     const SliceJob* __restrict__ slices,
                                                     uint32_t k, const BiasOut* __restrict__ bout,
                                                     const float* __restrict__ br,
                                                     double* __restrict__ recs) {
  __shared__ double sh[12 * 4];
  const SliceJob S = slices[blockIdx.x];
  const FinJob J = jobs[S.prod];
  const uint32_t tid = threadIdx.x;
  double* out = recs + (uint64_t)blockIdx.x * (4 + k);
  const bool biased = J.bias != 0;
  const float babs = biased ? __uint_as_float((uint32_t)bout[S.prod].babs) : 0.f;
  const float* adot = reinterpret_cast<const float*>(J.a_dot);
  const float* aabs = reinterpret_cast<const float*>(J.a_abs);
  const double* asq = reinterpret_cast<const double*>(J.a_sq);
  const float* pdot = reinterpret_cast<const float*>(J.p_dot);
  const float* pabs = reinterpret_cast<const float*>(J.p_abs);
  const double* psq = reinterpret_cast<const double*>(J.p_sq);
  const bool vec = k % 4 == 0 && (J.a_dot & 15) == 0 && (J.p_dot & 15) == 0;

  for (uint32_t j0 = 0; j0 < k; j0 += 8) {
    const bool first = j0 == 0;
    const uint32_t nj = min(8u, k - j0);
    float bj[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++)
      bj[jj] = (biased && (uint32_t)jj < nj) ? br[(uint64_t)S.prod * k + j0 + jj] : 0.f;
    // acc[0..3]: Σν², Σ|P|1², Σ‖P_i‖², Σ(A²(B²1))_i (first sweep); acc[4 + jj]: Σd².
    double acc[12];
#pragma unroll
    for (int t = 0; t < 12; t++) acc[t] = 0.0;
    for (uint32_t r = S.r0 + tid; r < S.r1; r += blockDim.x) {
      // A row's chunk partials are summed in fp64 in chunk order, then rounded to fp32 where
      // the reference's matvec output is fp32.
      double ab[8], pr[8];
#pragma unroll
      for (int jj = 0; jj < 8; jj++) ab[jj] = pr[jj] = 0.0;
      chunk_dots(adot, J.a_rows_pad, J.a_chunks, r, k, j0, nj, vec, ab);
      chunk_dots(pdot, J.p_rows_pad, J.p_chunks, r, k, j0, nj, vec, pr);
      if (first) {
        double nu = 0.0, t2 = 0.0, p1 = 0.0, pq = 0.0;
        chunk_sums(aabs, asq, J.a_rows_pad, J.a_chunks, r, nu, t2);
        chunk_sums(pabs, psq, J.p_rows_pad, J.p_chunks, r, p1, pq);
        float nuf = (float)nu;
        if (biased) nuf = nuf + babs;
        const float p1f = (float)p1;
        acc[0] += (double)nuf * (double)nuf;
        acc[1] += (double)p1f * (double)p1f;
        acc[2] += pq;
        acc[3] += (double)(float)t2;
      }
      // Residuals d_ij = A(Br_j)_i (+ bᵀr_j) − (Pr_j)_i in fp32.
#pragma unroll
      for (int jj = 0; jj < 8; jj++) {
        if ((uint32_t)jj < nj) {
          float abf = (float)ab[jj];
          if (biased) abf = abf + bj[jj];
          const float d = abf - (float)pr[jj];
          acc[4 + jj] += (double)d * (double)d;
        }
      }
    }
    block_sums<12>(acc, sh);
    if (tid == 0) {
      if (first)
        for (int t = 0; t < 4; t++) out[t] = acc[t];
      for (uint32_t jj = 0; jj < nj; jj++) out[4 + j0 + jj] = acc[4 + jj];
    }
  }
}

// One thread per product: the slices' records in order, then the row.
__global__ __launch_bounds__(256) void finish_final(const FinJob* __restrict__ jobs,
                                                    uint32_t n, uint32_t k, uint32_t guard,
                                                    const BiasOut* __restrict__ bout,
                                                    const double* __restrict__ recs,
                                                    double* __restrict__ rows) {
  const uint32_t pi = blockIdx.x * blockDim.x + threadIdx.x;
  if (pi >= n) return;
  const FinJob J = jobs[pi];
  double* out = rows + (uint64_t)pi * (5 + k);
  const double nan = __builtin_nan("");
  for (uint32_t col = 0; col < 4 + k; col++) {
    double t = 0.0;
    for (uint32_t sl = 0; sl < J.n_slices; sl++)
      t += recs[(uint64_t)(J.slice_first + sl) * (4 + k) + col];
    if (col < 2) out[col] = guard ? sqrt(t) : nan;
    else if (col == 2) out[2] = sqrt(t);
    else if (col == 3) out[3] = t;
    else out[1 + col] = sqrt(t);
  }
  out[4] = J.bias != 0 ? bout[pi].bsq : 0.0;
}

// ---- P-pass sums of fused products, from the chunk kernel's run records -------------------

// One fused product (freivalds.h): its P is a leaf whose message is 0x00 || header (head
// bytes) || P, and the chunk kernel wrote one record per run of a row.
struct FixJob {
  uint64_t p, r, seg;        // P, R [w][k], run records [J][n]
  uint64_t pdot, pabs, psq;  // the P job's partials: column chunk 0 of [rows_pad]
  uint64_t row_first;        // prefix of rows over the jobs before it
  uint32_t n, w;
  uint32_t head, esz;
  uint32_t J, k;             // record slots per row; challenges (1, 2 or 4)
};
static_assert(sizeof(FixJob) == 80, "FixJob layout");

// One thread per row: the row's records in chunk order (fp64), then the elements of the
// leaf's first bytes up to the first 128-byte boundary of the message (row 0) and of its last
// bytes after the last one (the last row), which no chunk's interior pairs took. Rounded to
// the P job's partial formats as one column chunk.
// `blk[b]`: the job of block b's first row (blk[gridDim.x] the last job), so a thread searches
// only the few jobs its block's rows span instead of all of them (a dozen dependent loads).
__global__ __launch_bounds__(256) void fused_rows(const FixJob* __restrict__ jobs,
                                                  const uint32_t* __restrict__ blk,
                                                  uint64_t n_threads) {
  const uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= n_threads) return;
  uint32_t lo = blk[blockIdx.x], hi = blk[blockIdx.x + 1];
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (jobs[mid].row_first <= g) lo = mid;
    else hi = mid - 1;
  }
  const FixJob J = jobs[lo];
  const uint32_t i = (uint32_t)(g - J.row_first);
  const uint64_t rb = (uint64_t)J.w * J.esz, H = J.head, L = H + (uint64_t)J.n * rb;
  const uint64_t hc = (H + 127) & ~uint64_t(127), lf = L & ~uint64_t(127);
  const uint64_t fs = max<uint64_t>(H + i * rb, hc), fe = min<uint64_t>(H + (i + 1) * rb, lf);
  double d[4] = {0.0, 0.0, 0.0, 0.0}, s1 = 0.0, s2 = 0.0;
  bool exact = false;
  if (fs < fe) {
    const char* rec = reinterpret_cast<const char*>(J.seg) + (uint64_t)kRunBytes * i;
    const uint64_t stride = (uint64_t)kRunBytes * J.n;
    auto add = [&](const v4f32& a, const u32x4& b) {
      for (uint32_t j = 0; j < J.k; j++) d[j] += (double)a[j];
      s1 += (double)__uint_as_float(b.x);
      exact |= b.y != 0u;
      s2 += __longlong_as_double((long long)((uint64_t)b.w << 32 | b.z));
    };
    // Four records' loads are issued before their sums, which are taken in record order.
    uint64_t left = ((fe - 1) >> 10) - (fs >> 10) + 1;
    for (; left >= 4; left -= 4, rec += 4 * stride) {
      v4f32 a[4];
      u32x4 b[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        a[u] = gload<v4f32>(rec + u * stride);
        b[u] = gload<u32x4>(rec + u * stride + 16);
      }
#pragma unroll
      for (int u = 0; u < 4; u++) add(a[u], b[u]);
    }
    for (; left > 0; left--, rec += stride) add(gload<v4f32>(rec), gload<u32x4>(rec + 16));
  }
  const float* R = reinterpret_cast<const float*>(J.r);
  auto elem = [&](uint64_t e) {
    return J.esz == 2 ? __uint_as_float((uint32_t)gload<uint16_t>(
                                            reinterpret_cast<const uint16_t*>(J.p) + e)
                                        << 16)
                      : gload<float>(reinterpret_cast<const float*>(J.p) + e);
  };
  auto rest = [&](uint64_t b0, uint64_t b1) {  // payload bytes [b0, b1) of row i
    for (uint64_t e = b0 / J.esz; e < b1 / J.esz; e++) {
      const float x = elem(e);
      const uint64_t col = e - (uint64_t)i * J.w;
      for (uint32_t j = 0; j < J.k; j++)
        d[j] += (double)x * (double)gload<float>(R + col * J.k + j);
      s1 += fabs((double)x);
      s2 += (double)x * (double)x;
    }
  };
  if (i == 0 && hc > H) rest(0, hc - H);
  if (i + 1 == J.n && lf < L) rest(lf - H, L - H);
  if (exact) {  // a run met exponents out of fp32 squares' range: the row's sums in fp64
    // (|x| too: the chunk kernel takes a bf16 pair's |x| with v_dot2, whose subnormal inputs
    // are those of a pair marked here)
    s1 = 0.0;
    s2 = 0.0;
    for (uint64_t e = (uint64_t)i * J.w; e < (uint64_t)(i + 1) * J.w; e++) {
      const double x = elem(e);
      s1 += fabs(x);
      s2 += x * x;
    }
  }
  float* pdot = reinterpret_cast<float*>(J.pdot);
  for (uint32_t j = 0; j < J.k; j++) gstore<float>(pdot + (uint64_t)i * J.k + j, (float)d[j]);
  gstore<float>(reinterpret_cast<float*>(J.pabs) + i, (float)s1);
  gstore<double>(reinterpret_cast<double*>(J.psq) + i, s2);
}

// ---- the plan ---------------------------------------------------------------------------

struct PassLaunch {
  uint32_t xt, weighted, sq64, njg;  // kernel variant
  uint64_t job_off;  // index into the job array
  uint32_t n_jobs;
  uint64_t blk_off;  // index into the block->job table
  uint32_t n_blocks;
};

struct FvPlan {
  size_t n = 0;
  uint32_t k = 0, guard = 1;
  char* base = nullptr;
  size_t total = 0;
  uint32_t* d_key = nullptr;
  uint32_t* d_queue = nullptr;  // a row pass's kQueues tile queue counters per stage (grid-limited)
  ChallengeItem* d_items_b3 = nullptr;  // items whose R is read by bf16 passes
  ChallengeItem* d_items_f4 = nullptr;
  uint32_t n_items = 0;
  uint64_t n_units = 0;
  float* d_r = nullptr;
  uint16_t* d_r_b3 = nullptr;
  float* d_r_f4 = nullptr;
  PassJob* d_jobs = nullptr;
  uint32_t* d_blk = nullptr;
  RedJob* d_red = nullptr;
  uint32_t n_red = 0;
  uint64_t n_red_threads = 0;
  FinJob* d_fin = nullptr;
  SliceJob* d_slices = nullptr;
  uint32_t n_slices = 0;
  uint32_t* d_biased = nullptr;  // indices of the products with a bias
  uint32_t n_biased = 0;
  BiasOut* d_bout = nullptr;
  float* d_br = nullptr;      // bᵀR_j per product, [n][k]
  double* d_recs = nullptr;   // slice records, [n_slices][4 + k]
  std::vector<PassLaunch> pass_b, pass_ap;  // B pass; then A and P passes
  TwinJob* d_twins = nullptr;     // the twin pass: one job per pair of twins
  uint32_t* d_twin_tile = nullptr;  // tile -> twin job
  uint32_t n_twins = 0, n_twin_tiles = 0;
  bool need_b3 = false, need_f4 = false;
  uint64_t bytes = 0;  // algorithmic bytes: A, B, P read once
  uint64_t r_floats = 0;
  // Host copies kept for fusing with a leaf plan.
  std::vector<pots_fv_product> h_prods;
  std::vector<uint64_t> h_r_off;    // product i's R at d_r + h_r_off[i] floats
  std::vector<PassJob> h_jobs;      // the ordered job array
  std::vector<uint32_t> h_src;      // original job index of each ordered job
  std::vector<uint32_t> h_blk;      // the block -> job table
  std::vector<FinJob> h_fin;
  std::unordered_map<uint64_t, int64_t> p_index;  // P address -> product (-1: shared)
  // Fused products: their run records and fix-up jobs, one allocation.
  uint32_t max_grid[POTS_FV_STAGES] = {};  // row-pass grid limits (0: a block per tile)
  bool fused = false;
  char* fbase = nullptr;
  FixJob* d_fix = nullptr;
  uint32_t n_fix = 0;
  uint64_t n_fix_rows = 0;
  uint32_t* d_fix_blk = nullptr;  // block -> first fix-up job (fused_rows)
};

// Packed operands (R, B·R) hold whole 32-row groups, one bf16 K-step of the row pass; rows past
// the matrix are zero.
static uint64_t pad32(uint64_t rows) { return (rows + 31) / 32 * 32; }

static uint32_t chunk_cols_for(uint32_t cols, uint32_t sstep, uint32_t cmax) {
  // At most cmax columns per chunk, in whole pipeline stages, balanced over the chunks (cmax
  // is a multiple of the stage width, so rounding up stays within it).
  const uint32_t n = std::max<uint32_t>(1, (cols + cmax - 1) / cmax);
  uint32_t c = (cols + n - 1) / n;
  c = (c + sstep - 1) / sstep * sstep;
  return std::max<uint32_t>(c, sstep);
}

// 16-slot column groups of a packed operand read by X of dtype xt, and how many of them one
// block computes (the kernel variant): all of them up to 4, else 4 per block.
static uint32_t groups_for(uint32_t xt, uint32_t k) {
  return xt == DT_BF16 ? groups_b3(k) : groups_f4(k);
}
static uint32_t njg_for(uint32_t xt, uint32_t k) { return std::min<uint32_t>(4, groups_for(xt, k)); }

}  // namespace pots

using namespace pots;

extern "C" int pots_fv_plan_create(size_t n, const pots_fv_product* prods, uint32_t k,
                                   uint32_t guard, void** plan) {
  if (!plan || !prods || n == 0 || n >= 0x7FFFFFFFull || k < 1 || k > 255) return POTS_E_ARG;
  FvPlan* P = new (std::nothrow) FvPlan;
  if (!P) return POTS_E_NOMEM;
  P->n = n;
  P->k = k;
  P->guard = guard ? 1 : 0;

  // Layout of the workspace, computed on the host.
  size_t at = 0;
  auto place = [&](size_t bytes) {
    size_t a = at;
    at = align_up(at + std::max<size_t>(bytes, 16), 256);
    return a;
  };
  const size_t o_key = place(32);
  const size_t o_queue = place(POTS_FV_STAGES * kQueues * sizeof(uint32_t));
  const uint64_t b3_per_row = (uint64_t)groups_b3(k) * 16;  // bf16 elements per row of V
  const uint64_t f4_per_row = (uint64_t)groups_f4(k) * 16;  // floats per row of V
  std::vector<ChallengeItem> items(n);
  uint64_t r_floats = 0, b3_elems = 0, f4_floats = 0, units = 0;
  for (size_t i = 0; i < n; i++) {
    const pots_fv_product& p = prods[i];
    if (p.n == 0 || p.q == 0 || p.w == 0 || p.m == 0 || !p.a || !p.b || !p.p) {
      delete P;
      return POTS_E_ARG;
    }
    if (p.a_dtype > 1 || p.b_dtype > 1 || p.p_dtype > 1 || p.a_trans > 1) {
      delete P;
      return POTS_E_ARG;
    }
    const uint64_t wpad = pad32(p.w);
    items[i].m = p.m;
    items[i].width = p.w;
    items[i].out_off = r_floats;
    items[i].unit_first = units;
    r_floats += (uint64_t)p.w * k;
    units += wpad / 16;
    // R packed in the layouts the B and P passes read.
    P->need_b3 |= p.b_dtype == DT_BF16 || p.p_dtype == DT_BF16;
    P->need_f4 |= p.b_dtype == DT_F32 || p.p_dtype == DT_F32;
    items[i].pk_off = 0;
    b3_elems += wpad * b3_per_row;
    f4_floats += wpad * f4_per_row;
  }
  P->n_items = (uint32_t)n;
  P->n_units = units;
  P->r_floats = r_floats;
  // Packed offsets: the same item order in both layouts.
  std::vector<ChallengeItem> items_b3 = items, items_f4 = items;
  {
    uint64_t ob = 0, of = 0;
    for (size_t i = 0; i < n; i++) {
      const uint64_t wpad = pad32(prods[i].w);
      items_b3[i].pk_off = ob;
      items_f4[i].pk_off = of;
      ob += wpad * b3_per_row;
      of += wpad * f4_per_row;
    }
  }
  const size_t o_items_b3 = place(n * sizeof(ChallengeItem));
  const size_t o_items_f4 = place(n * sizeof(ChallengeItem));
  const size_t o_r = place(r_floats * 4);
  const size_t o_rb3 = place(P->need_b3 ? b3_elems * 2 : 16);
  const size_t o_rf4 = place(P->need_f4 ? f4_floats * 4 : 16);

  // Twins: a product whose A is given transposed takes the row-major product over the same X
  // as its twin; the pair's A passes become one twin job (twin_pass).
  std::vector<int64_t> twin_of(n, -1);  // the other product of a pair
  std::vector<std::pair<uint32_t, uint32_t>> twins;  // (m₁: A = X, m₂: A = Xᵀ)
  {
    std::unordered_map<uint64_t, std::vector<uint32_t>> by_x;  // X address -> row-major A's
    for (size_t i = 0; i < n; i++)
      if (!prods[i].a_trans && prods[i].a_dtype == DT_BF16)
        by_x[reinterpret_cast<uint64_t>(prods[i].a)].push_back((uint32_t)i);
    for (size_t i = 0; i < n; i++) {
      const pots_fv_product& t = prods[i];
      if (!t.a_trans) continue;
      // X is [q, n] for the transposed product: rows of X = its q, columns = its n
      const uint32_t rows = t.q, cols = t.n;
      const uint64_t x = reinterpret_cast<uint64_t>(t.a);
      // (the twin pass addresses a tile's kTwinRows rows through 32-bit buffer offsets)
      bool ok = k <= 4 && t.a_dtype == DT_BF16 && rows % 16 == 0 && cols % kTwinColStep == 0 &&
                x % 16 == 0 && (t.lda * 2) % 16 == 0 && t.lda >= cols &&
                (uint64_t)kTwinRows * t.lda * 2 < 0x7FFFFFFFull;
      int64_t mate = -1;
      if (ok) {
        auto it = by_x.find(x);
        if (it != by_x.end())
          for (uint32_t j : it->second)
            if (twin_of[j] < 0 && prods[j].lda == t.lda && prods[j].n == rows &&
                prods[j].q == cols) {
              mate = j;
              break;
            }
      }
      if (mate < 0) {
        delete P;
        return POTS_E_ARG;
      }
      twin_of[i] = mate;
      twin_of[mate] = (int64_t)i;
      twins.emplace_back((uint32_t)mate, (uint32_t)i);
    }
  }

  // Jobs: B pass (one per product), then A pass and P pass.
  std::vector<PassJob> jobs;
  std::vector<uint64_t> job_part_bytes;  // where each job's partials go, filled below
  struct Shape {
    uint32_t rows, cols, dt;
    uint64_t x, ld;
  };
  auto make_job = [&](const Shape& s) {
    PassJob J;
    memset(&J, 0, sizeof J);
    J.x = s.x;
    J.ld = s.ld;
    J.rows = s.rows;
    J.cols = s.cols;
    J.rows_pad = (s.rows + kRowsPerBlock - 1) / kRowsPerBlock * kRowsPerBlock;
    J.chunk_cols = s.dt == DT_BF16
                       ? chunk_cols_for(s.cols, Geo<DT_BF16>::KSTEP * KU, Geo<DT_BF16>::CHUNK)
                       : chunk_cols_for(s.cols, Geo<DT_F32>::KSTEP * KU, Geo<DT_F32>::CHUNK);
    J.n_chunks = (s.cols + J.chunk_cols - 1) / J.chunk_cols;
    J.n_rg = J.rows_pad / kRowsPerBlock;
    J.n_jg = groups_for(s.dt, k);
    J.n_jt = (J.n_jg + njg_for(s.dt, k) - 1) / njg_for(s.dt, k);
    const uint32_t esz = s.dt == DT_BF16 ? 2 : 4;
    // The full stages address a wave's 16 rows by 32-bit offsets from its first row: a row
    // stride beyond that (rows of over 128 MiB) takes the guarded loads' 64-bit addresses.
    J.aligned = (s.x % 16 == 0) && ((s.ld * esz) % 16 == 0) &&
                (uint64_t)s.ld * esz * 16 < (1ull << 31);
    return J;
  };
  // Partial buffers, per job: dot [chunks][rows_pad][k] f32, abs [chunks][rows_pad] f32,
  // sq [chunks][rows_pad] f64.
  size_t part_bytes = 0;
  std::vector<size_t> off_dot, off_abs, off_sq;
  auto reserve_part = [&](const PassJob& J) {
    const uint64_t cr = (uint64_t)J.n_chunks * J.rows_pad;
    off_dot.push_back(part_bytes);
    part_bytes = align_up(part_bytes + cr * k * 4, 256);
    off_abs.push_back(part_bytes);
    part_bytes = align_up(part_bytes + cr * 4, 256);
    off_sq.push_back(part_bytes);
    part_bytes = align_up(part_bytes + cr * 8, 256);
  };
  // BR packed + b1 + b2 per product (A pass operands).
  size_t br_bytes = 0;
  std::vector<size_t> off_br, off_b1, off_b2;
  for (size_t i = 0; i < n; i++) {
    const pots_fv_product& p = prods[i];
    PassJob J = make_job({p.q, p.w, p.b_dtype, reinterpret_cast<uint64_t>(p.b), p.ldb});
    jobs.push_back(J);
    reserve_part(J);
    const uint64_t qpad = pad32(p.q);
    off_br.push_back(br_bytes);
    br_bytes = align_up(br_bytes + qpad * (p.a_dtype == DT_BF16 ? 2 * b3_per_row
                                                                : 4 * f4_per_row), 256);
    off_b1.push_back(br_bytes);
    br_bytes = align_up(br_bytes + (uint64_t)p.q * 4, 256);
    off_b2.push_back(br_bytes);
    br_bytes = align_up(br_bytes + (uint64_t)p.q * 4, 256);
    P->bytes += (uint64_t)p.n * p.q * (p.a_dtype == DT_BF16 ? 2 : 4) +
                (uint64_t)p.q * p.w * (p.b_dtype == DT_BF16 ? 2 : 4) +
                (uint64_t)p.n * p.w * (p.p_dtype == DT_BF16 ? 2 : 4);
  }
  for (size_t i = 0; i < n; i++) {
    const pots_fv_product& p = prods[i];
    PassJob J = make_job({p.n, p.q, p.a_dtype, reinterpret_cast<uint64_t>(p.a), p.lda});
    jobs.push_back(J);
    if (twin_of[i] >= 0) {  // its A pass is the twin job's: no row-pass partials
      J.n_chunks = 0;
      J.rows_pad = 0;
    }
    reserve_part(J);
  }
  for (size_t i = 0; i < n; i++) {
    const pots_fv_product& p = prods[i];
    PassJob J = make_job({p.n, p.w, p.p_dtype, reinterpret_cast<uint64_t>(p.p), p.ldp});
    jobs.push_back(J);
    reserve_part(J);
  }
  // Twin partials: m₁'s per tile column [n_ct][rows_pad1], m₂'s per tile row [n_rt][rows_pad2]
  std::vector<TwinJob> tw(twins.size());
  uint64_t twin_tiles = 0;
  for (size_t t = 0; t < twins.size(); t++) {
    const pots_fv_product& p1 = prods[twins[t].first];
    TwinJob& T = tw[t];
    memset(&T, 0, sizeof T);
    T.x = reinterpret_cast<uint64_t>(p1.a);
    T.ld = p1.lda;
    T.rows = p1.n;
    T.cols = p1.q;
    T.rows_pad1 = (T.rows + kRowsPerBlock - 1) / kRowsPerBlock * kRowsPerBlock;
    T.rows_pad2 = (T.cols + kRowsPerBlock - 1) / kRowsPerBlock * kRowsPerBlock;
    T.n_rt = (T.rows + kTwinRows - 1) / kTwinRows;
    T.n_ct = (T.cols + kTwinCols - 1) / kTwinCols;
    T.tile_first = twin_tiles;
    twin_tiles += (uint64_t)T.n_rt * T.n_ct;
    auto put = [&](uint64_t chunks, uint64_t rows_pad, uint64_t& dot, uint64_t& ab,
                   uint64_t& sq) {
      const uint64_t cr = chunks * rows_pad;
      dot = part_bytes;
      part_bytes = align_up(part_bytes + cr * k * 4, 256);
      ab = part_bytes;
      part_bytes = align_up(part_bytes + cr * 4, 256);
      sq = part_bytes;
      part_bytes = align_up(part_bytes + cr * 8, 256);
    };
    put(T.n_ct, T.rows_pad1, T.dot1, T.abs1, T.sq1);  // offsets for now
    put(T.n_rt, T.rows_pad2, T.dot2, T.abs2, T.sq2);
  }
  if (twin_tiles >= 0x7FFFFFFFull) {
    delete P;
    return POTS_E_ARG;
  }
  const size_t o_parts = place(part_bytes);
  const size_t o_br = place(br_bytes);
  // Biases as fp32 are the caller's; the bias pointer is used directly.

  // Group jobs into launches by (dtype, weighted, sq64) and order tiles within each launch.
  struct Pending {
    uint32_t xt, weighted, sq64;
    std::vector<uint32_t> idx;
  };
  auto group = [&](size_t first, size_t count, uint32_t weighted, uint32_t sq64,
                   const uint32_t* dts) {
    std::vector<Pending> out;
    for (uint32_t xt = 0; xt < 2; xt++) {
      Pending pd{xt, weighted, sq64, {}};
      for (size_t i = 0; i < count; i++)
        if (dts[i] == xt) pd.idx.push_back((uint32_t)(first + i));
      if (!pd.idx.empty()) out.push_back(pd);
    }
    return out;
  };
  std::vector<uint32_t> bdt(n), adt(n), pdt(n);
  for (size_t i = 0; i < n; i++) {
    bdt[i] = prods[i].b_dtype;
    adt[i] = prods[i].a_dtype;
    pdt[i] = prods[i].p_dtype;
  }
  for (size_t i = 0; i < n; i++)
    if (twin_of[i] >= 0) adt[i] = 2;  // in no row-pass launch: the twin pass takes its A
  std::vector<Pending> lb = group(0, n, 0, 0, bdt.data());
  std::vector<Pending> la = group(n, n, 1, 0, adt.data());
  std::vector<Pending> lp = group(2 * n, n, 0, 1, pdt.data());
  // Reorder the job array launch by launch and build each launch's block table.
  std::vector<PassJob> ordered;
  std::vector<uint32_t> blk_table;
  std::vector<uint32_t> ordered_src;  // original job index of each ordered job
  auto emit = [&](const std::vector<Pending>& ls, std::vector<PassLaunch>& dst) -> bool {
    for (const Pending& pd : ls) {
      PassLaunch L;
      L.xt = pd.xt;
      L.weighted = pd.weighted;
      L.sq64 = pd.sq64;
      L.njg = njg_for(pd.xt, k);
      L.job_off = ordered.size();
      L.n_jobs = (uint32_t)pd.idx.size();
      L.blk_off = blk_table.size();
      uint64_t blocks = 0;
      for (uint32_t src : pd.idx) {
        PassJob J = jobs[src];
        J.block_first = blocks;
        const uint64_t nb = (uint64_t)J.n_rg * J.n_chunks * J.n_jt;
        blk_table.insert(blk_table.end(), nb, (uint32_t)(ordered.size() - L.job_off));
        blocks += nb;
        ordered.push_back(J);
        ordered_src.push_back(src);
      }
      if (blocks >= 0x7FFFFFFFull) return false;
      L.n_blocks = (uint32_t)blocks;
      dst.push_back(L);
    }
    return true;
  };
  if (!emit(lb, P->pass_b) || !emit(la, P->pass_ap) || !emit(lp, P->pass_ap)) {
    delete P;
    return POTS_E_ARG;
  }
  const size_t o_jobs = place(ordered.size() * sizeof(PassJob));
  const size_t o_blk = place(blk_table.size() * 4);
  const size_t o_twins = place(tw.size() * sizeof(TwinJob));
  const size_t o_twin_tile = place(twin_tiles * 4);
  const size_t o_red = place(n * sizeof(RedJob));
  const size_t o_fin = place(n * sizeof(FinJob));
  // Finish: row slices of every product, the biased products, their bias terms, and one
  // record of 4 + k sums per slice.
  // A thread of a slice adds each of its rows' partials over the chunks in order, so a
  // product with many chunks (a wide A, or a twin's many tiles) gets smaller slices.
  std::vector<uint32_t> a_chunks(n);
  for (size_t i = 0; i < n; i++) a_chunks[i] = jobs[n + i].n_chunks;
  for (size_t t = 0; t < twins.size(); t++) {
    a_chunks[twins[t].first] = tw[t].n_ct;
    a_chunks[twins[t].second] = tw[t].n_rt;
  }
  std::vector<SliceJob> slices;
  std::vector<uint32_t> slice_first(n), slice_rows(n), biased;
  for (size_t i = 0; i < n; i++) {
    const uint32_t chunks = std::max(a_chunks[i], jobs[2 * n + i].n_chunks);
    uint32_t sr = kSliceRows;
    while (sr > 64 && (uint64_t)sr * chunks > 8ull * kSliceRows) sr /= 2;
    slice_rows[i] = sr;
    slice_first[i] = (uint32_t)slices.size();
    for (uint32_t r0 = 0; r0 < prods[i].n; r0 += sr)
      slices.push_back(SliceJob{(uint32_t)i, r0, std::min(prods[i].n, r0 + sr), 0});
    if (prods[i].bias) biased.push_back((uint32_t)i);
  }
  const size_t o_slices = place(slices.size() * sizeof(SliceJob));
  const size_t o_biased = place(biased.size() * 4);
  const size_t o_bout = place(n * sizeof(BiasOut));
  const size_t o_bias_r = place(n * k * 4);
  const size_t o_recs = place(slices.size() * (4 + k) * 8);
  P->total = at;

  hipError_t e = hipMalloc(reinterpret_cast<void**>(&P->base), P->total);
  if (e != hipSuccess) {
    note_hip_error(e, "hipMalloc(freivalds plan)", __FILE__, __LINE__);
    delete P;
    return e == hipErrorOutOfMemory ? POTS_E_NOMEM : POTS_E_HIP;
  }
  // Packed operands: rows past each matrix and unused slots must read as zero (a zero column of
  // X times a NaN would not be zero); the runs rewrite only the used entries.
  e = hipMemset(P->base, 0, P->total);
  if (e != hipSuccess) {
    note_hip_error(e, "hipMemset(freivalds plan)", __FILE__, __LINE__);
    (void)hipFree(P->base);
    delete P;
    return POTS_E_HIP;
  }
  const uint64_t base = reinterpret_cast<uint64_t>(P->base);
  P->d_key = reinterpret_cast<uint32_t*>(P->base + o_key);
  P->d_queue = reinterpret_cast<uint32_t*>(P->base + o_queue);
  P->d_items_b3 = reinterpret_cast<ChallengeItem*>(P->base + o_items_b3);
  P->d_items_f4 = reinterpret_cast<ChallengeItem*>(P->base + o_items_f4);
  P->d_r = reinterpret_cast<float*>(P->base + o_r);
  P->d_r_b3 = reinterpret_cast<uint16_t*>(P->base + o_rb3);
  P->d_r_f4 = reinterpret_cast<float*>(P->base + o_rf4);
  P->d_jobs = reinterpret_cast<PassJob*>(P->base + o_jobs);
  P->d_blk = reinterpret_cast<uint32_t*>(P->base + o_blk);
  P->d_red = reinterpret_cast<RedJob*>(P->base + o_red);
  P->d_fin = reinterpret_cast<FinJob*>(P->base + o_fin);
  P->d_slices = reinterpret_cast<SliceJob*>(P->base + o_slices);
  P->n_slices = (uint32_t)slices.size();
  P->d_biased = reinterpret_cast<uint32_t*>(P->base + o_biased);
  P->n_biased = (uint32_t)biased.size();
  P->d_bout = reinterpret_cast<BiasOut*>(P->base + o_bout);
  P->d_br = reinterpret_cast<float*>(P->base + o_bias_r);
  P->d_recs = reinterpret_cast<double*>(P->base + o_recs);
  P->d_twins = reinterpret_cast<TwinJob*>(P->base + o_twins);
  P->d_twin_tile = reinterpret_cast<uint32_t*>(P->base + o_twin_tile);
  P->n_twins = (uint32_t)tw.size();
  P->n_twin_tiles = (uint32_t)twin_tiles;

  // Fill the job pointers now that addresses are known.
  for (size_t oi = 0; oi < ordered.size(); oi++) {
    PassJob& J = ordered[oi];
    const uint32_t src = ordered_src[oi];
    J.pdot = base + o_parts + off_dot[src];
    J.pabs = base + o_parts + off_abs[src];
    J.psq = base + o_parts + off_sq[src];
    const size_t pi = src % n;
    const pots_fv_product& p = prods[pi];
    if (src < n) {  // B pass: V = R in B's layout
      J.v = p.b_dtype == DT_BF16 ? base + o_rb3 + 2 * items_b3[pi].pk_off
                                 : base + o_rf4 + 4 * items_f4[pi].pk_off;
    } else if (src < 2 * n) {  // A pass: V = packed B·R, weights b1 and b2
      J.v = base + o_br + off_br[pi];
      J.u = base + o_br + off_b1[pi];
      J.w = base + o_br + off_b2[pi];
    } else {  // P pass: V = R in P's layout
      J.v = p.p_dtype == DT_BF16 ? base + o_rb3 + 2 * items_b3[pi].pk_off
                                 : base + o_rf4 + 4 * items_f4[pi].pk_off;
    }
  }
  // The original job index -> ordered position, for the reduction and finish tables.
  std::vector<size_t> pos(jobs.size());
  for (size_t oi = 0; oi < ordered.size(); oi++) pos[ordered_src[oi]] = oi;
  // A B pass of one column chunk for a bf16 A pass writes the reduction's outputs itself
  // (PassJob::pack); the reduction takes the others.
  std::vector<RedJob> red;
  red.reserve(n);
  uint64_t gthreads = 0;
  for (size_t i = 0; i < n; i++) {
    PassJob& J = ordered[pos[i]];
    if (J.n_chunks == 1 && prods[i].a_dtype == DT_BF16 && prods[i].b_dtype == DT_BF16) {
      J.pack = 1u | (twin_of[i] >= 0 ? 2u : 0u);
      J.vout = base + o_br + off_br[i];
      J.uo = base + o_br + off_b1[i];
      J.wo = base + o_br + off_b2[i];
      continue;
    }
    red.emplace_back();
    RedJob& R = red.back();
    R.pdot = J.pdot;
    R.pabs = J.pabs;
    R.psq = J.psq;
    R.vout = base + o_br + off_br[i];
    R.u = base + o_br + off_b1[i];
    R.w = base + o_br + off_b2[i];
    R.group_first = gthreads;
    R.rows = prods[i].q;
    R.rows_pad = J.rows_pad;
    R.n_chunks = J.n_chunks;
    R.a_dt = prods[i].a_dtype;
    R.u_slots = twin_of[i] >= 0;  // a twin's |A|·b1 runs on the matrix cores
    gthreads += (uint64_t)(pad32(prods[i].q) / 8) * k;
  }
  P->n_red = (uint32_t)red.size();
  P->n_red_threads = gthreads;
  std::vector<FinJob> fin(n);
  for (size_t i = 0; i < n; i++) {
    const PassJob& A = ordered[pos[n + i]];
    const PassJob& Pp = ordered[pos[2 * n + i]];
    FinJob& F = fin[i];
    F.a_dot = A.pdot;
    F.a_abs = A.pabs;
    F.a_sq = A.psq;
    F.p_dot = Pp.pdot;
    F.p_abs = Pp.pabs;
    F.p_sq = Pp.psq;
    F.r = base + o_r + 4 * items[i].out_off;
    F.bias = reinterpret_cast<uint64_t>(prods[i].bias);
    F.n = prods[i].n;
    F.w = prods[i].w;
    F.a_rows_pad = A.rows_pad;
    F.a_chunks = A.n_chunks;
    F.p_rows_pad = Pp.rows_pad;
    F.p_chunks = Pp.n_chunks;
    F.slice_first = slice_first[i];
    F.n_slices = (uint32_t)((prods[i].n + slice_rows[i] - 1) / slice_rows[i]);
  }
  std::vector<uint32_t> twin_tile(twin_tiles);
  for (size_t t = 0; t < tw.size(); t++) {
    TwinJob& T = tw[t];
    const uint32_t i1 = twins[t].first, i2 = twins[t].second;
    const uint64_t parts = base + o_parts;
    T.dot1 += parts, T.abs1 += parts, T.sq1 += parts;
    T.dot2 += parts, T.abs2 += parts, T.sq2 += parts;
    T.v1 = base + o_br + off_br[i1];
    T.u1 = base + o_br + off_b1[i1];
    T.w1 = base + o_br + off_b2[i1];
    T.v2 = base + o_br + off_br[i2];
    T.w2 = base + o_br + off_b2[i2];
    FinJob& F1 = fin[i1];
    F1.a_dot = T.dot1, F1.a_abs = T.abs1, F1.a_sq = T.sq1;
    F1.a_rows_pad = T.rows_pad1, F1.a_chunks = T.n_ct;
    FinJob& F2 = fin[i2];
    F2.a_dot = T.dot2, F2.a_abs = T.abs2, F2.a_sq = T.sq2;
    F2.a_rows_pad = T.rows_pad2, F2.a_chunks = T.n_rt;
    std::fill(twin_tile.begin() + T.tile_first,
              twin_tile.begin() + T.tile_first + (uint64_t)T.n_rt * T.n_ct, (uint32_t)t);
  }
  // Upload the tables.
  auto up = [&](size_t off, const void* src, size_t bytes) -> int {
    if (!bytes) return POTS_E_OK;
    POTS_HIP(hipMemcpy(P->base + off, src, bytes, hipMemcpyHostToDevice));
    return POTS_E_OK;
  };
  int rc = POTS_E_OK;
  if ((rc = up(o_items_b3, items_b3.data(), n * sizeof(ChallengeItem))) ||
      (rc = up(o_items_f4, items_f4.data(), n * sizeof(ChallengeItem))) ||
      (rc = up(o_jobs, ordered.data(), ordered.size() * sizeof(PassJob))) ||
      (rc = up(o_blk, blk_table.data(), blk_table.size() * 4)) ||
      (rc = up(o_red, red.data(), red.size() * sizeof(RedJob))) ||
      (rc = up(o_fin, fin.data(), n * sizeof(FinJob))) ||
      (rc = up(o_slices, slices.data(), slices.size() * sizeof(SliceJob))) ||
      (rc = up(o_biased, biased.data(), biased.size() * 4)) ||
      (rc = up(o_twins, tw.data(), tw.size() * sizeof(TwinJob))) ||
      (rc = up(o_twin_tile, twin_tile.data(), twin_tile.size() * 4))) {
    (void)hipFree(P->base);
    delete P;
    return rc;
  }
  P->h_prods.assign(prods, prods + n);
  P->h_r_off.resize(n);
  for (size_t i = 0; i < n; i++) {
    P->h_r_off[i] = items[i].out_off;
    const uint64_t a = reinterpret_cast<uint64_t>(prods[i].p);
    auto it = P->p_index.find(a);
    if (it == P->p_index.end()) P->p_index.emplace(a, (int64_t)i);
    else it->second = -1;  // two products share this P: neither is fused
  }
  P->h_jobs = std::move(ordered);
  P->h_src = std::move(ordered_src);
  P->h_blk = std::move(blk_table);
  P->h_fin = std::move(fin);
  *plan = P;
  return POTS_E_OK;
}

namespace pots {

bool fv_fuse_candidate(void* fv, uint64_t payload, uint64_t len, uint32_t kind,
                       FusedProduct* out) {
  FvPlan* P = static_cast<FvPlan*>(fv);
  if (!P || P->fused || !(P->k == 1 || P->k == 2 || P->k == 4)) return false;
  auto it = P->p_index.find(payload);
  if (it == P->p_index.end() || it->second < 0) return false;
  const uint32_t i = (uint32_t)it->second;
  const pots_fv_product& p = P->h_prods[i];
  const uint32_t esz = p.p_dtype == DT_BF16 ? 2 : 4;
  const bool kind_ok = (p.p_dtype == DT_BF16 && kind == POTS_KIND_BF16) ||
                       (p.p_dtype == DT_F32 && kind == POTS_KIND_F32);
  const uint64_t row_bytes = (uint64_t)p.w * esz;
  if (!kind_ok || p.ldp != p.w || len != (uint64_t)p.n * row_bytes || row_bytes < 1024 ||
      row_bytes >= 0x80000000ull || p.n >= 0x80000000u)
    return false;
  out->r = reinterpret_cast<uint64_t>(P->d_r) + 4 * P->h_r_off[i];
  out->n = p.n;
  out->w = p.w;
  out->esz = esz;
  out->prod = i;
  out->k = P->k;
  return true;
}

int fv_fuse_commit(void* fv, const std::vector<uint32_t>& prods,
                   const std::vector<uint32_t>& head_len, std::vector<uint64_t>* seg_out) {
  FvPlan* P = static_cast<FvPlan*>(fv);
  if (!P || P->fused || prods.size() != head_len.size()) return POTS_E_ARG;
  const size_t n = P->n;
  std::vector<uint8_t> fused(n, 0);
  for (uint32_t i : prods) {
    if (i >= n || fused[i]) return POTS_E_ARG;
    fused[i] = 1;
  }
  // Position of each original job in the ordered array.
  std::vector<size_t> pos(3 * n);
  for (size_t oi = 0; oi < P->h_src.size(); oi++) pos[P->h_src[oi]] = oi;

  // One allocation: the fix-up jobs, then each product's records.
  size_t at = 0;
  auto place = [&](size_t bytes) {
    size_t a = at;
    at = align_up(at + std::max<size_t>(bytes, 16), 256);
    return a;
  };
  const size_t o_fix = place(prods.size() * sizeof(FixJob));
  uint64_t all_rows = 0;
  for (uint32_t i : prods) all_rows += P->h_prods[i].n;
  const uint64_t fix_blocks = (all_rows + 255) / 256;
  const size_t o_fix_blk = place((fix_blocks + 1) * 4);
  std::vector<size_t> o_seg(prods.size());
  for (size_t f = 0; f < prods.size(); f++) {
    const pots_fv_product& p = P->h_prods[prods[f]];
    const uint64_t rb = (uint64_t)p.w * (p.p_dtype == DT_BF16 ? 2 : 4);
    o_seg[f] = place((uint64_t)p.n * ((rb + 1023) / 1024 + 1) * kRunBytes);
  }
  char* fbase = nullptr;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&fbase), at);
  if (e != hipSuccess) {
    note_hip_error(e, "hipMalloc(fused records)", __FILE__, __LINE__);
    return e == hipErrorOutOfMemory ? POTS_E_NOMEM : POTS_E_HIP;
  }
  const uint64_t fb = reinterpret_cast<uint64_t>(fbase);
  std::vector<FixJob> fix(prods.size());
  uint64_t rows = 0;
  seg_out->assign(prods.size(), 0);
  for (size_t f = 0; f < prods.size(); f++) {
    const uint32_t i = prods[f];
    const pots_fv_product& p = P->h_prods[i];
    const PassJob& J = P->h_jobs[pos[2 * n + i]];
    FixJob& x = fix[f];
    memset(&x, 0, sizeof x);
    x.p = reinterpret_cast<uint64_t>(p.p);
    x.r = reinterpret_cast<uint64_t>(P->d_r) + 4 * P->h_r_off[i];
    x.seg = fb + o_seg[f];
    x.pdot = J.pdot;
    x.pabs = J.pabs;
    x.psq = J.psq;
    x.row_first = rows;
    x.n = p.n;
    x.w = p.w;
    x.head = head_len[f];
    x.esz = p.p_dtype == DT_BF16 ? 2 : 4;
    x.J = (uint32_t)(((uint64_t)p.w * x.esz + 1023) / 1024 + 1);
    x.k = P->k;
    rows += p.n;
    (*seg_out)[f] = x.seg;
  }
  std::vector<uint32_t> fix_blk(fix_blocks + 1);
  for (size_t f = 0, b = 0; b < fix_blocks; b++) {
    while (f + 1 < fix.size() && fix[f + 1].row_first <= b * 256) f++;
    fix_blk[b] = (uint32_t)f;
  }
  fix_blk[fix_blocks] = fix.empty() ? 0u : (uint32_t)(fix.size() - 1);
  // The P pass without the fused products: each P launch keeps its other jobs, packed at the
  // front of its ranges of the job array and the block table.
  std::vector<PassLaunch> launches = P->pass_ap;
  std::vector<PassJob> jobs = P->h_jobs;
  std::vector<uint32_t> blk = P->h_blk;
  for (PassLaunch& L : launches) {
    if (L.weighted) continue;  // A pass
    uint32_t kept = 0;
    uint64_t blocks = 0;
    for (uint32_t j = 0; j < L.n_jobs; j++) {
      const size_t oi = L.job_off + j;
      if (fused[P->h_src[oi] - 2 * n]) continue;
      PassJob J = P->h_jobs[oi];
      J.block_first = blocks;
      const uint64_t nb = (uint64_t)J.n_rg * J.n_chunks * J.n_jt;
      std::fill(blk.begin() + L.blk_off + blocks, blk.begin() + L.blk_off + blocks + nb, kept);
      blocks += nb;
      jobs[L.job_off + kept++] = J;
    }
    L.n_jobs = kept;
    L.n_blocks = (uint32_t)blocks;
  }
  std::vector<FinJob> fin = P->h_fin;
  for (uint32_t i : prods) fin[i].p_chunks = 1;
  auto up = [&](void* dst, const void* src, size_t bytes) -> int {
    if (!bytes) return POTS_E_OK;
    POTS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return POTS_E_OK;
  };
  int rc;
  if ((rc = up(fbase + o_fix, fix.data(), fix.size() * sizeof(FixJob))) ||
      (rc = up(fbase + o_fix_blk, fix_blk.data(), fix_blk.size() * 4)) ||
      (rc = up(P->d_jobs, jobs.data(), jobs.size() * sizeof(PassJob))) ||
      (rc = up(P->d_blk, blk.data(), blk.size() * 4)) ||
      (rc = up(P->d_fin, fin.data(), n * sizeof(FinJob)))) {
    // The device tables may be half rewritten: the plan is unusable, and says so.
    P->fused = true;
    P->fbase = fbase;
    P->n_fix = 0;
    return rc;
  }
  P->pass_ap = launches;
  P->h_jobs = std::move(jobs);
  P->h_blk = std::move(blk);
  P->h_fin = std::move(fin);
  P->fused = true;
  P->fbase = fbase;
  P->d_fix = reinterpret_cast<FixJob*>(fbase + o_fix);
  P->d_fix_blk = reinterpret_cast<uint32_t*>(fbase + o_fix_blk);
  P->n_fix = (uint32_t)prods.size();
  P->n_fix_rows = rows;
  return POTS_E_OK;
}

}  // namespace pots

template <uint32_t XT, bool W, bool S, uint32_t NJG>
static void launch_pass(const FvPlan* P, const PassLaunch& L, uint32_t max_grid,
                        uint32_t* queue, hipStream_t s) {
  const bool queued = max_grid != 0 && max_grid < L.n_blocks;
  const uint32_t grid = queued ? max_grid : L.n_blocks;
  if (queued) {  // a block or two per CU beside other work: each lane loads its own V
    hipLaunchKernelGGL(queue_reset, dim3(1), dim3(kQueues), 0, s, queue);
    hipLaunchKernelGGL((row_pass<XT, W, S, NJG, false>), dim3(grid), dim3(256), 0, s,
                       P->d_jobs + L.job_off, P->d_blk + L.blk_off, P->k, L.n_blocks, queue);
  } else {  // a block per tile: the block shares each stage's V through LDS
    hipLaunchKernelGGL((row_pass<XT, W, S, NJG, true>), dim3(grid), dim3(256), 0, s,
                       P->d_jobs + L.job_off, P->d_blk + L.blk_off, P->k, L.n_blocks,
                       nullptr);
  }
}

template <uint32_t XT, bool W, bool S>
static int launch_njg(const FvPlan* P, const PassLaunch& L, uint32_t g, uint32_t* q,
                      hipStream_t s) {
  switch (L.njg) {
    case 1: launch_pass<XT, W, S, 1>(P, L, g, q, s); return POTS_E_OK;
    case 2: launch_pass<XT, W, S, 2>(P, L, g, q, s); return POTS_E_OK;
    case 3: launch_pass<XT, W, S, 3>(P, L, g, q, s); return POTS_E_OK;
    case 4: launch_pass<XT, W, S, 4>(P, L, g, q, s); return POTS_E_OK;
    default: return POTS_E_ARG;
  }
}

// A pass launch of stage `stage` (1 B, 3 A, 4 P) with grid limit g; the stage's tile queue
// counters are the plan's d_queue[kQueues·stage ..].
static int run_pass(const FvPlan* P, const PassLaunch& L, int stage, hipStream_t s) {
  if (L.n_blocks == 0) return POTS_E_OK;
  const uint32_t key = L.xt * 4 + L.weighted * 2 + L.sq64;
  const uint32_t g = P->max_grid[stage];
  uint32_t* q = P->d_queue + (size_t)kQueues * stage;
  int rc;
  switch (key) {
    case 0: rc = launch_njg<DT_F32, false, false>(P, L, g, q, s); break;
    case 1: rc = launch_njg<DT_F32, false, true>(P, L, g, q, s); break;
    case 2: rc = launch_njg<DT_F32, true, false>(P, L, g, q, s); break;
    case 4: rc = launch_njg<DT_BF16, false, false>(P, L, g, q, s); break;
    case 5: rc = launch_njg<DT_BF16, false, true>(P, L, g, q, s); break;
    case 6: rc = launch_njg<DT_BF16, true, false>(P, L, g, q, s); break;
    default: return POTS_E_ARG;
  }
  if (rc != POTS_E_OK) return rc;
  POTS_HIP(hipGetLastError());
  return POTS_E_OK;
}

// One stage of a plan's run: 0 challenges, 1 B pass, 2 reduce of B's vectors, 3 A pass,
// 4 P pass, 5 rows. The stages run in this order on one stream; each reads what the earlier
// ones wrote.
static int run_stage(FvPlan* P, int stage, const uint8_t* d_key, double* d_rows,
                     hipStream_t s) {
  int rc;
  switch (stage) {
    case 0:
      POTS_HIP(hipMemcpyAsync(P->d_key, d_key, 32, hipMemcpyDeviceToDevice, s));
      // R in row-major form (for the bias term and the API) and in the packed layouts.
      if ((rc = challenges_enqueue(P->d_key, P->d_items_b3, P->n_items, P->n_units, P->k,
                                   P->d_r, P->need_b3 ? P->d_r_b3 : nullptr, nullptr, s)) !=
          POTS_E_OK)
        return rc;
      if (P->need_f4 &&
          (rc = challenges_enqueue(P->d_key, P->d_items_f4, P->n_items, P->n_units, P->k,
                                   nullptr, nullptr, P->d_r_f4, s)) != POTS_E_OK)
        return rc;
      return POTS_E_OK;
    case 1:
      for (const PassLaunch& L : P->pass_b)
        if ((rc = run_pass(P, L, 1, s)) != POTS_E_OK) return rc;
      return POTS_E_OK;
    case 2: {
      const uint64_t blocks = (P->n_red_threads + 255) / 256;
      if (blocks == 0) return POTS_E_OK;
      hipLaunchKernelGGL(reduce_b, dim3((uint32_t)blocks), dim3(256), 0, s, P->d_red, P->n_red,
                         P->n_red_threads, P->k);
      POTS_HIP(hipGetLastError());
      return POTS_E_OK;
    }
    case 3:  // the A pass: the row pass over the A's that are no twin's, then the twins'
      if ((rc = run_stage(P, POTS_FV_STAGE_A_ROWS, d_key, d_rows, s)) != POTS_E_OK) return rc;
      return run_stage(P, POTS_FV_STAGE_TWINS, d_key, d_rows, s);
    case POTS_FV_STAGE_A_ROWS:
    case POTS_FV_STAGE_P_PASS:
      for (const PassLaunch& L : P->pass_ap)
        if ((L.weighted != 0) == (stage == POTS_FV_STAGE_A_ROWS) &&
            (rc = run_pass(P, L, stage == POTS_FV_STAGE_A_ROWS ? 3 : 4, s)) != POTS_E_OK)
          return rc;
      return POTS_E_OK;
    case POTS_FV_STAGE_TWINS:
      if (P->n_twin_tiles) {
        const uint32_t g = P->max_grid[3];
        const bool queued = g != 0 && g < P->n_twin_tiles;
        uint32_t* q = P->d_queue + (size_t)kQueues * 3;
        if (queued) hipLaunchKernelGGL(queue_reset, dim3(1), dim3(kQueues), 0, s, q);
        hipLaunchKernelGGL(twin_pass, dim3(queued ? g : P->n_twin_tiles), dim3(256), 0, s,
                           P->d_twins, P->d_twin_tile, P->k, P->n_twin_tiles,
                           queued ? q : nullptr);
        POTS_HIP(hipGetLastError());
      }
      return POTS_E_OK;
    case 4:  // the P pass, then the fused products' records
      if ((rc = run_stage(P, POTS_FV_STAGE_P_PASS, d_key, d_rows, s)) != POTS_E_OK) return rc;
      return run_stage(P, POTS_FV_STAGE_P_FUSED, d_key, d_rows, s);
    case POTS_FV_STAGE_P_FUSED:
      if (P->fused) {
        if (P->n_fix == 0) return POTS_E_HIP;  // a fusion that failed half way
        hipLaunchKernelGGL(fused_rows, dim3((uint32_t)((P->n_fix_rows + 255) / 256)), dim3(256),
                           0, s, P->d_fix, P->d_fix_blk, P->n_fix_rows);
        POTS_HIP(hipGetLastError());
      }
      return POTS_E_OK;
    case 5:
      if (P->n_biased) {
        hipLaunchKernelGGL(bias_terms, dim3(P->n_biased), dim3(256), 0, s, P->d_fin,
                           P->d_biased, P->k, P->d_bout, P->d_br);
        POTS_HIP(hipGetLastError());
      }
      hipLaunchKernelGGL(finish_slices, dim3(P->n_slices), dim3(256), 0, s, P->d_fin,
                         P->d_slices, P->k, P->d_bout, P->d_br, P->d_recs);
      POTS_HIP(hipGetLastError());
      hipLaunchKernelGGL(finish_final, dim3((uint32_t)((P->n + 255) / 256)), dim3(256), 0, s,
                         P->d_fin, (uint32_t)P->n, P->k, P->guard, P->d_bout, P->d_recs,
                         d_rows);
      POTS_HIP(hipGetLastError());
      return POTS_E_OK;
    default:
      return POTS_E_ARG;
  }
}

extern "C" int pots_fv_plan_run(void* plan, const uint8_t* d_key, double* d_rows, void* stream) {
  if (!plan || !d_key || !d_rows) return POTS_E_ARG;
  FvPlan* P = static_cast<FvPlan*>(plan);
  if (P->fused) return POTS_E_ARG;  // stage 4 needs the leaf plan's chunk stage first
  for (int stage = 0; stage < POTS_FV_STAGES; stage++) {
    const int rc = run_stage(P, stage, d_key, d_rows, static_cast<hipStream_t>(stream));
    if (rc != POTS_E_OK) return rc;
  }
  return POTS_E_OK;
}

extern "C" int pots_fv_plan_run_stage(void* plan, int stage, const uint8_t* d_key,
                                      double* d_rows, void* stream) {
  if (!plan || !d_key || !d_rows || stage < 0 || stage > POTS_FV_STAGE_TWINS) return POTS_E_ARG;
  return run_stage(static_cast<FvPlan*>(plan), stage, d_key, d_rows,
                   static_cast<hipStream_t>(stream));
}

extern "C" int pots_fv_plan_set_grid(void* plan, int stage, uint32_t max_blocks) {
  if (!plan || (stage != 1 && stage != 3 && stage != 4)) return POTS_E_ARG;
  static_cast<FvPlan*>(plan)->max_grid[stage] = max_blocks;
  return POTS_E_OK;
}

extern "C" int pots_fv_plan_copy_challenges(const void* plan, float* d_out, void* stream) {
  if (!plan || !d_out) return POTS_E_ARG;
  const FvPlan* P = static_cast<const FvPlan*>(plan);
  POTS_HIP(hipMemcpyAsync(d_out, P->d_r, P->r_floats * 4, hipMemcpyDeviceToDevice,
                          static_cast<hipStream_t>(stream)));
  return POTS_E_OK;
}

extern "C" uint64_t pots_fv_plan_bytes(const void* plan) {
  return plan ? static_cast<const FvPlan*>(plan)->bytes : 0;
}

extern "C" uint32_t pots_fv_plan_twins(const void* plan) {
  return plan ? static_cast<const FvPlan*>(plan)->n_twins : 0;
}

extern "C" void pots_fv_plan_destroy(void* plan) {
  FvPlan* P = static_cast<FvPlan*>(plan);
  if (!P) return;
  if (P->base) (void)hipFree(P->base);
  if (P->fbase) (void)hipFree(P->fbase);
  delete P;
}
