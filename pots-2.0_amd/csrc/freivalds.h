// Shared definitions of the Fiat-Shamir and Freivalds kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace pots {

// One challenge matrix: product label m, its width (rows of R), where its row-major [width, k]
// fp32 copy goes (float offset) and where its packed copy goes (element offset), and the
// prefix of 16-row XOF units over the items before it.
struct ChallengeItem {
  uint32_t m;
  uint32_t width;
  uint64_t out_off;
  uint64_t pk_off;
  uint64_t unit_first;
};
static_assert(sizeof(ChallengeItem) == 32, "ChallengeItem layout");

// The packed operands of the row pass hold each K-group of PER rows (8 for bf16 X, 4 for
// fp32 X) as groups of 16 slots of PER values: slot 3·jl + t of group jg is term t of
// challenge column 5·jg + jl for bf16 X (hi, mid, lo), slot jl of group jg is column
// 16·jg + jl for fp32 X. The slots of K-group G, group jg start at ((G·n_jg + jg)·16) · PER
// elements.
__host__ __device__ inline uint32_t groups_b3(uint32_t k) { return (k + 4) / 5; }
__host__ __device__ inline uint32_t groups_f4(uint32_t k) { return (k + 15) / 16; }

int challenges_enqueue(const uint32_t* d_key, const ChallengeItem* d_items, uint32_t n_items,
                       uint64_t n_units, uint32_t k, float* d_out, uint16_t* d_b3, float* d_f4,
                       hipStream_t s);

// ---- P-pass sums taken by the chunk kernel (a leaf plan fused with a Freivalds plan) ------
//
// A product whose P is a leaf of the transcript has its P-pass sums (P·R_j, Σ|p|, Σp² per
// row) taken by the leaf hasher while it streams that leaf, so P is read from HBM once for
// both checks. The hasher cuts each row into runs (the elements of one row inside one 1 KiB
// chunk) and writes one record per run: [J][n] records of kRunBytes, J = ceil(w·esz / 1024)
// + 1 slots per row, slot s of row i (at s·n + i) for the s-th chunk its elements fall in; a
// wave's lanes hold one class of chunks, which puts their records side by side. The
// Freivalds plan then adds each row's records and the few elements no chunk took (the leaf's
// first bytes up to a 128-byte boundary and its last bytes after one) in a fixed order.

constexpr uint32_t kRunBytes = 32;  // float d[4], float s1, exact flag, double s2

// What the leaf plan needs of a product it fuses.
struct FusedProduct {
  uint64_t r;     // R [w][k] fp32, row-major
  uint32_t n, w;  // P's rows and columns
  uint32_t esz;   // 2 (bf16) or 4 (fp32)
  uint32_t prod;  // index of the product in the plan
  uint32_t k;     // the plan's challenges per product: 1, 2 or 4
};

// The product of `fv` whose P is this leaf's payload, if it can be fused: k of 1, 2 or 4, P
// contiguous with the leaf's kind, rows of at least 1 KiB, not yet fused. Returns false
// otherwise.
bool fv_fuse_candidate(void* fv, uint64_t payload, uint64_t len, uint32_t kind,
                       FusedProduct* out);

// Fuse the chosen products: their P-pass sums come from run records from now on. Allocates
// the records (seg_out[i] for prods[i]) and rebuilds the P pass without them. head_len[i] is
// the bytes of 0x00 || header before product i's payload in its leaf message. A plan is fused
// at most once. Returns POTS_E_*.
int fv_fuse_commit(void* fv, const std::vector<uint32_t>& prods,
                   const std::vector<uint32_t>& head_len, std::vector<uint64_t>* seg_out);

// An fp32 value v as three bf16 terms hi + mid + lo == v exactly: each term keeps the top 8
// significant bits of what is left (truncation toward zero leaves a remainder that is exact in
// fp32, and after two terms at most 8 significant bits remain). So an MFMA over bf16 operands
// with fp32 accumulation multiplies a bf16 matrix by v with exact products.
__device__ __forceinline__ void split_bf16x3(float v, uint16_t& hi, uint16_t& mid,
                                             uint16_t& lo) {
  const uint32_t b0 = __float_as_uint(v);
  hi = (uint16_t)(b0 >> 16);
  const float r1 = v - __uint_as_float(b0 & 0xFFFF0000u);
  const uint32_t b1 = __float_as_uint(r1);
  mid = (uint16_t)(b1 >> 16);
  const float r2 = r1 - __uint_as_float(b1 & 0xFFFF0000u);
  lo = (uint16_t)(__float_as_uint(r2) >> 16);
}

}  // namespace pots
