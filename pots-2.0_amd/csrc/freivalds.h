// Shared definitions of the Fiat-Shamir and Freivalds kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
