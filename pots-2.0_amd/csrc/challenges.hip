// Fiat-Shamir challenge matrices on gfx950.
//
// Reference: verification/verifier/matmul_check/challenges.py:22-106 and
// verification/commitment/native.c:50-139 (fill_rows, pots_challenges). Vector j of product m
// is the keyed BLAKE3 XOF of the 6-byte label 0x10 || m (4 bytes BE) || j, key = the claimed
// root h; its 4·width output bytes read as little-endian words w give the entries
// (2(w >> 8) + 1 - 2^24) / 2^24, exact in fp32. Item i's matrix is [width_i, k], row-major,
// vector j in column j - 1.
//
// The label fits one block of one chunk, so XOF output block t (entries 16t .. 16t+15) is
// one compression of that block with counter t and flags KEYED_HASH | CHUNK_START |
// CHUNK_END | ROOT, all 16 output words kept. One lane computes one block of one vector;
// lanes are ordered (item, t, j) with j fastest, so the k lanes of a row block write
// neighbouring columns.
//
// Besides the row-major matrix, a lane can write the same entries in the two operand
// layouts the Freivalds row pass reads (freivalds.h): "bf16x3" (each fp32 entry as three
// bf16 terms whose sum is exact, 8 rows per K-group) and "f32x4" (fp32, 4 rows per K-group).
// Rows past `width` up to the next multiple of 16 are written as zero.
#include <string.h>

#include <new>
#include <vector>

#include "blake3_device.h"
#include "common.h"
#include "freivalds.h"

namespace pots {

__global__ __launch_bounds__(256) void xof_kernel(const uint32_t* __restrict__ key,
                                                  const ChallengeItem* __restrict__ items,
                                                  uint32_t n_items, uint64_t n_threads,
                                                  uint32_t k, float* __restrict__ out,
                                                  uint16_t* __restrict__ out_b3,
                                                  float* __restrict__ out_f4) {
  const uint64_t g = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= n_threads) return;
  const uint64_t unit = g / k;
  const uint32_t j = (uint32_t)(g - unit * k);  // 0-based vector
  uint32_t lo = 0, hi = n_items - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) >> 1;
    if (items[mid].unit_first <= unit) lo = mid;
    else hi = mid - 1;
  }
  const ChallengeItem it = items[lo];
  const uint32_t t = (uint32_t)(unit - it.unit_first);
  uint32_t cv[8], m[16], w[16];
#pragma unroll
  for (int i = 0; i < 8; i++) cv[i] = key[i];
  const uint32_t mm = it.m, jj = j + 1;
  // Label bytes 0x10, m >> 24, m >> 16, m >> 8, m, j, then zero padding.
  m[0] = 0x10u | ((mm >> 24) & 0xFFu) << 8 | ((mm >> 16) & 0xFFu) << 16 | ((mm >> 8) & 0xFFu) << 24;
  m[1] = (mm & 0xFFu) | jj << 8;
#pragma unroll
  for (int i = 2; i < 16; i++) m[i] = 0;
  b3_compress_xof(cv, m, t, 6, B3_KEYED_HASH | B3_CHUNK_START | B3_CHUNK_END | B3_ROOT, w);
  float r[16];
#pragma unroll
  for (int s = 0; s < 16; s++) {
    const int32_t num = 2 * (int32_t)(w[s] >> 8) + 1 - (1 << 24);
    r[s] = (16u * t + s < it.width) ? (float)num * 0x1p-24f : 0.0f;
  }
  if (out) {
    float* col = out + it.out_off + j;
#pragma unroll
    for (int s = 0; s < 16; s++)
      if (16u * t + s < it.width) col[(uint64_t)(16u * t + s) * k] = r[s];
  }
  if (out_b3) {
    // K-groups 2t and 2t + 1 (8 rows each); the three terms of column j go to slots
    // 3(j mod 5) + term of group j / 5.
    const uint32_t njg = groups_b3(k), jg = j / 5, slot = 3 * (j % 5);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      uint16_t pl[3][8];
#pragma unroll
      for (int e = 0; e < 8; e++) split_bf16x3(r[8 * h + e], pl[0][e], pl[1][e], pl[2][e]);
      uint16_t* grp = out_b3 + it.pk_off + (((uint64_t)(2 * t + h) * njg + jg) * 16 + slot) * 8;
#pragma unroll
      for (int p = 0; p < 3; p++)
        *reinterpret_cast<uint4*>(grp + 8 * p) =
            make_uint4(pl[p][0] | (uint32_t)pl[p][1] << 16, pl[p][2] | (uint32_t)pl[p][3] << 16,
                       pl[p][4] | (uint32_t)pl[p][5] << 16, pl[p][6] | (uint32_t)pl[p][7] << 16);
    }
  }
  if (out_f4) {
    // K-groups 4t .. 4t + 3 (4 rows each); column j in slot j mod 16 of group j / 16.
    const uint32_t njg = groups_f4(k), jg = j / 16, slot = j % 16;
#pragma unroll
    for (int h = 0; h < 4; h++) {
      float4* dst = reinterpret_cast<float4*>(
          out_f4 + it.pk_off + (((uint64_t)(4 * t + h) * njg + jg) * 16 + slot) * 4);
      *dst = make_float4(r[4 * h], r[4 * h + 1], r[4 * h + 2], r[4 * h + 3]);
    }
  }
}

int challenges_enqueue(const uint32_t* d_key, const ChallengeItem* d_items, uint32_t n_items,
                       uint64_t n_units, uint32_t k, float* d_out, uint16_t* d_b3, float* d_f4,
                       hipStream_t s) {
  if (n_items == 0) return POTS_E_OK;
  const uint64_t threads = n_units * k;
  const uint64_t blocks = (threads + 255) / 256;
  if (blocks >= 0x7FFFFFFFull) return POTS_E_ARG;
  hipLaunchKernelGGL(xof_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, d_key, d_items,
                     n_items, threads, k, d_out, d_b3, d_f4);
  POTS_HIP(hipGetLastError());
  return POTS_E_OK;
}

}  // namespace pots

using namespace pots;

extern "C" int pots_challenges(const uint8_t key[32], uint32_t k, size_t n, const uint32_t* ms,
                               const uint32_t* widths, const uint64_t* offsets, float* out,
                               uint32_t n_threads) {
  (void)n_threads;
  if (n == 0) return POTS_E_OK;
  if (!key || !ms || !widths || !offsets || !out || k < 1 || k > 255 || n >= 0xFFFFFFFFull)
    return POTS_E_ARG;
  std::vector<ChallengeItem> items(n);
  uint64_t units = 0, end = 0;
  for (size_t i = 0; i < n; i++) {
    if (ms[i] == 0 || widths[i] == 0) return POTS_E_ARG;
    items[i] = ChallengeItem{ms[i], widths[i], offsets[i], 0, units};
    units += (widths[i] + 15) / 16;
    end = std::max<uint64_t>(end, offsets[i] + (uint64_t)widths[i] * k);
  }
  const bool dev_out = is_device_pointer(out);
  const size_t meta = align_up(32 + n * sizeof(ChallengeItem), 256);
  void* buf = nullptr;
  int rc;
  if ((rc = arena_get(5, meta + (dev_out ? 0 : end * 4), &buf)) != POTS_E_OK) return rc;
  char* b = static_cast<char*>(buf);
  POTS_HIP(hipMemcpy(b, key, 32, hipMemcpyHostToDevice));
  POTS_HIP(hipMemcpy(b + 32, items.data(), n * sizeof(ChallengeItem), hipMemcpyHostToDevice));
  float* d_out = dev_out ? out : reinterpret_cast<float*>(b + meta);
  if ((rc = challenges_enqueue(reinterpret_cast<const uint32_t*>(b),
                               reinterpret_cast<const ChallengeItem*>(b + 32), (uint32_t)n,
                               units, k, d_out, nullptr, nullptr, 0)) != POTS_E_OK)
    return rc;
  if (!dev_out) {
    // Copy back only what the items cover (the caller's buffer may hold other data between).
    for (size_t i = 0; i < n; i++)
      POTS_HIP(hipMemcpy(out + offsets[i], d_out + offsets[i], (size_t)widths[i] * k * 4,
                         hipMemcpyDeviceToHost));
  } else {
    POTS_HIP(hipDeviceSynchronize());
  }
  return POTS_E_OK;
}
