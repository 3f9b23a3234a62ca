// The outer RFC 6962 Merkle tree over leaf digests, on gfx950.
//
// Reference: verification/commitment/native.c:312-337 (build_tree, pots_merkle_tree) and
// verification/commitment/merkle.py:153-224 (hash_node, _split, merkle_root, _tree_nodes).
//
// The tree is written straight into the pre-order node buffer the reference defines: the node
// of a range [lo, hi) with n > 1 leaves sits at p, its left child (the first k leaves, k the
// largest power of two below n) at p + 1 and its right child at p + 2k. The tree is built
// level by level: at level l the ranges are [j 2^l, min((j + 1) 2^l, n)); a range that fits
// in one level-(l-1) range is the same node as that child (RFC 6962 promotes an unpaired node
// rather than duplicating it), so only ranges longer than 2^(l-1) are hashed, each reading its
// two children from their pre-order slots. One launch per level; each lane finds its node's
// pre-order slot by walking down from the root.
//
// H_node(l, r) = BLAKE3(0x01 || l || r): a 65-byte message, one chunk of two blocks.
#include <string.h>

#include "blake3_device.h"
#include "common.h"

namespace pots {

__device__ __forceinline__ uint64_t split_of(uint64_t s) {  // largest power of two below s >= 2
  return 1ull << (63 - __clzll(s - 1));
}

__device__ __forceinline__ uint64_t preorder_slot(uint64_t lo, uint64_t hi, uint64_t n) {
  uint64_t p = 0, a = 0, b = n;
  while (a != lo || b != hi) {
    const uint64_t k = split_of(b - a);
    if (lo < a + k) {
      p += 1;
      b = a + k;
    } else {
      p += 2 * k;
      a += k;
    }
  }
  return p;
}

__device__ __forceinline__ void load8(const uint8_t* p, uint32_t w[8]) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  const uint4 a = q[0], b = q[1];
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

__device__ __forceinline__ void store8(uint8_t* p, const uint32_t w[8]) {
  uint4* q = reinterpret_cast<uint4*>(p);
  q[0] = make_uint4(w[0], w[1], w[2], w[3]);
  q[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// BLAKE3(0x01 || l || r) of two 32-byte digests given as little-endian words.
__device__ __forceinline__ void hash_node_words(const uint32_t l[8], const uint32_t r[8],
                                                uint32_t out[8]) {
  uint32_t s[16], m[16], cv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    s[i] = l[i];
    s[i + 8] = r[i];
  }
  m[0] = 0x01u | (s[0] << 8);
#pragma unroll
  for (int i = 1; i < 16; i++) m[i] = (s[i - 1] >> 24) | (s[i] << 8);
  b3_iv(cv);
  b3_compress_cv(cv, m, 0, 64, B3_CHUNK_START, cv);
  uint32_t m2[16];
  m2[0] = s[15] >> 24;
#pragma unroll
  for (int i = 1; i < 16; i++) m2[i] = 0;
  b3_compress_cv(cv, m2, 0, 1, B3_CHUNK_END | B3_ROOT, out);
}

__global__ __launch_bounds__(256) void place_leaves(const uint8_t* __restrict__ leaves,
                                                    uint8_t* __restrict__ nodes, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  uint32_t w[8];
  load8(leaves + 32 * i, w);
  store8(nodes + 32 * preorder_slot(i, i + 1, n), w);
}

__global__ __launch_bounds__(256) void tree_level(uint8_t* __restrict__ nodes, uint64_t n,
                                                  uint32_t level) {
  const uint64_t j = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t span = 1ull << level, half = span >> 1;
  const uint64_t lo = j * span;
  if (lo >= n) return;
  const uint64_t hi = min(lo + span, n);
  if (hi - lo <= half) return;  // promoted: the same node as its only child
  const uint64_t p = preorder_slot(lo, hi, n);
  uint32_t l[8], r[8], h[8];
  load8(nodes + 32 * (p + 1), l);
  load8(nodes + 32 * (p + 2 * half), r);
  hash_node_words(l, r, h);
  store8(nodes + 32 * p, h);
}

static int tree_enqueue(size_t n, const uint8_t* d_leaves, uint8_t* d_nodes, hipStream_t s) {
  const uint64_t nb = (n + 255) / 256;
  hipLaunchKernelGGL(place_leaves, dim3((uint32_t)nb), dim3(256), 0, s, d_leaves, d_nodes,
                     (uint64_t)n);
  POTS_HIP(hipGetLastError());
  for (uint32_t level = 1; (1ull << (level - 1)) < n; level++) {
    const uint64_t count = (n + (1ull << level) - 1) >> level;
    hipLaunchKernelGGL(tree_level, dim3((uint32_t)((count + 255) / 256)), dim3(256), 0, s,
                       d_nodes, (uint64_t)n, level);
    POTS_HIP(hipGetLastError());
  }
  return POTS_E_OK;
}

}  // namespace pots

using namespace pots;

extern "C" int pots_merkle_tree_async(size_t n, const uint8_t* d_leaves, uint8_t* d_nodes,
                                      void* stream) {
  if (n == 0 || !d_leaves || !d_nodes) return POTS_E_ARG;
  return tree_enqueue(n, d_leaves, d_nodes, static_cast<hipStream_t>(stream));
}

extern "C" int pots_merkle_tree(size_t n, const uint8_t* leaves, uint8_t* nodes) {
  if (n == 0 || !leaves || !nodes) return POTS_E_ARG;
  const bool dev_in = is_device_pointer(leaves), dev_out = is_device_pointer(nodes);
  const size_t in_bytes = 32 * n, out_bytes = 32 * (2 * n - 1);
  const uint8_t* d_in = leaves;
  uint8_t* d_out = nodes;
  int rc;
  if (!dev_in || !dev_out) {
    void* buf = nullptr;
    if ((rc = arena_get(2, align_up(in_bytes, 256) + out_bytes, &buf)) != POTS_E_OK) return rc;
    if (!dev_in) {
      POTS_HIP(hipMemcpy(buf, leaves, in_bytes, hipMemcpyHostToDevice));
      d_in = static_cast<const uint8_t*>(buf);
    }
    if (!dev_out) d_out = static_cast<uint8_t*>(buf) + align_up(in_bytes, 256);
  }
  if ((rc = tree_enqueue(n, d_in, d_out, 0)) != POTS_E_OK) return rc;
  if (!dev_out) POTS_HIP(hipMemcpy(nodes, d_out, out_bytes, hipMemcpyDeviceToHost));
  else POTS_HIP(hipDeviceSynchronize());
  return POTS_E_OK;
}
