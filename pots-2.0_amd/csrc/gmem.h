// Loads and stores through the global address space.
//
// Pointers that come out of a descriptor in memory are generic (flat) to the compiler, and a
// flat access counts against both the vector-memory and the LDS/scalar wait counters, so the
// compiler waits for everything before using any of it. Casting to address space 1 makes the
// access a global_load/global_store, which waits only for the loads it needs; every pointer
// these helpers take is device memory.
#pragma once

#include <hip/hip_runtime.h>

namespace pots {

#define POTS_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ T gload(const void* p) {
  return *(const POTS_GLOBAL T*)(p);
}

template <typename T>
__device__ __forceinline__ void gstore(void* p, const T& v) {
  *(POTS_GLOBAL T*)(p) = v;
}

// The GPU hands a launch's blocks to its 8 XCDs in turn (block b to XCD b mod 8), and each
// XCD has its own L2. Block b of a launch of n blocks taking unit xcd_block(b, n) gives each
// XCD a contiguous range of units, so neighbouring units that read the same small data (rows
// of R, a column chunk's B·R) run beside one L2 instead of each XCD fetching it. A bijection
// on [0, n).
constexpr uint32_t kXcds = 8;
__device__ __forceinline__ uint32_t xcd_block(uint32_t b, uint32_t n) {
  const uint32_t per = n / kXcds, rem = n % kXcds;
  const uint32_t x = b % kXcds, i = b / kXcds;
  return x < rem ? x * (per + 1) + i : rem * (per + 1) + (x - rem) * per + i;
}

}  // namespace pots
