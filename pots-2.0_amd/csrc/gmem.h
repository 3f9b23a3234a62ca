// Loads and stores through the global address space.
//
// Pointers that come out of a descriptor in memory are generic (flat) to the compiler, and a
// flat access counts against both the vector-memory and the LDS/scalar wait counters, so the
// compiler waits for everything before using any of it. Casting to address space 1 makes the
// access a global_load/global_store, which waits only for the loads it needs; every pointer
// these helpers take is device memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Buffer loads: a 128-bit resource in scalar registers (a wave-uniform base address, no
// range limit below 4 GiB) plus a 32-bit per-lane offset and a 32-bit wave-uniform offset. A
// global load of a 64-bit address needs its address built in vector registers per load, and
// those temporaries can land on registers a load still in flight will write, which makes the
// compiler wait for that load first; a buffer load keeps the address in its offsets.
typedef __amdgpu_buffer_rsrc_t brsrc;

__device__ __forceinline__ brsrc make_rsrc(const void* base) {
  // dword 3: 32-bit data format (gfx9 buffer loads need a valid one), no swizzle
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7FFFFFFF,
                                           0x00020000);
}

typedef uint32_t bload_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bload_u32x4 bload128(brsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(bload_u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
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
