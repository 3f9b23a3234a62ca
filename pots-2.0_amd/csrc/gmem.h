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

}  // namespace pots
