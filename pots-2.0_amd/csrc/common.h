// Shared host-side helpers of libpots_mi355x: error codes, HIP error mapping and a per-device
// grow-only scratch arena for the synchronous entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/pots_mi355x.h"

namespace pots {

// Remember the first HIP error of the current call and turn it into POTS_E_HIP.
#define POTS_HIP(expr)                                                                    \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess) {                                                               \
      ::pots::note_hip_error(e_, #expr, __FILE__, __LINE__);                              \
      return e_ == hipErrorOutOfMemory ? POTS_E_NOMEM : POTS_E_HIP;                       \
    }                                                                                     \
  } while (0)

void note_hip_error(hipError_t e, const char* what, const char* file, int line);

// Set the calling thread's pots_last_error() text.
void note_error(const std::string& msg);

// A device buffer that only grows, one per (device, slot), kept for the life of the process.
// The synchronous entry points use it for metadata and intermediate chaining values; the
// stream-ordered ones take caller-provided workspace instead.
struct Arena {
  void* ptr = nullptr;
  size_t bytes = 0;
};

int arena_get(int slot, size_t bytes, void** out);

// Pinned host staging of the same kind.
int pinned_get(int slot, size_t bytes, void** out);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Whether `p` is device memory of the current device (or managed), as opposed to host memory.
bool is_device_pointer(const void* p);

}  // namespace pots
