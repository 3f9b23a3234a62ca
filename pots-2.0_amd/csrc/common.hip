// Host-side helpers: error strings, arenas, pointer classification, version.
#include <string.h>

#include <string>

#include "common.h"

namespace pots {

static thread_local std::string g_last_error;

void note_hip_error(hipError_t e, const char* what, const char* file, int line) {
  char buf[512];
  snprintf(buf, sizeof buf, "%s (%d) from %s at %s:%d", hipGetErrorString(e), (int)e, what,
           file, line);
  g_last_error = buf;
}

void note_error(const std::string& msg) { g_last_error = msg; }

namespace {
constexpr int kMaxDevices = 64;
constexpr int kSlots = 8;
std::mutex g_arena_mu;
Arena g_dev[kMaxDevices][kSlots];
Arena g_host[kMaxDevices][kSlots];
}  // namespace

int arena_get(int slot, size_t bytes, void** out) {
  int dev = 0;
  POTS_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices || slot < 0 || slot >= kSlots) return POTS_E_ARG;
  std::lock_guard<std::mutex> lock(g_arena_mu);
  Arena& a = g_dev[dev][slot];
  if (a.bytes < bytes) {
    if (a.ptr) {
      POTS_HIP(hipDeviceSynchronize());  // earlier work on the old buffer must be done
      POTS_HIP(hipFree(a.ptr));
      a.ptr = nullptr;
      a.bytes = 0;
    }
    size_t want = align_up(bytes < (1u << 20) ? (1u << 20) : bytes + bytes / 4, 4096);
    POTS_HIP(hipMalloc(&a.ptr, want));
    a.bytes = want;
  }
  *out = a.ptr;
  return POTS_E_OK;
}

int pinned_get(int slot, size_t bytes, void** out) {
  int dev = 0;
  POTS_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices || slot < 0 || slot >= kSlots) return POTS_E_ARG;
  std::lock_guard<std::mutex> lock(g_arena_mu);
  Arena& a = g_host[dev][slot];
  if (a.bytes < bytes) {
    if (a.ptr) {
      POTS_HIP(hipDeviceSynchronize());
      POTS_HIP(hipHostFree(a.ptr));
      a.ptr = nullptr;
      a.bytes = 0;
    }
    size_t want = align_up(bytes < (1u << 20) ? (1u << 20) : bytes + bytes / 4, 4096);
    POTS_HIP(hipHostMalloc(&a.ptr, want, hipHostMallocDefault));
    a.bytes = want;
  }
  *out = a.ptr;
  return POTS_E_OK;
}

bool is_device_pointer(const void* p) {
  hipPointerAttribute_t attr;
  memset(&attr, 0, sizeof attr);
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // unregistered host memory reports an error; clear it
    return false;
  }
  return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

}  // namespace pots

extern "C" const char* pots_mi355x_version(void) { return "pots-mi355x 0.1.0 gfx950"; }

extern "C" const char* pots_last_error(void) { return pots::g_last_error.c_str(); }

// One BLAKE3 chunk per lane: a wavefront compresses 64 chunks with each instruction.
extern "C" size_t pots_simd_degree(void) { return 64; }

extern "C" const char* pots_blake3_version(void) { return "spec (gfx950 kernels)"; }
