// The NaN/Inf test of one buffer on gfx950 (reference: verification/commitment/native.c:146-169
// block_finite and :263-308 pots_all_finite). The leaf-hashing kernel fuses the same test
// into its loads; this entry point serves callers that test one buffer alone.
#include "common.h"

namespace pots {

// Word-granular scan: a trailing partial value is ignored, as in the reference.
__global__ __launch_bounds__(256) void finite_kernel(const uint32_t* __restrict__ p,
                                                     uint64_t words, uint32_t kind,
                                                     uint32_t* __restrict__ bad) {
  const bool halves = kind != POTS_KIND_F32;
  const uint32_t thr = kind == POTS_KIND_F16 ? 0xF8000000u : 0xFF000000u;
  uint32_t acc = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < words;
       i += (uint64_t)gridDim.x * 256) {
    const uint32_t w = p[i];
    acc = max(acc, max(w << 1, halves ? w << 17 : 0u));
  }
  if (acc >= thr) atomicOr(bad, 1u);
}

__global__ void finite_tail16(const uint16_t* __restrict__ p, uint32_t kind,
                              uint32_t* __restrict__ bad) {
  const uint16_t mask = kind == POTS_KIND_BF16 ? 0x7f80 : 0x7c00;
  if ((uint16_t)(*p & mask) == mask) atomicOr(bad, 1u);
}

}  // namespace pots

using namespace pots;

extern "C" int pots_all_finite(const uint8_t* p, uint64_t nbytes, uint8_t kind,
                               uint32_t n_threads) {
  (void)n_threads;
  if (nbytes == 0 || kind < POTS_KIND_F32 || kind > POTS_KIND_F16) return 1;
  if (!p) return POTS_E_ARG;
  void* buf = nullptr;
  int rc;
  const bool dev = is_device_pointer(p);
  const uint8_t* d = p;
  const uint64_t vbytes = kind == POTS_KIND_F32 ? nbytes / 4 * 4 : nbytes / 2 * 2;
  if ((rc = arena_get(3, dev ? 256 : align_up(vbytes, 256) + 256, &buf)) != POTS_E_OK) return rc;
  uint32_t* d_bad = static_cast<uint32_t*>(buf);
  if (!dev) {
    d = static_cast<uint8_t*>(buf) + 256;
    POTS_HIP(hipMemcpy(const_cast<uint8_t*>(d), p, vbytes, hipMemcpyHostToDevice));
  }
  if (reinterpret_cast<uintptr_t>(d) % 4 != 0) {
    // An unaligned device view: copy it to an aligned buffer first.
    void* al = nullptr;
    if ((rc = arena_get(4, align_up(vbytes, 256), &al)) != POTS_E_OK) return rc;
    POTS_HIP(hipMemcpy(al, d, vbytes, hipMemcpyDeviceToDevice));
    d = static_cast<const uint8_t*>(al);
  }
  POTS_HIP(hipMemset(d_bad, 0, 4));
  const uint64_t words = vbytes / 4;
  if (words) {
    uint64_t blocks = (words + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(finite_kernel, dim3((uint32_t)blocks), dim3(256), 0, 0,
                       reinterpret_cast<const uint32_t*>(d), words, (uint32_t)kind, d_bad);
    POTS_HIP(hipGetLastError());
  }
  if (vbytes % 4)  // one trailing 16-bit value
    hipLaunchKernelGGL(finite_tail16, dim3(1), dim3(1), 0, 0,
                       reinterpret_cast<const uint16_t*>(d + words * 4), (uint32_t)kind, d_bad);
  uint32_t h = 0;
  POTS_HIP(hipMemcpy(&h, d_bad, 4, hipMemcpyDeviceToHost));
  return h ? 0 : 1;
}
