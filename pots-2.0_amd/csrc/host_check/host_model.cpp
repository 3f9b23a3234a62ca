// A host model of the HIP runtime calls that libpots_mi355x's host code makes, for a CPU-only
// build of that code under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU, no HIP
// runtime): device memory is host memory from malloc, copies and fills are memcpy and memset,
// streams and events are complete as soon as they are made, and a kernel launch fails. The
// plan builders and the store reader run on it unchanged, every host-side access checked.
//
// Pointer attributes report memory from hipMalloc as device memory and anything else as
// unregistered host memory, as the runtime does. A __device__ variable registered by the
// library gets a zeroed host buffer of its size, which hipGetSymbolAddress returns.

#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>

namespace {

// Made on first use: the library's module constructors register their __device__
// variables before this file's own globals would be constructed.
struct State {
  std::mutex mu;
  std::map<uintptr_t, size_t> device;     // base → bytes of each hipMalloc allocation
  std::map<const void*, void*> symbols;   // host shadow of a __device__ variable → its memory
};

State& state() {
  static State* s = new State;  // never destroyed: registrations may outlive static teardown
  return *s;
}

thread_local hipError_t g_last = hipSuccess;
int g_event_tag, g_stream_tag;

hipError_t set(hipError_t e) {
  if (e != hipSuccess) g_last = e;
  return e;
}

bool on_device(const void* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  State& st = state();
  std::lock_guard<std::mutex> lock(st.mu);
  auto it = st.device.upper_bound(a);
  if (it == st.device.begin()) return false;
  --it;
  return a < it->first + it->second || (it->second == 0 && a == it->first);
}

}  // namespace

extern "C" {

hipError_t hipMalloc(void** ptr, size_t size) {
  if (!ptr) return set(hipErrorInvalidValue);
  void* p = malloc(size ? size : 1);
  if (!p) return set(hipErrorOutOfMemory);
  State& st = state();
  std::lock_guard<std::mutex> lock(st.mu);
  st.device[reinterpret_cast<uintptr_t>(p)] = size;
  *ptr = p;
  return hipSuccess;
}

hipError_t hipFree(void* ptr) {
  if (!ptr) return hipSuccess;
  State& st = state();
  std::lock_guard<std::mutex> lock(st.mu);
  auto it = st.device.find(reinterpret_cast<uintptr_t>(ptr));
  if (it == st.device.end()) return set(hipErrorInvalidValue);
  st.device.erase(it);
  free(ptr);
  return hipSuccess;
}

hipError_t hipHostMalloc(void** ptr, size_t size, unsigned int) {
  if (!ptr) return set(hipErrorInvalidValue);
  *ptr = malloc(size ? size : 1);
  return *ptr ? hipSuccess : set(hipErrorOutOfMemory);
}

hipError_t hipHostFree(void* ptr) {
  free(ptr);
  return hipSuccess;
}

hipError_t hipMemcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind) {
  if (bytes && (!dst || !src)) return set(hipErrorInvalidValue);
  if (bytes) memmove(dst, src, bytes);
  return hipSuccess;
}

hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind,
                          hipStream_t) {
  return hipMemcpy(dst, src, bytes, kind);
}

hipError_t hipMemset(void* dst, int value, size_t bytes) {
  if (bytes && !dst) return set(hipErrorInvalidValue);
  if (bytes) memset(dst, value, bytes);
  return hipSuccess;
}

hipError_t hipPointerGetAttributes(hipPointerAttribute_t* attr, const void* ptr) {
  if (!attr) return set(hipErrorInvalidValue);
  memset(attr, 0, sizeof *attr);
  if (!on_device(ptr)) return set(hipErrorInvalidValue);  // unregistered host memory
  attr->type = hipMemoryTypeDevice;
  attr->device = 0;
  attr->devicePointer = const_cast<void*>(ptr);
  return hipSuccess;
}

hipError_t hipGetDevice(int* device) {
  if (!device) return set(hipErrorInvalidValue);
  *device = 0;
  return hipSuccess;
}

hipError_t hipSetDevice(int device) {
  return device == 0 ? hipSuccess : set(hipErrorInvalidDevice);
}

hipError_t hipDeviceSynchronize(void) { return hipSuccess; }

hipError_t hipGetLastError(void) {
  const hipError_t e = g_last;
  g_last = hipSuccess;
  return e;
}

const char* hipGetErrorString(hipError_t e) {
  switch (e) {
    case hipSuccess: return "no error";
    case hipErrorInvalidValue: return "invalid argument (host model)";
    case hipErrorOutOfMemory: return "out of memory (host model)";
    case hipErrorNoDevice: return "no device: the host model launches no kernel";
    default: return "error (host model)";
  }
}

hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned int) {
  if (!stream) return set(hipErrorInvalidValue);
  *stream = reinterpret_cast<hipStream_t>(&g_stream_tag);
  return hipSuccess;
}

hipError_t hipStreamDestroy(hipStream_t) { return hipSuccess; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }

hipError_t hipEventCreateWithFlags(hipEvent_t* event, unsigned) {
  if (!event) return set(hipErrorInvalidValue);
  *event = reinterpret_cast<hipEvent_t>(&g_event_tag);
  return hipSuccess;
}

hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventDestroy(hipEvent_t) { return hipSuccess; }

hipError_t hipLaunchKernel(const void*, dim3, dim3, void**, size_t, hipStream_t) {
  return set(hipErrorNoDevice);
}

hipError_t hipGetSymbolAddress(void** dev_ptr, const void* symbol) {
  if (!dev_ptr) return set(hipErrorInvalidValue);
  State& st = state();
  std::lock_guard<std::mutex> lock(st.mu);
  auto it = st.symbols.find(symbol);
  if (it == st.symbols.end()) return set(hipErrorInvalidSymbol);
  *dev_ptr = it->second;
  return hipSuccess;
}

// What the compiler's module constructors call for each translation unit with kernels.
void** __hipRegisterFatBinary(const void*) {
  static void* module = nullptr;
  return &module;
}

void __hipUnregisterFatBinary(void**) {}

void __hipRegisterFunction(void**, const void*, char*, const char*, unsigned int, uint3*,
                           uint3*, dim3*, dim3*, int*) {}

void __hipRegisterVar(void**, void* var, char*, char*, int, size_t size, int, int) {
  void* mem = calloc(1, size ? size : 1);
  if (!mem) abort();
  State& st = state();
  std::lock_guard<std::mutex> lock(st.mu);
  st.device[reinterpret_cast<uintptr_t>(mem)] = size;
  st.symbols[var] = mem;
}

hipError_t __hipPushCallConfiguration(dim3, dim3, size_t, hipStream_t) { return hipSuccess; }

hipError_t __hipPopCallConfiguration(dim3* grid, dim3* block, size_t* shared,
                                     hipStream_t* stream) {
  if (grid) *grid = dim3(1, 1, 1);
  if (block) *block = dim3(1, 1, 1);
  if (shared) *shared = 0;
  if (stream) *stream = nullptr;
  return hipSuccess;
}

}  // extern "C"
