// Check 6a on gfx950: the SGD update identity of every linear weight, from its committed
// leaves, in one streaming pass.
//
// Reference: verification/verifier/checks.py:380-451 (_update_identity,
// _update_identity_reference) and :301-377 (_fast_rho_max), with the weight's gradient
// G = chain_gradient(its weight-gradient product leaves) (verification/computation/
// interface.py:169-180): the parts widened to fp32 and added in order. Per entry i, in fp32
// with every operation rounded on its own (no contraction), as the reference's torch ops
// round them:
//   ηG_i = fl(η·G_i),  R_i = |W_{t+1,i} − (W_t,i − ηG_i)|,  scale_i = fl(ε_W·(|W_t,i| + |ηG_i|))
// and ρ_i = 0 when R_i = 0, else fl64(R_i) / fl64(scale_i). Per weight the kernel returns
// ρ_max (the maximum, NaN if any ρ_i is NaN, as torch's max), the first index whose R_i or
// scale_i is not finite, and the first index whose ρ_i is not ≤ τ_W; the host words the
// reference's rejection from those.
//
// Work split: a block of 256 threads takes 8192 consecutive entries of one weight, a thread 8
// consecutive entries per step with 16-byte loads (4-byte loads where a pointer is not 16-byte
// aligned, and for a weight's last partial step); each wave reduces its maximum and first
// indices and makes one atomic update per output. ρ_max is kept as the bit pattern of a non-negative double,
// whose unsigned order is its numeric order with NaN above +inf.
#include <math.h>
#include <string.h>

#include <new>
#include <vector>

#include "common.h"
#include "gmem.h"

namespace pots {

constexpr uint32_t kUpdThreads = 256;
constexpr uint32_t kUpdVec = 8;    // consecutive entries a thread takes per step
constexpr uint32_t kUpdSteps = 4;  // steps per block
constexpr uint32_t kUpdTile = kUpdThreads * kUpdVec * kUpdSteps;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct UpdJob {
  uint64_t w_t, w_next;                    // fp32 [n]
  uint64_t parts[POTS_UPDATE_MAX_PARTS];   // gradient parts, [n] each
  uint32_t part_dt[POTS_UPDATE_MAX_PARTS]; // 0 fp32, 1 bf16
  uint32_t n_parts, vec;  // vec: every pointer 16-byte aligned (8-entry vector loads)
  uint64_t n;
  uint64_t block_first;
  double tau_w;
};

struct UpdOut {  // per weight, device side
  uint64_t rho_bits;
  uint64_t first_nonfinite;
  uint64_t first_over;
};
static_assert(sizeof(UpdOut) == sizeof(pots_update_result), "result layout");

__device__ __forceinline__ float load_part(uint64_t base, uint32_t dt, uint64_t i) {
  if (dt == 1) return __uint_as_float((uint32_t)gload<uint16_t>(reinterpret_cast<const uint16_t*>(base) + i) << 16);
  return gload<float>(reinterpret_cast<const float*>(base) + i);
}

__global__ __launch_bounds__(kUpdThreads) void update_init(UpdOut* __restrict__ out, uint32_t n) {
  const uint32_t t = blockIdx.x * kUpdThreads + threadIdx.x;
  if (t < n) {
    out[t].rho_bits = 0;
    out[t].first_nonfinite = ~0ull;
    out[t].first_over = ~0ull;
  }
}

// The per-thread state of the reduction.
struct UpdAcc {
  double rho_max = 0.0;
  bool nan_seen = false;
  uint64_t first_nf = ~0ull, first_over = ~0ull;
  __device__ __forceinline__ void add(float w, float w1, float g, float eta, float eps_w,
                                      double tau_w, uint64_t i) {
    const float eg = eta * g;
    const float r = fabsf(w1 - (w - eg));
    const float s = eps_w * (fabsf(w) + fabsf(eg));
    if (!(isfinite(r) && isfinite(s)) && i < first_nf) first_nf = i;
    const double rho = r == 0.f ? 0.0 : (double)r / (double)s;
    if (rho != rho) nan_seen = true;
    else if (rho > rho_max) rho_max = rho;
    if (!(rho <= tau_w) && i < first_over) first_over = i;
  }
};

__device__ __forceinline__ void load8(const float* p, uint64_t i, float v[8]) {
  const u32x4 a = gload<u32x4>(p + i), b = gload<u32x4>(p + i + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    v[e] = __uint_as_float(a[e]);
    v[4 + e] = __uint_as_float(b[e]);
  }
}

__device__ __forceinline__ void load8_part(uint64_t base, uint32_t dt, uint64_t i, float v[8]) {
  if (dt == 1) {
    const u32x4 a = gload<u32x4>(reinterpret_cast<const uint16_t*>(base) + i);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[2 * e] = __uint_as_float(a[e] << 16);
      v[2 * e + 1] = __uint_as_float(a[e] & 0xFFFF0000u);
    }
  } else {
    load8(reinterpret_cast<const float*>(base), i, v);
  }
}

__global__ __launch_bounds__(kUpdThreads) void update_kernel(const UpdJob* __restrict__ jobs,
                                                             const uint32_t* __restrict__ blk_job,
                                                             float eta, float eps_w,
                                                             UpdOut* __restrict__ out) {
  const uint32_t ji = blk_job[blockIdx.x];
  const UpdJob& J = jobs[ji];
  const uint64_t n = J.n;
  const uint64_t base = (uint64_t)(blockIdx.x - J.block_first) * kUpdTile;
  const float* wt = reinterpret_cast<const float*>(J.w_t);
  const float* wn = reinterpret_cast<const float*>(J.w_next);
  const double tau_w = J.tau_w;
  UpdAcc acc;
#pragma unroll 1
  for (uint32_t st = 0; st < kUpdSteps; st++) {
    const uint64_t i0 = base + ((uint64_t)st * kUpdThreads + threadIdx.x) * kUpdVec;
    if (i0 >= n) break;
    if (J.vec && i0 + kUpdVec <= n) {
      // 8 consecutive entries with 16-byte loads, every load issued before the arithmetic
      float w[8], w1[8], g[8], h[8];
      load8(wt, i0, w);
      load8(wn, i0, w1);
      load8_part(J.parts[0], J.part_dt[0], i0, g);
      for (uint32_t p = 1; p < J.n_parts; p++) {
        load8_part(J.parts[p], J.part_dt[p], i0, h);
#pragma unroll
        for (int e = 0; e < 8; e++) g[e] = g[e] + h[e];
      }
#pragma unroll
      for (int e = 0; e < 8; e++) acc.add(w[e], w1[e], g[e], eta, eps_w, tau_w, i0 + e);
    } else {
      for (uint64_t i = i0; i < i0 + kUpdVec && i < n; i++) {
        float g = load_part(J.parts[0], J.part_dt[0], i);
        for (uint32_t p = 1; p < J.n_parts; p++) g = g + load_part(J.parts[p], J.part_dt[p], i);
        acc.add(gload<float>(wt + i), gload<float>(wn + i), g, eta, eps_w, tau_w, i);
      }
    }
  }
  uint64_t bits = acc.nan_seen ? 0x7FF8000000000000ull
                               : (uint64_t)__double_as_longlong(acc.rho_max);
  uint64_t first_nf = acc.first_nf, first_over = acc.first_over;
  // wave reductions, then one lane per wave updates the weight's outputs
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t b2 = __shfl_xor(bits, o);
    const uint64_t f2 = __shfl_xor(first_nf, o);
    const uint64_t v2 = __shfl_xor(first_over, o);
    bits = b2 > bits ? b2 : bits;
    first_nf = f2 < first_nf ? f2 : first_nf;
    first_over = v2 < first_over ? v2 : first_over;
  }
  if ((threadIdx.x & 63) == 0) {
    UpdOut* o = out + ji;
    if (bits) atomicMax(reinterpret_cast<unsigned long long*>(&o->rho_bits), bits);
    if (first_nf != ~0ull) atomicMin(reinterpret_cast<unsigned long long*>(&o->first_nonfinite), first_nf);
    if (first_over != ~0ull) atomicMin(reinterpret_cast<unsigned long long*>(&o->first_over), first_over);
  }
}

struct UpdatePlan {
  size_t n = 0;
  float eta = 0.f, eps_w = 0.f;
  char* base = nullptr;
  UpdJob* d_jobs = nullptr;
  uint32_t* d_blk = nullptr;
  uint32_t n_blocks = 0;
  uint64_t bytes = 0;  // algorithmic bytes read per run
};

}  // namespace pots

using namespace pots;

extern "C" int pots_update_plan_create(size_t n, const pots_update_weight* weights, float eta,
                                       float eps_w, void** plan) {
  if (!plan || !weights || n == 0 || n >= 0x7FFFFFFFull) return POTS_E_ARG;
  if (!(eta > 0.f) || !isfinite(eta) || !(eps_w > 0.f) || !isfinite(eps_w)) return POTS_E_ARG;
  std::vector<UpdJob> jobs(n);
  std::vector<uint32_t> blk;
  uint64_t bytes = 0;
  for (size_t i = 0; i < n; i++) {
    const pots_update_weight& w = weights[i];
    // an empty weight may come with null data pointers
    if ((w.n && (!w.w_t || !w.w_next)) || w.n_parts < 1 || w.n_parts > POTS_UPDATE_MAX_PARTS)
      return POTS_E_ARG;
    UpdJob& J = jobs[i];
    memset(&J, 0, sizeof J);
    J.w_t = reinterpret_cast<uint64_t>(w.w_t);
    J.w_next = reinterpret_cast<uint64_t>(w.w_next);
    J.n_parts = w.n_parts;
    for (uint32_t p = 0; p < w.n_parts; p++) {
      if ((w.n && !w.parts[p]) || w.part_dtype[p] > 1) return POTS_E_ARG;
      J.parts[p] = reinterpret_cast<uint64_t>(w.parts[p]);
      J.part_dt[p] = w.part_dtype[p];
      bytes += w.n * (w.part_dtype[p] == 1 ? 2 : 4);
    }
    J.n = w.n;
    J.tau_w = w.tau_w;
    bool aligned = (J.w_t % 16 == 0) && (J.w_next % 16 == 0);
    for (uint32_t p = 0; p < w.n_parts; p++) aligned = aligned && J.parts[p] % 16 == 0;
    J.vec = aligned ? 1 : 0;
    J.block_first = blk.size();
    const uint64_t nb = (w.n + kUpdTile - 1) / kUpdTile;
    if (blk.size() + nb >= 0x7FFFFFFFull) return POTS_E_ARG;
    blk.insert(blk.end(), nb, (uint32_t)i);
    bytes += 8 * w.n;
  }
  UpdatePlan* P = new (std::nothrow) UpdatePlan;
  if (!P) return POTS_E_NOMEM;
  P->n = n;
  P->eta = eta;
  P->eps_w = eps_w;
  P->n_blocks = (uint32_t)blk.size();
  P->bytes = bytes;
  const size_t o_blk = align_up(n * sizeof(UpdJob), 256);
  const size_t total = o_blk + std::max<size_t>(blk.size(), 1) * 4;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&P->base), total);
  if (e != hipSuccess) {
    note_hip_error(e, "hipMalloc(update plan)", __FILE__, __LINE__);
    delete P;
    return e == hipErrorOutOfMemory ? POTS_E_NOMEM : POTS_E_HIP;
  }
  P->d_jobs = reinterpret_cast<UpdJob*>(P->base);
  P->d_blk = reinterpret_cast<uint32_t*>(P->base + o_blk);
  e = hipMemcpy(P->d_jobs, jobs.data(), n * sizeof(UpdJob), hipMemcpyHostToDevice);
  if (e == hipSuccess && !blk.empty())
    e = hipMemcpy(P->d_blk, blk.data(), blk.size() * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    note_hip_error(e, "hipMemcpy(update plan)", __FILE__, __LINE__);
    (void)hipFree(P->base);
    delete P;
    return POTS_E_HIP;
  }
  *plan = P;
  return POTS_E_OK;
}

extern "C" int pots_update_plan_run(void* plan, pots_update_result* d_out, void* stream) {
  UpdatePlan* P = static_cast<UpdatePlan*>(plan);
  if (!P || !d_out) return POTS_E_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  UpdOut* out = reinterpret_cast<UpdOut*>(d_out);
  hipLaunchKernelGGL(update_init, dim3((uint32_t)((P->n + kUpdThreads - 1) / kUpdThreads)),
                     dim3(kUpdThreads), 0, s, out, (uint32_t)P->n);
  POTS_HIP(hipGetLastError());
  if (P->n_blocks) {
    hipLaunchKernelGGL(update_kernel, dim3(P->n_blocks), dim3(kUpdThreads), 0, s, P->d_jobs,
                       P->d_blk, P->eta, P->eps_w, out);
    POTS_HIP(hipGetLastError());
  }
  return POTS_E_OK;
}

extern "C" uint64_t pots_update_plan_bytes(void* plan) {
  UpdatePlan* P = static_cast<UpdatePlan*>(plan);
  return P ? P->bytes : 0;
}

extern "C" void pots_update_plan_destroy(void* plan) {
  UpdatePlan* P = static_cast<UpdatePlan*>(plan);
  if (!P) return;
  if (P->base) (void)hipFree(P->base);
  delete P;
}
