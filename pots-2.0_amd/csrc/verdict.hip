// Per-product verdicts of check 5 on gfx950, in IEEE fp64.
//
// Reference: verification/verifier/matmul_check/freivalds.py:324-335 (finish_row), :450-468
// (band_unit, _measure), verification/verifier/matmul_check/sizing.py:16-43 (e_m, term_ratio)
// and verification/verifier/checks.py:926-956 (_judge_product). The arithmetic is the
// reference's Python float arithmetic operation by operation: the same order of operations,
// correctly rounded division and square root, no fused multiply-add (the file is compiled
// with contraction off), and constants (√2, σ_r) passed in from the host as the exact doubles
// Python computes. Comparisons are written "not (x <= bound)" so NaN rejects.
//
// Codes: 0 accept, 1 a non-finite number, 2 the cancellation guard, 3 a residual above τ·unit
// (with the first failing challenge j, 1-based). The smallest rejecting product index goes to
// *first_fail (which the caller initialises to n).
#pragma clang fp contract(off)

#include <math.h>

#include "common.h"

namespace pots {

struct VerdictSpec {
  double kappa_max;
  uint32_t q;       // contraction length of the checked matmul (+1 with a bias)
  uint32_t n;       // rows of A
  uint32_t biased;  // a bias term adds n·‖b‖² to U²
  uint32_t pad;
};
static_assert(sizeof(VerdictSpec) == 24, "VerdictSpec layout");

__device__ __forceinline__ bool finite(double x) { return isfinite(x); }

__global__ __launch_bounds__(256) void verdict_kernel(
    const double* __restrict__ rows, uint32_t k, const VerdictSpec* __restrict__ specs, uint32_t n,
    double eps_in, double eps_acc, double tau, double sigma_r, double sqrt2, uint32_t guard,
    uint32_t judge, int32_t* __restrict__ codes, double* __restrict__ finished,
    uint32_t* __restrict__ first_fail) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const double* r = rows + (uint64_t)i * (5 + k);
  const VerdictSpec s = specs[i];
  const double nu = r[0], p_abs1 = r[1], p_norm = r[2];
  double u2 = r[3];
  if (s.biased) u2 += (double)s.n * r[4];
  const double u = sqrt(u2);
  double kappa;
  if (p_abs1 > 0) kappa = nu / p_abs1;
  else kappa = nu == 0 ? 1.0 : INFINITY;
  // band_unit(q, eps_in, eps_acc, p_norm, u)
  const double sq = sqrt((double)s.q);
  double unit;
  if (p_norm == 0) {
    unit = sigma_r * sq * eps_acc * u;
  } else {
    double ratio;  // term_ratio(p_norm, u) with p_norm != 0
    ratio = u / p_norm;
    double em;
    if (isnan(ratio)) em = NAN;
    else em = sqrt2 * eps_in + sq * eps_acc * (ratio > 1.0 ? ratio : 1.0);
    unit = sigma_r * em * p_norm;
  }
  int32_t code = 0, jfail = 0;
  bool bad = !finite(p_norm) || !finite(u) || !finite(unit);
  if (guard) bad = bad || !finite(nu) || !finite(p_abs1);
  for (uint32_t j = 0; j < k; j++) bad = bad || !finite(r[5 + j]);
  if (bad) {
    code = 1;
  } else if (judge) {
    if (guard && !(nu <= s.kappa_max * p_abs1)) {
      code = 2;
    } else {
      for (uint32_t j = 0; j < k; j++) {
        if (!(r[5 + j] <= tau * unit)) {
          code = 3;
          jfail = (int32_t)j + 1;
          break;
        }
      }
    }
  }
  codes[2 * i] = code;
  codes[2 * i + 1] = jfail;
  if (finished) {
    double* f = finished + (uint64_t)i * 3;
    f[0] = guard ? kappa : NAN;
    f[1] = unit;
    f[2] = u;
  }
  if (code != 0) atomicMin(first_fail, i);
}

__global__ void fill_u32v(uint32_t* p, uint32_t v) { *p = v; }

}  // namespace pots

using namespace pots;

extern "C" int pots_verdicts_async(size_t n, const double* d_rows, uint32_t k,
                                   const void* d_specs, double eps_in, double eps_acc,
                                   double tau, double sigma_r, double sqrt2, uint32_t guard,
                                   uint32_t judge, int32_t* d_codes, double* d_finished,
                                   uint32_t* d_first_fail, void* stream) {
  if (n == 0) return POTS_E_OK;
  if (!d_rows || !d_specs || !d_codes || !d_first_fail || k < 1 || n >= 0xFFFFFFFFull)
    return POTS_E_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_u32v, dim3(1), dim3(1), 0, s, d_first_fail, (uint32_t)n);
  POTS_HIP(hipGetLastError());
  hipLaunchKernelGGL(verdict_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, d_rows,
                     k, static_cast<const VerdictSpec*>(d_specs), (uint32_t)n, eps_in, eps_acc,
                     tau, sigma_r, sqrt2, guard, judge, d_codes, d_finished, d_first_fail);
  POTS_HIP(hipGetLastError());
  return POTS_E_OK;
}
