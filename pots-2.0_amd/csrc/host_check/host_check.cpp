// A driver for the sanitized CPU build of libpots_mi355x's host code (host_model.cpp stands in
// for the HIP runtime). Two modes:
//
//   host_check scan FILE...   pots_store_scan over the files (the untrusted prover files of an
//                             on-disk transcript); one line per file with what the scan found,
//                             and for a file it takes, the checksum of the storage bytes that
//                             pots_store_load (host mode) reads from it. Then pots_store_load's
//                             refusals of bad segments and short files.
//   host_check plans SEED N   N randomized Freivalds plans (shapes, strides, dtypes, biases,
//                             twins, k, guard) and leaf plans over their P (fused and not) and
//                             other leaves, each built and destroyed; the twin count and the
//                             refusals are checked against what the generator made.
//
// Exit status 0 when every result is as expected; the sanitizers abort on any finding.

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime.h>

#include <random>
#include <string>
#include <vector>

#include "../../../include/pots_mi355x.h"

namespace {

uint64_t fnv1a(const uint8_t* p, uint64_t n) {
  uint64_t h = 1469598103934665603ull;
  for (uint64_t i = 0; i < n; i++) h = (h ^ p[i]) * 1099511628211ull;
  return h;
}

int scan(int argc, char** argv) {
  const uint32_t n = (uint32_t)(argc - 2);
  std::vector<const char*> paths(argv + 2, argv + argc);
  std::vector<pots_stored_tensor> out(n);
  if (pots_store_scan(n, paths.data(), out.data(), 4) != POTS_E_OK) {
    fprintf(stderr, "pots_store_scan refused its arguments\n");
    return 1;
  }
  for (uint32_t k = 0; k < n; k++) {
    const pots_stored_tensor& r = out[k];
    printf("%d", r.status);
    if (r.status == POTS_STORE_OK) {
      printf(" %u %u %llu %llu %llu", r.ndim, r.dtype, (unsigned long long)r.data_offset,
             (unsigned long long)r.storage_bytes, (unsigned long long)r.storage_offset);
      for (uint32_t d = 0; d < r.ndim && d < POTS_STORE_MAX_DIM; d++)
        printf(" %lld", (long long)r.size[d]);
      printf(" /");
      for (uint32_t d = 0; d < r.ndim && d < POTS_STORE_MAX_DIM; d++)
        printf(" %lld", (long long)r.stride[d]);
      uint64_t h = fnv1a(nullptr, 0);
      if (r.storage_bytes) {
        std::vector<uint8_t> buf(r.storage_bytes);
        pots_store_segment seg{0, 0, r.data_offset, r.storage_bytes, 0};
        const int rc = pots_store_load(1, &paths[k], 1, &seg, buf.data(), -1, nullptr, 0, 2);
        if (rc != POTS_E_OK) {
          fprintf(stderr, "%s: pots_store_load %d: %s\n", paths[k], rc, pots_last_error());
          return 1;
        }
        h = fnv1a(buf.data(), buf.size());
      }
      printf(" %016llx", (unsigned long long)h);
    }
    printf("\n");
  }
  // pots_store_load's own refusals, on the first file
  if (n) {
    uint8_t dst[64];
    const char* p = paths[0];
    const pots_store_segment bad[][2] = {
        {{1, 0, 0, 8, 0}, {0, 0, 0, 0, 0}},   // a file index past the list
        {{0, 0, 0, 0, 0}, {0, 0, 0, 0, 0}},   // an empty segment
        {{0, 0, 0, 16, 8}, {0, 0, 0, 16, 0}},  // out of order
    };
    for (const auto& s : bad)
      if (pots_store_load(1, &p, s[1].bytes ? 2 : 1, s, dst, -1, nullptr, 0, 1) != POTS_E_ARG) {
        fprintf(stderr, "pots_store_load took a bad segment\n");
        return 1;
      }
    pots_store_segment past{0, 0, 1ull << 40, 8, 0};  // past the end of the file
    if (pots_store_load(1, &p, 1, &past, dst, -1, nullptr, 0, 1) != POTS_E_IO) {
      fprintf(stderr, "pots_store_load read past the end of a file\n");
      return 1;
    }
  }
  return 0;
}

struct Rng {
  std::mt19937_64 g;
  explicit Rng(uint64_t seed) : g(seed) {}
  uint64_t below(uint64_t n) { return g() % n; }
  template <class T, size_t N>
  T pick(const T (&xs)[N]) { return xs[below(N)]; }
  bool chance(double p) { return std::uniform_real_distribution<double>(0, 1)(g) < p; }
};

void* device(size_t bytes, std::vector<void*>& owned) {
  void* p = nullptr;
  if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) abort();
  memset(p, 0, bytes ? bytes : 1);
  owned.push_back(p);
  return p;
}

uint64_t g_twins = 0, g_fused = 0;  // what the plans took, over all of them

// One randomized Freivalds plan and the leaf plans over its products' P; false on an
// unexpected outcome.
bool one_plan(Rng& R, int iter) {
  std::vector<void*> owned;
  const uint32_t ks[] = {1, 2, 3, 4, 4, 5, 8, 16};
  const uint32_t k = R.pick(ks);
  const uint32_t ns[] = {1, 3, 16, 17, 64, 100, 128, 256};
  const uint32_t qs[] = {1, 5, 32, 128, 130, 256, 4100};
  const uint32_t ws[] = {1, 7, 32, 33, 512, 600};
  const uint32_t pads[] = {0, 0, 0, 8, 13};
  const size_t np = 1 + R.below(24);
  std::vector<pots_fv_product> prods;
  std::vector<bool> mated;  // a row-major bf16 A already taken as some twin's X
  uint32_t twins = 0;
  for (size_t i = 0; i < np; i++) {
    pots_fv_product p{};
    const bool bf = R.chance(0.7);
    p.a_dtype = bf ? POTS_DT_BF16 : (R.chance(0.8) ? POTS_DT_F32 : POTS_DT_BF16);
    p.b_dtype = bf ? POTS_DT_BF16 : (R.chance(0.8) ? POTS_DT_F32 : POTS_DT_BF16);
    p.p_dtype = R.chance(0.5) ? POTS_DT_BF16 : POTS_DT_F32;
    const size_t es_a = p.a_dtype == POTS_DT_BF16 ? 2 : 4;
    // a twin: A = Xᵀ of an earlier row-major bf16 A that the twin pass can take
    long mate = -1;
    if (k <= 4 && R.chance(0.35)) {
      for (size_t j = 0; j < prods.size(); j++) {
        const pots_fv_product& x = prods[j];
        if (!mated[j] && !x.a_trans && x.a_dtype == POTS_DT_BF16 && x.n % 16 == 0 &&
            x.q % 128 == 0 && (2 * x.lda) % 16 == 0) {
          mate = (long)j;
          break;
        }
      }
    }
    if (mate >= 0) {
      const pots_fv_product& x = prods[(size_t)mate];
      p.a = x.a;
      p.lda = x.lda;
      p.a_trans = 1;
      p.a_dtype = POTS_DT_BF16;
      p.n = x.q;
      p.q = x.n;
      mated[(size_t)mate] = true;
      twins++;
    } else {
      p.n = R.pick(ns);
      p.q = R.pick(qs);
      p.lda = p.q + R.pick(pads) * (R.chance(0.5) ? 8 : 1);
      p.a = device((size_t)p.n * p.lda * es_a, owned);
    }
    p.w = R.pick(ws);
    p.ldb = p.w + R.pick(pads);
    p.ldp = R.chance(0.7) ? p.w : p.w + R.pick(pads);
    p.b = device((size_t)p.q * p.ldb * (p.b_dtype == POTS_DT_BF16 ? 2 : 4), owned);
    p.p = device((size_t)p.n * p.ldp * (p.p_dtype == POTS_DT_BF16 ? 2 : 4), owned);
    p.bias = R.chance(0.2) ? static_cast<const float*>(device(4ull * p.w, owned)) : nullptr;
    p.m = (uint32_t)(i + 1 + R.below(3) * 1000);
    prods.push_back(p);
    mated.push_back(false);
  }
  void* fv = nullptr;
  int rc = pots_fv_plan_create(prods.size(), prods.data(), k, (uint32_t)R.below(2), &fv);
  if (rc != POTS_E_OK) {
    fprintf(stderr, "plan %d: pots_fv_plan_create %d (%s)\n", iter, rc, pots_last_error());
    return false;
  }
  if (pots_fv_plan_twins(fv) != twins || pots_fv_plan_bytes(fv) == 0) {
    fprintf(stderr, "plan %d: %u twins, %u made\n", iter, pots_fv_plan_twins(fv), twins);
    return false;
  }
  g_twins += twins;
  (void)pots_fv_plan_set_grid(fv, 3, (uint32_t)R.below(600));
  (void)pots_fv_plan_set_grid(fv, 1, (uint32_t)R.below(600));

  // leaves: each product's P (header 0x00 || 11 bytes, so the payload may be fused) and a few
  // others of any length
  std::vector<uint8_t> hdr;
  std::vector<uint64_t> hoff, ptr, len;
  std::vector<uint32_t> hlen, hidx;
  std::vector<uint8_t> kind;
  const uint32_t n_hdr = 1 + (uint32_t)R.below(6);
  for (uint32_t h = 0; h < n_hdr; h++) {
    const uint32_t l = h == 0 ? 11 : (uint32_t)R.below(41);
    hoff.push_back(hdr.size());
    hlen.push_back(l);
    for (uint32_t b = 0; b < l; b++) hdr.push_back((uint8_t)R.below(256));
  }
  for (const pots_fv_product& p : prods) {
    hidx.push_back(0);
    ptr.push_back(reinterpret_cast<uint64_t>(p.p));
    len.push_back((uint64_t)p.n * p.ldp * (p.p_dtype == POTS_DT_BF16 ? 2 : 4));
    kind.push_back(p.p_dtype == POTS_DT_BF16 ? POTS_KIND_BF16 : POTS_KIND_F32);
  }
  const size_t extra = R.below(8);
  for (size_t e = 0; e < extra; e++) {
    const uint64_t l = R.chance(0.2) ? 0 : R.below(5000);
    hidx.push_back((uint32_t)R.below(n_hdr));
    ptr.push_back(l ? reinterpret_cast<uint64_t>(device(l, owned)) : 0);
    len.push_back(l);
    kind.push_back((uint8_t)R.below(4));
  }
  const size_t nl = ptr.size();
  for (int fused = 0; fused < 2; fused++) {
    void* leaf = nullptr;
    rc = fused ? pots_leaf_plan_create_fused(nl, hdr.data(), hoff.data(), hlen.data(),
                                             hidx.data(), ptr.data(), len.data(), kind.data(),
                                             fv, &leaf)
               : pots_leaf_plan_create(nl, hdr.data(), hoff.data(), hlen.data(), hidx.data(),
                                       ptr.data(), len.data(), kind.data(), &leaf);
    if (rc != POTS_E_OK) {
      fprintf(stderr, "plan %d: leaf plan (fused %d) %d (%s)\n", iter, fused, rc,
              pots_last_error());
      return false;
    }
    uint64_t msg = 0, chunks = 0, records = 0;
    if (pots_leaf_plan_fused_stats(leaf, &msg, &chunks, &records) != POTS_E_OK ||
        pots_leaf_plan_chunks(leaf) == 0 || (!fused && pots_leaf_plan_fused(leaf) != 0)) {
      fprintf(stderr, "plan %d: leaf plan stats\n", iter);
      return false;
    }
    if (fused) g_fused += pots_leaf_plan_fused(leaf);
    (void)pots_leaf_plan_set_grid(leaf, (uint32_t)R.below(300));
    pots_leaf_plan_destroy(leaf);
  }
  // refusals: a kind out of range; a transposed A with no twin in the plan
  kind[0] = 9;
  void* leaf = nullptr;
  if (pots_leaf_plan_create(nl, hdr.data(), hoff.data(), hlen.data(), hidx.data(), ptr.data(),
                            len.data(), kind.data(), &leaf) != POTS_E_ARG) {
    fprintf(stderr, "plan %d: a bad kind was taken\n", iter);
    return false;
  }
  pots_fv_plan_destroy(fv);
  pots_fv_product lone = prods[0];
  lone.a_trans = 1;
  lone.a_dtype = POTS_DT_BF16;
  void* refused = nullptr;
  if (pots_fv_plan_create(1, &lone, k, 1, &refused) != POTS_E_ARG) {
    fprintf(stderr, "plan %d: a transposed A without a twin was taken\n", iter);
    return false;
  }
  for (void* p : owned) (void)hipFree(p);
  return true;
}

int plans(uint64_t seed, int count) {
  Rng R(seed);
  for (int i = 0; i < count; i++)
    if (!one_plan(R, i)) return 1;
  printf("plans ok: %d (%llu twins, %llu fused leaves)\n", count,
         (unsigned long long)g_twins, (unsigned long long)g_fused);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc >= 2 && !strcmp(argv[1], "scan")) return scan(argc, argv);
  if (argc == 4 && !strcmp(argv[1], "plans"))
    return plans(strtoull(argv[2], nullptr, 10), atoi(argv[3]));
  fprintf(stderr, "usage: host_check scan FILE... | host_check plans SEED COUNT\n");
  return 2;
}
