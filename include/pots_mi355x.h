/* libpots_mi355x — the C ABI of the MI355X verifier and commitment engine.
 *
 * Everything here runs on the current HIP device (gfx950). Pointers are plain addresses; a
 * "device" argument must be device memory of the current device, a "host" argument host
 * memory, and an argument documented as "host or device" may be either (the library asks HIP
 * which it is). Streams are passed as `void *` holding a hipStream_t (0 = the null stream).
 * No entry point throws; each returns a status (POTS_E_*) or a documented value, and
 * pots_last_error() describes the last HIP failure of the calling thread.
 *
 * The first group mirrors the reference's native batch (pacifai/pots-2.0,
 * verification/commitment/native.c) entry point by entry point, so the reference's ctypes
 * binding (verification/commitment/native.py:241-261) can load this library instead: the
 * names, argument order and meaning are the reference's, the hashing runs on the GPU, and
 * payloads and outputs may live in HBM. `n_threads` is accepted and ignored.
 */
#ifndef POTS_MI355X_H
#define POTS_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define POTS_E_OK 0
#define POTS_E_NOMEM (-1)   /* the reference's "out of memory, nothing written" */
#define POTS_E_HIP (-3)     /* a HIP call failed; see pots_last_error() */
#define POTS_E_ARG (-4)     /* an argument is out of range or inconsistent */

/* Finiteness kinds (native.c:146-150): which payload values are tested for NaN/Inf. */
#define POTS_KIND_NONE 0
#define POTS_KIND_F32 1
#define POTS_KIND_BF16 2
#define POTS_KIND_F16 3

/* "pots-mi355x <version> gfx950". */
const char *pots_mi355x_version(void);

/* The last HIP error message of the calling thread, or "" if none. */
const char *pots_last_error(void);

/* Replaces native.c:341 pots_simd_degree: chunks compressed per instruction (64, one BLAKE3
 * chunk per lane of a wavefront). */
size_t pots_simd_degree(void);

/* Replaces native.c:343 pots_blake3_version: which BLAKE3 implementation hashes ("spec
 * (gfx950 kernels)": this library's own, written from the BLAKE3 specification). */
const char *pots_blake3_version(void);

/* ---- the reference's entry points --------------------------------------------------- */

/* Replaces native.c:243 pots_hash_leaves. Leaf i's digest BLAKE3(0x00 || header || payload)
 * goes to out + 32 i, the header being hdr_buf[hdr_off[u] : + hdr_len[u]] for u = hdr_idx[i]
 * and the payload payload_len[i] bytes at the address payload_ptr[i] (host or device memory).
 * kind[i] selects the NaN/Inf test (POTS_KIND_*). Metadata arrays and `out` are host memory.
 *
 * Returns the smallest i whose payload holds a non-finite value, or n when none does; the
 * digests before it are valid, those at or after it unspecified. Returns SIZE_MAX when a HIP
 * call fails (nothing valid written). Synchronous. */
size_t pots_hash_leaves(size_t n, const uint8_t *hdr_buf, const uint64_t *hdr_off,
                        const uint32_t *hdr_len, const uint32_t *hdr_idx,
                        const uint64_t *payload_ptr, const uint64_t *payload_len,
                        const uint8_t *kind, uint8_t *out, uint32_t n_threads);

/* No counterpart in the reference: pots_hash_leaves for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, results and return values, bit for bit; it calls no hipMalloc,
 * hipFree or other allocating routine. Its workspace (the plan's descriptors and chaining
 * values, staged host payloads, the digests before their copy out) lives in a static 64 MiB
 * device array, one per GPU, held until the process ends: about 2 M chunks of 1 KiB, i.e.
 * some 2 GiB of leaf bytes in device memory (host payloads also take their size in it). A
 * larger request returns SIZE_MAX with the reason in pots_last_error(), before any GPU work.
 * The array belongs to the library's code object: loading the library reserves its 64 MiB
 * of device memory on each GPU where the code is loaded, even if this entry point is never
 * called.
 * Calls in one process are serialised, since they share the array; calls from two processes
 * on one GPU use separate arrays. Synchronous, on the null stream. */
size_t pots_hash_leaves_noalloc(size_t n, const uint8_t *hdr_buf, const uint64_t *hdr_off,
                                const uint32_t *hdr_len, const uint32_t *hdr_idx,
                                const uint64_t *payload_ptr, const uint64_t *payload_len,
                                const uint8_t *kind, uint8_t *out, uint32_t n_threads);

/* Replaces native.c:299 pots_all_finite: 1 when every value of the nbytes bytes at p (host
 * or device) is finite under `kind` (kind 0: always 1), 0 when one is NaN or Inf, a negative
 * POTS_E_* on failure. Synchronous. */
int pots_all_finite(const uint8_t *p, uint64_t nbytes, uint8_t kind, uint32_t n_threads);

/* Replaces native.c:335 pots_merkle_tree (which returns void): the 2n - 1 node hashes of the
 * RFC 6962 tree over n >= 1 leaf digests, pre-order (root first; for a range at p with left
 * half of k leaves, the left child at p + 1 and the right child at p + 2k), H_node(l, r) =
 * BLAKE3(0x01 || l || r). `leaves` (32 n bytes) and `nodes` (32 (2n - 1) bytes) are host or
 * device memory. Returns POTS_E_*. Synchronous. */
int pots_merkle_tree(size_t n, const uint8_t *leaves, uint8_t *nodes);

/* ---- stream-ordered entry points for a transcript resident in HBM ------------------- */

/* A leaf-hashing plan: the leaves' metadata uploaded once, the chunk decomposition and the
 * per-level reduction schedule computed, and the workspace allocated. Arguments as for
 * pots_hash_leaves, with every payload already in device memory (payload_ptr holds device
 * addresses; the arrays themselves are host memory). The caller keeps the payloads alive and
 * unmodified while runs of the plan are in flight. Returns POTS_E_*; *plan is set on success.
 * Replaces the batching of verification/commitment/leaves.py:312-437. */
int pots_leaf_plan_create(size_t n, const uint8_t *hdr_buf, const uint64_t *hdr_off,
                          const uint32_t *hdr_len, const uint32_t *hdr_idx,
                          const uint64_t *payload_ptr, const uint64_t *payload_len,
                          const uint8_t *kind, void **plan);

/* Enqueue the plan on `stream`: digests to d_out (device, 32 n bytes) and the smallest
 * non-finite leaf index (or n) to *d_first_bad (device uint32). No allocation, no sync. */
int pots_leaf_plan_run(void *plan, uint8_t *d_out, uint32_t *d_first_bad, void *stream);

/* pots_leaf_plan_run is these stages in order: 0 the staging copies and the first-bad reset,
 * 1 the chunk kernel (every 1 KiB chunk's chaining value, the NaN/Inf test fused), 2 the
 * per-leaf BLAKE3 trees above the chunks. Enqueued on `stream` one at a time, so a caller can
 * time each stage; the caller keeps the order. No counterpart in the reference. */
#define POTS_LEAF_STAGES 3
/* Stage 1 is two kernels, which a caller may also enqueue apart (each once, both before
 * stage 2): the chunks of the leaves fused with a Freivalds plan's products
 * (pots_leaf_plan_create_fused; it reads the challenges), and the chunks of the others. */
#define POTS_LEAF_STAGE_FUSED_CHUNKS 3
#define POTS_LEAF_STAGE_PLAIN_CHUNKS 4
int pots_leaf_plan_run_stage(void *plan, int stage, uint8_t *d_out, uint32_t *d_first_bad,
                             void *stream);

/* Limit the chunk kernels' grid to max_blocks blocks of 256 lanes (0: no limit, one block per
 * 256 slots; a slot is one lane's run of up to four consecutive chunks). Each block then
 * hashes several blocks' worth of slots in turn, and the kernel
 * holds at most that many blocks' worth of the GPU, leaving the rest to work on other
 * streams (the Freivalds passes, which are bound by HBM, not by the VALUs hashing needs).
 * Results do not depend on it. No counterpart in the reference. */
int pots_leaf_plan_set_grid(void *plan, uint32_t max_blocks);

/* As pots_leaf_plan_create, and the leaves that are the P operand of a product of fv_plan (a
 * Freivalds plan, below) also have that product's P-pass sums taken by the chunk kernel while
 * it hashes them, so P is read from HBM once for both checks. A product qualifies when the
 * plan's k is 1, 2 or 4, its P is the leaf's whole payload (contiguous, same dtype: bf16 or fp32, at a
 * 16-byte aligned address after a 12-byte 0x00 || header, i.e. a 2-D tensor leaf), its rows
 * hold at least 1 KiB, and no other product shares that P. The Freivalds plan's stage 4 then
 * reads what the chunk stage (stage 1 of this plan) wrote for the same claimed root: run
 * fv stage 0, then this plan's stage 1, before fv stage 4 (pots_step_run keeps that order on
 * one stream; pots_fv_plan_run refuses a fused plan). A Freivalds plan is fused with at most
 * one leaf plan; destroy the leaf plan first. Digests are those of pots_leaf_plan_create; the
 * rows agree with the unfused plan's to fp32 rounding of the sums' order. No counterpart in
 * the reference: it reads P once in check 2 and again in check 5. */
int pots_leaf_plan_create_fused(size_t n, const uint8_t *hdr_buf, const uint64_t *hdr_off,
                                const uint32_t *hdr_len, const uint32_t *hdr_idx,
                                const uint64_t *payload_ptr, const uint64_t *payload_len,
                                const uint8_t *kind, void *fv_plan, void **plan);

/* Leaves of the plan whose product's P-pass sums its chunk stage takes (0 for an unfused
 * plan). */
uint32_t pots_leaf_plan_fused(const void *plan);

/* What one run of the fused chunk kernel moves: the fused leaves' message bytes (read), their
 * 1 KiB chunks (a 32-byte chaining value written each) and the run records it writes (32 bytes
 * each). Returns POTS_E_*. */
int pots_leaf_plan_fused_stats(const void *plan, uint64_t *msg_bytes, uint64_t *chunks,
                               uint64_t *records);

/* One step on one stream: fv stage 0, the leaf plan's stages, fv stages 1-5 (digests and
 * first-bad as pots_leaf_plan_run, rows as pots_fv_plan_run). For a fused pair of plans and
 * for two independent ones alike. No counterpart in the reference. */
int pots_step_run(void *leaf_plan, void *fv_plan, const uint8_t *d_key, uint8_t *d_digests,
                  uint32_t *d_first_bad, double *d_rows, void *stream);

/* Chunks (1 KiB BLAKE3 chunks) and message bytes the plan hashes. */
uint64_t pots_leaf_plan_chunks(const void *plan);
uint64_t pots_leaf_plan_bytes(const void *plan);

void pots_leaf_plan_destroy(void *plan);

/* The RFC 6962 tree over n leaf digests already in device memory, as pots_merkle_tree,
 * enqueued on `stream`; d_nodes (32 (2n - 1) bytes) is written in pre-order. */
int pots_merkle_tree_async(size_t n, const uint8_t *d_leaves, uint8_t *d_nodes, void *stream);

/* ---- Freivalds measurement and verdicts ---------------------------------------------- */

#define POTS_DT_F32 0
#define POTS_DT_BF16 1

/* One checked product P = A·B (+ 1·biasᵀ). All pointers are device memory; B and P are
 * row-major with the given row strides (elements). `bias` is fp32 [w] already rounded to the
 * operand format as the reference serves it (checks.py:439), or NULL. `m` is the product's
 * 1-based index, the challenge label.
 *
 * A is row-major with row stride lda when a_trans is 0. When a_trans is 1, A is the transpose
 * of a row-major X [q, n] at `a` with row stride lda, and another product of the same plan
 * must have that X as its row-major A (its twin: same pointer and lda, shape [q, n]); the
 * plan then reads X once for both (the twin pass). A transposed A is taken only in bf16, with
 * k <= 4, q a multiple of 16, n a multiple of 128, `a` and lda·2 multiples of 16 bytes;
 * anything else is POTS_E_ARG. No counterpart in the reference, which multiplies whatever
 * layout torch hands it. */
typedef struct {
  const void *a, *b, *p;
  const float *bias;
  uint64_t lda, ldb, ldp;
  uint32_t n, q, w, m;
  uint32_t a_dtype, b_dtype, p_dtype, a_trans;
} pots_fv_product;

/* A Freivalds plan over n products with k challenge vectors each: operand layout, column
 * chunking and workspace fixed once. Replaces the per-product torch op sequence of
 * verification/verifier/matmul_check/freivalds.py:290-321 and :384-410. guard = 0 leaves the
 * first two columns NaN (freivalds.py:309-312). */
int pots_fv_plan_create(size_t n, const pots_fv_product *products, uint32_t k, uint32_t guard,
                        void **plan);

/* Enqueue on `stream`: the challenge matrices keyed on the 32-byte d_key (device memory,
 * the claimed root), the three streaming passes and the reduction, writing one fp64 row per
 * product to d_rows [n][5 + k] in freivalds.ROW order (freivalds.py:255): nu, ‖|P|1‖, ‖P‖_F,
 * Σ_i (A²(B²1))_i, ‖b‖², residual_1..k. No allocation, no sync. */
int pots_fv_plan_run(void *plan, const uint8_t *d_key, double *d_rows, void *stream);

/* pots_fv_plan_run is these stages in order: 0 the challenge matrices, 1 the B pass
 * (b1 = B·R, b2 = (B²)·1), 2 the reduction of B's split-K partials, 3 the A pass (A·b1 and
 * (A²)·b2), 4 the P pass (P·R, Σ|P|, ΣP²), 5 the rows. Enqueued on `stream` one at a time,
 * so a caller can time each stage; the caller keeps the order. No counterpart in the
 * reference. */
#define POTS_FV_STAGES 6
/* Stage 4 is two parts, which a caller may also enqueue apart (each once, both after stage 2
 * and before stage 5): the P pass over the products not fused with a leaf plan, and the fused
 * products' sums from the records the leaf plan's chunk stage wrote (nothing when unfused). */
#define POTS_FV_STAGE_P_PASS 6
#define POTS_FV_STAGE_P_FUSED 7
/* Stage 3 is two parts as well, which a caller may enqueue apart (each once, both after
 * stage 2 and before stage 5): the row pass over the A operands of products that have no
 * twin, and the twin pass over the twins' shared operands (nothing when the plan has none). */
#define POTS_FV_STAGE_A_ROWS 8
#define POTS_FV_STAGE_TWINS 9
int pots_fv_plan_run_stage(void *plan, int stage, const uint8_t *d_key, double *d_rows,
                           void *stream);

/* Limit the row-pass grid of stage 1 (B pass), 3 (A pass) or 4 (P pass) to max_blocks blocks
 * of 256 lanes (0: no limit, one block per tile). Each block then takes several tiles in turn,
 * from a queue per XCD (a contiguous range of the tiles each, then the other XCDs' ranges),
 * and the pass holds at most that many blocks' worth of the GPU, so that a kernel on another
 * stream (the leaf hasher, which needs every SIMD's VALUs) can share the CUs. Results do not
 * depend on it. No counterpart in the reference. */
int pots_fv_plan_set_grid(void *plan, int stage, uint32_t max_blocks);

/* Copy the last run's row-major challenge matrices (fp32; product i's [w_i, k] block follows
 * product i-1's) to d_out (device, Σ w_i·k floats), enqueued on `stream`. */
int pots_fv_plan_copy_challenges(const void *plan, float *d_out, void *stream);

/* Bytes of A, B and P the plan reads (each once). */
uint64_t pots_fv_plan_bytes(const void *plan);

/* The pairs of twin products the plan reads through the twin pass (a_trans products and their
 * row-major twins): each pair's shared operand is read once. No counterpart in the
 * reference. */
uint32_t pots_fv_plan_twins(const void *plan);

void pots_fv_plan_destroy(void *plan);

/* Replaces native.c:119 pots_challenges: item i's [widths[i], k] fp32 matrix at out +
 * offsets[i] (out host or device memory), vector j of product ms[i] the keyed XOF of
 * 0x10 || ms[i] (BE) || j under key, entries (2(w >> 8) + 1 - 2^24) / 2^24. Synchronous. */
int pots_challenges(const uint8_t key[32], uint32_t k, size_t n, const uint32_t *ms,
                    const uint32_t *widths, const uint64_t *offsets, float *out,
                    uint32_t n_threads);

/* Per-product verdicts from fp64 rows d_rows [n][5 + k] (device), on `stream`. d_specs is
 * device memory of n records { double kappa_max; uint32_t q, n, biased, pad; } (q the
 * checked contraction length, +1 with a bias). Writes (code, j) int32 pairs to d_codes
 * (0 accept, 1 non-finite, 2 cancellation guard, 3 residual of challenge j above tau·unit),
 * optionally (kappa, unit, U) to d_finished [n][3], and the smallest rejecting index (or n)
 * to *d_first_fail. sigma_r and sqrt2 are 1/√3 and √2 as the caller's doubles. Replaces
 * freivalds.py:324-335,450-468 and checks.py:926-956. */
int pots_verdicts_async(size_t n, const double *d_rows, uint32_t k, const void *d_specs,
                        double eps_in, double eps_acc, double tau, double sigma_r, double sqrt2,
                        uint32_t guard, uint32_t judge, int32_t *d_codes, double *d_finished,
                        uint32_t *d_first_fail, void *stream);

/* ---- check 6a: the SGD update identity of the linear weights ----------------------- */

/* One linear weight: W_t and W_{t+1} (fp32, n entries each) and the parts of its gradient G
 * (its committed weight-gradient products, fp32 or bf16, n entries each, summed in order in
 * fp32: chain_gradient, verification/computation/interface.py:169-180). All device memory,
 * contiguous. tau_w is the weight's band (bands.py tau_w_for). */
#define POTS_UPDATE_MAX_PARTS 8
typedef struct pots_update_weight {
  const void *w_t;
  const void *w_next;
  const void *parts[POTS_UPDATE_MAX_PARTS];
  uint32_t part_dtype[POTS_UPDATE_MAX_PARTS]; /* 0 fp32, 1 bf16 */
  uint32_t n_parts;
  uint32_t pad;
  uint64_t n;
  double tau_w;
} pots_update_weight;

/* Per weight, in device memory: rho_bits is ρ_max = max_i ρ_i as the bits of a double (NaN
 * if any ρ_i is NaN, 0 for an empty weight); first_nonfinite and first_over are the smallest
 * index whose R_i or scale_i is not finite, and whose ρ_i is not ≤ tau_w, or UINT64_MAX. */
typedef struct pots_update_result {
  uint64_t rho_bits;
  uint64_t first_nonfinite;
  uint64_t first_over;
} pots_update_result;

/* A plan over n weights, with the step size eta and ε_W (eps_w) already rounded to fp32 (the
 * reference multiplies fp32 tensors by them as fp32 scalars). Replaces the per-weight work of
 * checks.py:380-451 (_update_identity, _update_identity_reference; ρ_max bit for bit as
 * _fast_rho_max, checks.py:301-377, obtains it): R = |W_{t+1} − (W_t − η·G)|,
 * scale = ε_W·(|W_t| + |η·G|) in fp32, ρ_i = 0 if R_i = 0 else fl64(R_i)/fl64(scale_i). */
int pots_update_plan_create(size_t n, const pots_update_weight *weights, float eta, float eps_w,
                            void **plan);
/* Enqueue the pass; d_out holds n results (device). Stream-ordered, no allocation, no sync. */
int pots_update_plan_run(void *plan, pots_update_result *d_out, void *stream);
/* Bytes one run reads: W_t, W_{t+1} and every gradient part once. */
uint64_t pots_update_plan_bytes(void *plan);
void pots_update_plan_destroy(void *plan);

/* ---- Stored steps: leaf files to device memory ------------------------------------------
 *
 * The on-disk transcript store (verification/transcript/store.py:285-380, DiskStore) writes
 * one torch.save file per leaf. Its reader (store.py:347-357, DiskStore.leaf) unpickles each
 * file into pageable host memory with torch.load; the checks then copy the tensors to the GPU
 * one by one. These two entry points replace that read for a whole step: a parallel scan of
 * the files' ZIP directories and pickles (no Python, nothing executed), then parallel reads
 * of the storage bytes into pinned staging and DMA into one device buffer. */

#define POTS_E_IO (-5) /* a file could not be opened or read; see pots_last_error() */

/* Element types of a stored tensor, from its pickled storage class (torch.FloatStorage ...). */
#define POTS_STORE_F32 1
#define POTS_STORE_F64 2
#define POTS_STORE_F16 3
#define POTS_STORE_BF16 4
#define POTS_STORE_I64 5
#define POTS_STORE_I32 6
#define POTS_STORE_I16 7
#define POTS_STORE_I8 8
#define POTS_STORE_U8 9
#define POTS_STORE_BOOL 10

/* Scan status of one file. */
#define POTS_STORE_OK 0     /* one plain tensor, described below */
#define POTS_STORE_OTHER 1  /* anything else (a record's dict, a tensor that needs grad, a
                               big-endian or compressed archive, ...): read it with torch.load */
#define POTS_STORE_UNREADABLE 2 /* not a ZIP archive that can be read; torch.load fails too */

#define POTS_STORE_MAX_DIM 8

/* What pots_store_scan found in one file: a tensor of `ndim` dims with these sizes and
 * strides (elements) at `storage_offset` elements into a storage of `storage_bytes` bytes,
 * stored uncompressed at `data_offset` in the file. Fields other than status are meaningful
 * only for POTS_STORE_OK. */
typedef struct pots_stored_tensor {
  uint64_t data_offset;
  uint64_t storage_bytes;
  uint64_t storage_offset;
  int64_t size[POTS_STORE_MAX_DIM];
  int64_t stride[POTS_STORE_MAX_DIM];
  uint32_t ndim;
  uint32_t dtype; /* POTS_STORE_F32 ... */
  int32_t status; /* POTS_STORE_OK ... */
  uint32_t pad;
} pots_stored_tensor;

/* Scan n_files files on n_threads host threads (0: 8). Accepts exactly the pickle torch.save
 * writes for one tensor that does not require grad, torch._utils._rebuild_tensor_v2(storage,
 * offset, size, stride, False, OrderedDict()), with a little-endian byte order record and the
 * storage's record stored; its opcodes are walked, never executed. Returns POTS_E_OK (each
 * file's own outcome is in its status) or POTS_E_ARG. Host only: needs no GPU. */
int pots_store_scan(uint32_t n_files, const char *const *paths, pots_stored_tensor *out,
                    uint32_t n_threads);

/* One piece of a file for pots_store_load: `bytes` bytes at `file_offset` of file `file` go
 * to `dst_offset` bytes into the destination. */
typedef struct pots_store_segment {
  uint32_t file;
  uint32_t pad;
  uint64_t file_offset;
  uint64_t bytes;
  uint64_t dst_offset;
} pots_store_segment;

/* Copy the segments (sorted by dst_offset, not overlapping) into `dst`. With dst_device >= 0,
 * dst is memory of that device: n_threads host threads (0: 8) each read their share of the
 * spans into two slots of the pinned host `staging` (staging_bytes, at least 2·n_threads·64
 * KiB, from hipHostMalloc) and send each slot with one hipMemcpyAsync on a stream of their
 * own. With dst_device < 0, dst is host memory read into directly (staging unused). Bytes
 * between segments that fall inside one span are written with unspecified values. Returns
 * after every copy has completed: POTS_E_OK, POTS_E_IO (a short or failed read), POTS_E_HIP
 * or POTS_E_ARG. */
int pots_store_load(uint32_t n_files, const char *const *paths, uint32_t n_segs,
                    const pots_store_segment *segs, void *dst, int dst_device, void *staging,
                    uint64_t staging_bytes, uint32_t n_threads);

#ifdef __cplusplus
}
#endif

#endif /* POTS_MI355X_H */
