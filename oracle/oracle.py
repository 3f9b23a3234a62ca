"""TEST INFRASTRUCTURE — the CPU oracle for the MI355X hot path. Not the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this module, and only as the checker (or, in the bench, as the timed CPU baseline). The
product in ``pots-2.0_amd/`` never imports it.

Each function restates the reference (pacifai/pots-2.0) on the CPU; the citation after each
name is the reference code it follows:

- ``blake3`` / ``hash_leaf`` / ``hash_node`` — BLAKE3 from the spec (``blake3_spec.c``),
  ``verification/commitment/merkle.py:37-44,153-155``.
- ``hash_leaves`` — ``verification/commitment/native.c:243`` (``native_twin.c``; with
  ``simd=True`` ``blake3_simd.c``, the same leaves 16 chunks per AVX-512 instruction, as the
  reference's BLAKE3 library hashes them on the CPU).
- ``merkle_tree`` / ``merkle_root`` / ``verify_path`` — ``native.c:315-337``,
  ``merkle.py:181-224,309-328``.
- ``tensor_leaf_header`` / ``encode_record`` — ``verification/commitment/encoding.py:45-56``,
  ``setup/records.py:83-86``.
- ``challenge_matrices`` / ``entries`` — ``native.c:71-139``,
  ``verification/verifier/matmul_check/challenges.py:46-106``.
- ``safe_norm`` / ``measure_product_row`` / ``measure_products_rows`` — the plain formulas of
  ``verification/verifier/matmul_check/freivalds.py:101-119,413-447`` in torch-CPU fp32.
- ``measure_row_f64`` — the same numbers in float64 throughout, the "true" values honest
  residuals are compared with in band units.
- ``finish_row`` / ``band_unit`` / ``judge`` — ``freivalds.py:324-335,450-468``,
  ``sizing.py:16-43``, ``verification/verifier/checks.py:926-956``.
- ``chain_gradient`` / ``update_identity`` — check 6a's update identity,
  ``verification/computation/interface.py:169-180`` and
  ``verification/verifier/checks.py:380-451`` (``_update_identity_reference``), in torch-CPU
  fp32 with the ratio in float64.

Pinning (what checks this oracle, so a wrong restatement fails a test): the reference's
known-answer tests (``tests/verification/verifier/matmul_check/test_challenges.py:86-137``,
``tests/verification/commitment/test_merkle.py:27-34``, ``test_encoding.py:22-30``,
``test_sizing.py:20-25``), BLAKE3's published test vectors for the unkeyed empty and
short inputs, agreement with the independent recursive BLAKE3 of ``blake3_tree.py`` on
multi-chunk inputs, brute-force tree shapes, the closed forms of every Freivalds column
(all-ones operands: nu = ||(|P|1)|| = sqrt(n) q w, ||P||_F = q sqrt(n w), U^2 = n q w;
non-negative operands: kappa = 1; integer operands with one planted entry: residual j equals
|delta r[col, j]| exactly in fp64), their invariants (a forged entry stands out, bias as a
ones column, U <= nu, scale invariance), and the
update identity's exact small cases (R = 0 for an exactly rounded step, closed-form ρ for
power-of-two entries, 0/0 and r/0, an fp32 quotient that underflows) together with the
outcomes the reference's own update-identity tests state; see ``tests/test_oracle.py``.
"""

from __future__ import annotations

import ctypes
import math
import os
import struct
import subprocess
from collections.abc import Sequence
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

TAG_WEIGHT, TAG_PRODUCT, TAG_MLP_RECORD = 0x02, 0x03, 0x04
TAG_RECORD, INT32_CODE = 0x01, 0x10
DTYPE_CODES = {torch.float32: 0x01, torch.bfloat16: 0x02, torch.float16: 0x03,
               torch.int32: 0x10}
FINITE_KIND = {torch.float32: 1, torch.bfloat16: 2, torch.float16: 3, torch.int32: 0}
SIGMA_R = 1.0 / math.sqrt(3.0)
UNIT_ROUNDOFF = {torch.float32: 2.0**-24, torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11}


def build() -> Path:
    """Compile ``liboracle.so`` with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, sz, u32, u64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint64
        L.oracle_blake3.argtypes = [vp, sz, vp, u64, vp, sz]
        L.oracle_blake3.restype = None
        L.oracle_hash_leaves.argtypes = [sz, vp, vp, vp, vp, vp, vp, vp, vp, u32]
        L.oracle_hash_leaves.restype = sz
        L.oracle_hash_leaves_simd.argtypes = [sz, vp, vp, vp, vp, vp, vp, vp, vp, u32]
        L.oracle_hash_leaves_simd.restype = sz
        L.oracle_simd_degree.argtypes = []
        L.oracle_simd_degree.restype = ctypes.c_int
        L.oracle_all_finite.argtypes = [vp, u64, ctypes.c_uint8]
        L.oracle_all_finite.restype = ctypes.c_int
        L.oracle_merkle_tree.argtypes = [sz, vp, vp]
        L.oracle_merkle_tree.restype = None
        L.oracle_challenges.argtypes = [vp, u32, sz, vp, vp, vp, vp, u32]
        L.oracle_challenges.restype = ctypes.c_int
        L.oracle_compress.argtypes = [vp, vp, u64, u32, u32, vp]
        L.oracle_compress.restype = None
        _lib = L
    return _lib


def _threads() -> int:
    return max(1, len(os.sched_getaffinity(0)))


# ---- BLAKE3 and the Merkle tree ----------------------------------------------------------

def blake3(data: bytes, *, key: bytes | None = None, length: int = 32, seek: int = 0) -> bytes:
    data = bytes(data)
    out = ctypes.create_string_buffer(length)
    kb = None if key is None else ctypes.create_string_buffer(bytes(key), 32)
    lib().oracle_blake3(data, len(data), kb, seek, out, length)
    return out.raw


def compress(cv: Sequence[int], block: bytes, counter: int, block_len: int,
             flags: int) -> list[int]:
    cvb = np.asarray(cv, dtype=np.uint32)
    out = np.zeros(16, dtype=np.uint32)
    blk = bytes(block).ljust(64, b"\0")
    lib().oracle_compress(cvb.ctypes.data, blk, counter, block_len, flags, out.ctypes.data)
    return out.tolist()


def hash_leaf(*parts: bytes) -> bytes:
    return blake3(b"\x00" + b"".join(bytes(p) for p in parts))


def hash_node(left: bytes, right: bytes) -> bytes:
    return blake3(b"\x01" + left + right)


def merkle_tree(leaf_hashes: Sequence[bytes]) -> bytes:
    n = len(leaf_hashes)
    out = ctypes.create_string_buffer(32 * (2 * n - 1))
    lib().oracle_merkle_tree(n, b"".join(leaf_hashes), out)
    return out.raw


def merkle_root(leaf_hashes: Sequence[bytes]) -> bytes:
    return merkle_tree(leaf_hashes)[:32]


def merkle_root_recursive(leaf_hashes: Sequence[bytes]) -> bytes:
    """RFC 6962 MTH by its recursive definition (merkle.py:181-193), no pre-order buffer."""
    def mth(lo: int, hi: int) -> bytes:
        if hi - lo == 1:
            return leaf_hashes[lo]
        k = 1 << ((hi - lo - 1).bit_length() - 1)
        return hash_node(mth(lo, lo + k), mth(lo + k, hi))
    return mth(0, len(leaf_hashes))


def verify_path(leaf_hash: bytes, index: int, n_leaves: int, path: Sequence[bytes],
                root: bytes) -> bool:
    """RFC 9162 §2.1.3.2 inclusion proof (merkle.py:309-328)."""
    if not 0 <= index < n_leaves:
        return False
    fn, sn, r = index, n_leaves - 1, leaf_hash
    for p in path:
        if sn == 0:
            return False
        if fn & 1 or fn == sn:
            r = hash_node(p, r)
            while not fn & 1 and fn != 0:
                fn >>= 1
                sn >>= 1
        else:
            r = hash_node(r, p)
        fn >>= 1
        sn >>= 1
    return sn == 0 and r == root


# ---- leaf encoding --------------------------------------------------------------------------

def tensor_leaf_header(tag: int, t: torch.Tensor) -> bytes:
    shape = tuple(t.shape)
    return struct.pack(f">BBB{len(shape)}I", tag, DTYPE_CODES[t.dtype], len(shape), *shape)


def payload_bytes(t: torch.Tensor) -> bytes:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.reshape(-1).numpy().tobytes()


def encode_record(ids: torch.Tensor, targets: torch.Tensor, mask: torch.Tensor) -> bytes:
    head = struct.pack(">BBI", TAG_RECORD, INT32_CODE, ids.numel())
    return head + payload_bytes(ids) + payload_bytes(targets) + payload_bytes(mask)


def tensor_leaf_hash(tag: int, t: torch.Tensor) -> bytes:
    return hash_leaf(tensor_leaf_header(tag, t), payload_bytes(t))


def simd_degree() -> int:
    """Chunks ``hash_leaves(..., simd=True)`` compresses per instruction: 16 with AVX-512, 1
    (the spec hasher) without."""
    return int(lib().oracle_simd_degree())


def hash_leaves(items: Sequence[tuple[bytes, torch.Tensor | bytes, int]],
                threads: int | None = None, simd: bool = False) -> tuple[list[bytes], int]:
    """``oracle_hash_leaves`` over ``(header, payload, kind)`` items (CPU payloads): the
    digests (those from the first bad leaf on are not meaningful) and the first bad index.
    ``simd`` takes the 16-lane chunk compressor of ``blake3_simd.c`` (the bench's CPU
    baseline, at the reference's CPU speed), checked against the spec hasher by the tests."""
    n = len(items)
    if n == 0:
        return [], 0
    headers = [bytes(h) for h, _, _ in items]
    hdr_buf = b"".join(headers) or b"\0"
    hdr_len = np.array([len(h) for h in headers], dtype=np.uint32)
    hdr_off = np.concatenate([[0], np.cumsum(hdr_len[:-1], dtype=np.uint64)]).astype(np.uint64)
    hdr_idx = np.arange(n, dtype=np.uint32)
    keep = []
    ptrs = np.zeros(n, dtype=np.uint64)
    lens = np.zeros(n, dtype=np.uint64)
    for i, (_, p, _) in enumerate(items):
        if isinstance(p, torch.Tensor):
            p = p.detach().cpu().contiguous()
            keep.append(p)
            ptrs[i], lens[i] = p.data_ptr(), p.nbytes
        else:
            b = np.frombuffer(bytes(p), dtype=np.uint8).copy()
            keep.append(b)
            ptrs[i], lens[i] = b.ctypes.data, b.nbytes
    kind = np.array([k for _, _, k in items], dtype=np.uint8)
    out = np.zeros((n, 32), dtype=np.uint8)
    fn = lib().oracle_hash_leaves_simd if simd else lib().oracle_hash_leaves
    bad = fn(n, hdr_buf, hdr_off.ctypes.data, hdr_len.ctypes.data, hdr_idx.ctypes.data,
             ptrs.ctypes.data, lens.ctypes.data, kind.ctypes.data, out.ctypes.data,
             threads or _threads())
    del keep
    if bad == (1 << 64) - 1:
        raise MemoryError("oracle_hash_leaves_simd: out of memory or a header over 1 KiB")
    return [bytes(r) for r in out], int(bad)


def all_finite(t: torch.Tensor) -> bool:
    t = t.detach().cpu().contiguous()
    return bool(lib().oracle_all_finite(t.data_ptr(), t.nbytes, FINITE_KIND[t.dtype]))


# ---- challenges -------------------------------------------------------------------------

def encode_label(m: int, j: int) -> bytes:
    return struct.pack(">BIB", 0x10, m, j)


def entries(words: np.ndarray) -> np.ndarray:
    """``(2(w >> 8) + 1 − 2^24) / 2^24`` in float32 (challenges.py:59-72), via int64."""
    a = (np.asarray(words, dtype=np.uint32) >> np.uint32(8)).astype(np.int64)
    return ((2 * a + 1 - (1 << 24)).astype(np.float32) / np.float32(1 << 24))


def challenge_matrices(h: bytes, ms: Sequence[int], k: int, width: int,
                       threads: int | None = None) -> torch.Tensor:
    n = len(ms)
    out = np.zeros(n * width * k, dtype=np.float32)
    msa = np.asarray(ms, dtype=np.uint32)
    widths = np.full(n, width, dtype=np.uint32)
    offs = (np.arange(n, dtype=np.uint64) * np.uint64(width * k)).astype(np.uint64)
    rc = lib().oracle_challenges(bytes(h), k, n, msa.ctypes.data, widths.ctypes.data,
                                 offs.ctypes.data, out.ctypes.data, threads or _threads())
    if rc != 0:
        raise RuntimeError(f"oracle_challenges returned {rc}")
    return torch.from_numpy(out).view(n, width, k)


def challenge_matrix_xof(h: bytes, m: int, k: int, width: int) -> torch.Tensor:
    """One XOF call per vector, then the entry map (challenges.py:46-56,75-85)."""
    cols = [entries(np.frombuffer(blake3(encode_label(m, j), key=h, length=4 * width),
                                  dtype="<u4")) for j in range(1, k + 1)]
    return torch.from_numpy(np.stack(cols, axis=1))


# ---- Freivalds rows ------------------------------------------------------------------------

def safe_norm(x: torch.Tensor, dim: int | None = None) -> torch.Tensor:
    """``freivalds._safe_norm`` (freivalds.py:101-119): ``s·‖x/s‖`` with
    ``s = 2^⌊log₂ max|x|⌋``; the unscaled norm where ``max|x|`` is 0 or not finite."""
    a = x.abs()
    amax = a.amax() if dim is None else a.amax(dim=dim)
    ok = torch.isfinite(amax) & (amax > 0)
    _, exp = torch.frexp(torch.where(ok, amax, torch.ones_like(amax)))
    s = torch.ldexp(torch.ones_like(amax), exp - 1)
    scaled = s * torch.linalg.vector_norm(x / (s if dim is None else s.unsqueeze(dim)), dim=dim)
    return torch.where(ok, scaled, torch.linalg.vector_norm(x, dim=dim))


def measure_product_row(a: torch.Tensor, b: torch.Tensor, p: torch.Tensor, r: torch.Tensor,
                        bias: torch.Tensor | None = None) -> list[float]:
    """The row ``[ν, ‖|P|·1‖, ‖P‖_F, ΣA²(B²1), ‖b‖², res_1..k]`` of one product by the plain
    formulas of ``_measure_product_reference`` (freivalds.py:413-430), fp32 on the CPU,
    given its challenge matrix ``r`` [w, k]."""
    a, b, p, r = (x.detach().cpu().float() for x in (a, b, p, r))
    width = b.shape[1]
    with torch.no_grad():
        ones = torch.ones(width, 1, dtype=torch.float32)
        nu_vec, ab_r = a.abs() @ (b.abs() @ ones), a @ (b @ r)
        u2 = float((a.square() @ (b.square() @ ones)).double().sum())
        bias_sq = 0.0
        if bias is not None:
            bias = bias.detach().cpu().float()
            nu_vec, ab_r = nu_vec + bias.abs() @ ones, ab_r + bias @ r
            bias_sq = float(bias.double().square().sum())
        nu = float(safe_norm(nu_vec))
        p_abs1 = float(safe_norm(p.abs() @ ones))
        res = safe_norm(ab_r - p @ r, dim=0).tolist()
        p_norm = float(safe_norm(p))
    return [nu, p_abs1, p_norm, u2, bias_sq, *res]


def measure_products_rows(a: torch.Tensor, b: torch.Tensor, p: torch.Tensor,
                          r: torch.Tensor) -> list[list[float]]:
    """``_measure_products_reference`` (freivalds.py:433-447) as rows: stacked members
    ``[B,n,q]·[B,q,w]`` against ``[B,n,w]``, each with its own ``r[i]`` [w, k]."""
    a, b, p, r = (x.detach().cpu().float() for x in (a, b, p, r))
    n_b, width = a.shape[0], b.shape[2]
    with torch.no_grad():
        ones = torch.ones(width, 1, dtype=torch.float32)
        nu = safe_norm((a.abs() @ (b.abs() @ ones)).reshape(n_b, -1), dim=1).tolist()
        u2 = (a.square() @ (b.square() @ ones)).double().reshape(n_b, -1).sum(1).tolist()
        p_abs1 = safe_norm((p.abs() @ ones).reshape(n_b, -1), dim=1).tolist()
        res = safe_norm(a @ (b @ r) - p @ r, dim=1).tolist()
        p_norm = safe_norm(p.reshape(n_b, -1), dim=1).tolist()
    return [[nu[i], p_abs1[i], p_norm[i], u2[i], 0.0, *res[i]] for i in range(n_b)]


def measure_row_f64(a: torch.Tensor, b: torch.Tensor, p: torch.Tensor, r: torch.Tensor,
                    bias: torch.Tensor | None = None) -> list[float]:
    """The row in float64 throughout: the operands' values widened exactly, every product and
    sum in float64. It is the yardstick for the rounding-level columns."""
    a, b, p, r = (x.detach().cpu().double() for x in (a, b, p, r))
    with torch.no_grad():
        nu_vec = a.abs() @ b.abs().sum(1)
        ab_r = a @ (b @ r)
        u2 = float((a.square() @ b.square().sum(1)).sum())
        bias_sq = 0.0
        if bias is not None:
            bias = bias.detach().cpu().double()
            nu_vec = nu_vec + bias.abs().sum()
            ab_r = ab_r + bias @ r
            bias_sq = float(bias.square().sum())
        res = torch.linalg.vector_norm(ab_r - p @ r, dim=0).tolist()
        return [float(torch.linalg.vector_norm(nu_vec)),
                float(torch.linalg.vector_norm(p.abs().sum(1))),
                float(torch.linalg.vector_norm(p)), u2, bias_sq, *res]


# ---- finishing and judging ----------------------------------------------------------------

def e_m(q: int, eps_in: float, eps_acc: float, u_ratio: float = 1.0) -> float:
    """sizing.py:16-27."""
    if math.isnan(u_ratio):
        return math.nan
    return math.sqrt(2.0) * eps_in + math.sqrt(q) * eps_acc * max(1.0, u_ratio)


def term_ratio(p_norm: float, u: float) -> float:
    """sizing.py:30-38."""
    if p_norm == 0 and u == 0:
        return 1.0
    if p_norm == 0:
        return math.inf if u > 0 else math.nan
    return u / p_norm


def band_unit(q: int, eps_in: float, eps_acc: float, p_norm: float, u: float) -> float:
    """freivalds.py:450-459."""
    if p_norm == 0:
        return SIGMA_R * math.sqrt(q) * eps_acc * u
    return SIGMA_R * e_m(q, eps_in, eps_acc, term_ratio(p_norm, u)) * p_norm


def finish_row(row: Sequence[float], *, q: int, n: int, eps_in: float, eps_acc: float,
               biased: bool = False) -> dict:
    """freivalds.py:324-335 and :462-468: κ, U, the band unit and the normalized residuals."""
    nu, p_abs1, p_norm, u2, bias_sq, *res = row
    if biased:
        u2 += n * bias_sq
    u = math.sqrt(u2)
    kappa = nu / p_abs1 if p_abs1 > 0 else (1.0 if nu == 0 else float("inf"))
    unit = band_unit(q, eps_in, eps_acc, p_norm, u)
    normalized = tuple(x / unit if unit > 0 else (0.0 if x == 0 else float("inf"))
                       for x in res)
    return {"nu": nu, "p_abs1": p_abs1, "kappa": kappa, "residuals": tuple(res),
            "p_norm": p_norm, "unit": unit, "normalized": normalized, "u": u}


# Verdict codes, the same numbering the product's verdict kernel writes.
ACCEPT, NONFINITE, KAPPA, RESIDUAL = 0, 1, 2, 3


def judge(mp: dict, *, tau: float, kappa_max: float, guard: bool = True) -> tuple[int, int]:
    """``checks._judge_product`` (checks.py:926-956) as ``(code, j)``: non-finite first, then
    the cancellation guard ``ν ≤ κ_max·‖|P|·1‖``, then ``res_j ≤ τ·unit`` for j = 1..k; every
    comparison written ``not (x <= bound)`` so NaN rejects. ``j`` is the failing challenge
    (1-based) for a residual rejection, else 0."""
    vals = ([mp["nu"], mp["p_abs1"]] if guard else []) + [mp["p_norm"], mp["u"], mp["unit"],
                                                           *mp["residuals"]]
    if any(not math.isfinite(v) for v in vals):
        return NONFINITE, 0
    if guard and not mp["nu"] <= kappa_max * mp["p_abs1"]:
        return KAPPA, 0
    for j, x in enumerate(mp["residuals"], start=1):
        if not x <= tau * mp["unit"]:
            return RESIDUAL, j
    return ACCEPT, 0


# ---- check 6a: the update identity --------------------------------------------------------

def chain_gradient(parts: Sequence[torch.Tensor], dtype: torch.dtype = torch.float32
                   ) -> torch.Tensor:
    """``interface.chain_gradient`` (interface.py:169-180): the parts widened to ``dtype``
    and added in order, out of place."""
    g = None
    for p in parts:
        p = p.detach().cpu()
        g = p.to(dtype) if g is None else g + p.to(dtype)
    if g is None:
        raise ValueError("a gradient needs at least one product")
    return g


def update_identity(w_t: torch.Tensor, w_next: torch.Tensor, parts: Sequence[torch.Tensor],
                    eta: float, eps_w: float, tau_w: float) -> dict:
    """``checks._update_identity_reference`` (checks.py:380-451) on whole CPU tensors:
    ``R = |W_{t+1} − (W_t − η·G)|`` and ``scale = ε_W·(|W_t| + |η·G|)`` in fp32 (``η`` and
    ``ε_W`` multiply as fp32 scalars, as torch does), ``ρ = 0`` where ``R = 0`` else
    ``fl64(R)/fl64(scale)``. Returns ``rho_max`` (torch's max, NaN-propagating; 0 when
    empty), ``first_nonfinite`` (first index whose R or scale is not finite) and
    ``first_over`` (first index with ``not ρ ≤ τ_W``), each ``None`` when there is none, and
    the flat ``r`` and ``scale``."""
    g = chain_gradient(parts, torch.float32)
    w_t, w_next = w_t.detach().cpu(), w_next.detach().cpu()
    with torch.no_grad():
        eta_g = eta * g
        r = (w_next - (w_t - eta_g)).abs()
        scale = eps_w * (w_t.abs() + eta_g.abs())
        finite = torch.isfinite(r) & torch.isfinite(scale)
        r64 = r.double()
        rho = torch.where(r64 == 0, torch.zeros_like(r64), r64 / scale.double())
    rho_max = float(rho.max()) if rho.numel() else 0.0
    nf = (~finite).reshape(-1).nonzero()
    ov = (~(rho <= tau_w)).reshape(-1).nonzero()
    return {"rho_max": rho_max, "first_nonfinite": int(nf[0]) if nf.numel() else None,
            "first_over": int(ov[0]) if ov.numel() else None,
            "r": r.reshape(-1), "scale": scale.reshape(-1)}
