"""The binding to ``libpots_mi355x.so``, the gfx950 kernels behind the hot path.

Reference: verification/commitment/native.py:229-368. The reference builds BLAKE3's C library
and its ``native.c`` for the host CPU and loads them with ctypes; this module loads the HIP
library instead, with the same class name, method names, argument meaning and errors, so its
callers (``merkle``, ``leaves``, ``challenges``) are unchanged. Payload addresses may be HBM
addresses; the kernels read the leaves where they lie.

There is no CPU path: if the library is missing or no GPU is visible, :func:`get` raises
``RuntimeError`` (as the reference's failed build does). :func:`enabled` and :func:`disabled`
keep their meaning as a switch the callers can read, but this build has one implementation,
so the hashing runs on the GPU either way.

torch is imported before the library is loaded on purpose: torch ships its own HIP runtime
with the same soname as ROCm's, and loading torch first makes this library bind to that one
runtime instead of a second copy.
"""

from __future__ import annotations

import atexit
import ctypes
import os
import threading
import weakref
from collections.abc import Callable, Iterator, Sequence
from typing import Any
from contextlib import contextmanager
from pathlib import Path

import numpy as np
import torch

PACKAGE_ROOT = Path(__file__).resolve().parents[2]
LIB_PATH = Path(os.environ.get("POTS_MI355X_LIB", PACKAGE_ROOT / "libpots_mi355x.so"))

# Every live plan, so that the process frees their device memory at exit while the HIP runtime
# is certainly up: an atexit handler runs before the interpreter tears its objects down, and
# the runtime's own destructors run after that. A plan closed earlier leaves the set by itself.
_LIVE_PLANS: weakref.WeakSet = weakref.WeakSet()


@atexit.register
def _close_live_plans() -> None:
    # leaf plans first: a fused leaf plan writes into its Freivalds plan's memory
    plans = sorted(list(_LIVE_PLANS), key=lambda p: not isinstance(p, LeafPlan))
    if plans and torch.cuda.is_available():
        torch.cuda.synchronize()
    for plan in plans:
        try:
            plan.close()
        except Exception:
            pass

KIND_NONE, KIND_F32, KIND_BF16, KIND_F16 = 0, 1, 2, 3
FINITE_KIND: dict[torch.dtype, int] = {
    torch.float32: KIND_F32, torch.bfloat16: KIND_BF16, torch.float16: KIND_F16,
    torch.int32: KIND_NONE,
}

E_OK, E_NOMEM, E_HIP, E_ARG, E_IO = 0, -1, -3, -4, -5


def _create(lib: Native, make: Callable[[], int], what: str) -> None:
    """A plan's create call. The plans take their device memory with hipMalloc, beside
    torch's caching allocator, which keeps the blocks a program has freed: when the device
    is out of memory, those go back to the driver (``torch.cuda.empty_cache``) and the call
    runs once more."""
    rc = make()
    if rc == E_NOMEM:
        torch.cuda.empty_cache()
        rc = make()
    lib._check(rc, what)
_SIZE_MAX = (1 << (8 * ctypes.sizeof(ctypes.c_size_t))) - 1


def build() -> Path:
    """Compile the library in place (``pots-2.0_amd/build.py``)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("_pots_build", PACKAGE_ROOT / "build.py")
    mod = importlib.util.module_from_spec(spec)
    assert spec.loader is not None
    spec.loader.exec_module(mod)
    return mod.build()


def _stream(stream: torch.cuda.Stream | None) -> ctypes.c_void_p:
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


class NativeError(RuntimeError):
    """A call into the library failed (a HIP error or a rejected argument)."""


_vp, _sz, _u8, _u32, _u64, _int = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint8,
                                   ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int)


def _addr(a: np.ndarray) -> int:
    return a.ctypes.data


class Native:
    """The loaded library."""

    def __init__(self, path: Path) -> None:
        self.path = path
        lib = ctypes.CDLL(str(path))
        sigs = {
            "pots_mi355x_version": ([], ctypes.c_char_p),
            "pots_last_error": ([], ctypes.c_char_p),
            "pots_simd_degree": ([], _sz),
            "pots_blake3_version": ([], ctypes.c_char_p),
            "pots_hash_leaves": ([_sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32], _sz),
            "pots_hash_leaves_noalloc": ([_sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32],
                                         _sz),
            "pots_all_finite": ([_vp, _u64, _u8, _u32], _int),
            "pots_merkle_tree": ([_sz, _vp, _vp], _int),
            "pots_leaf_plan_create": ([_sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                       ctypes.POINTER(_vp)], _int),
            "pots_leaf_plan_run": ([_vp, _vp, _vp, _vp], _int),
            "pots_leaf_plan_run_stage": ([_vp, _int, _vp, _vp, _vp], _int),
            "pots_leaf_plan_set_grid": ([_vp, _u32], _int),
            "pots_leaf_plan_chunks": ([_vp], _u64),
            "pots_leaf_plan_bytes": ([_vp], _u64),
            "pots_leaf_plan_destroy": ([_vp], None),
            "pots_leaf_plan_create_fused": ([_sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             ctypes.POINTER(_vp)], _int),
            "pots_leaf_plan_fused": ([_vp], _u32),
            "pots_leaf_plan_fused_stats": ([_vp, _vp, _vp, _vp], _int),
            "pots_step_run": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp], _int),
            "pots_merkle_tree_async": ([_sz, _vp, _vp, _vp], _int),
            "pots_challenges": ([_vp, _u32, _sz, _vp, _vp, _vp, _vp, _u32], _int),
            "pots_fv_plan_create": ([_sz, _vp, _u32, _u32, ctypes.POINTER(_vp)], _int),
            "pots_fv_plan_run": ([_vp, _vp, _vp, _vp], _int),
            "pots_fv_plan_run_stage": ([_vp, _int, _vp, _vp, _vp], _int),
            "pots_fv_plan_copy_challenges": ([_vp, _vp, _vp], _int),
            "pots_fv_plan_set_grid": ([_vp, _int, _u32], _int),
            "pots_fv_plan_bytes": ([_vp], _u64),
            "pots_fv_plan_twins": ([_vp], _u32),
            "pots_fv_plan_destroy": ([_vp], None),
            "pots_verdicts_async": ([_sz, _vp, _u32, _vp, ctypes.c_double, ctypes.c_double,
                                     ctypes.c_double, ctypes.c_double, ctypes.c_double, _u32,
                                     _u32, _vp, _vp, _vp, _vp], _int),
            "pots_update_plan_create": ([_sz, _vp, ctypes.c_float, ctypes.c_float,
                                         ctypes.POINTER(_vp)], _int),
            "pots_update_plan_run": ([_vp, _vp, _vp], _int),
            "pots_update_plan_bytes": ([_vp], _u64),
            "pots_update_plan_destroy": ([_vp], None),
        }
        for name, (args, res) in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        self._lib = lib
        self.version = lib.pots_mi355x_version().decode()
        self.blake3_version = lib.pots_blake3_version().decode()
        self.simd_degree = int(lib.pots_simd_degree())

    # ---- errors --------------------------------------------------------------------------

    def _check(self, rc: int, what: str) -> None:
        if rc == E_OK:
            return
        if rc == E_ARG:
            raise ValueError(f"{what}: argument rejected by libpots_mi355x")
        msg = self._lib.pots_last_error().decode()
        raise NativeError(f"{what} failed with {rc}: {msg}")

    # ---- the reference's methods ---------------------------------------------------------

    def hash_leaves(self, hdr_buf: bytes, hdr_off: np.ndarray, hdr_len: np.ndarray,
                    hdr_idx: np.ndarray, payload_ptr: np.ndarray, payload_len: np.ndarray,
                    kind: np.ndarray, *, threads: int = 1,
                    noalloc: bool = False) -> tuple[np.ndarray, int]:
        """``(digests, first_bad)`` of native.py:286-311: leaf ``i``'s digest is
        ``BLAKE3(0x00 ‖ header ‖ payload)``, uint8 ``[n, 32]``; ``first_bad`` is the first leaf
        whose payload holds NaN or Inf, or ``n``. Payload addresses may be host or device
        memory; the caller keeps them alive until the call returns. ``noalloc`` takes the
        entry point that allocates no device memory (``pots_hash_leaves_noalloc``, bounded
        by its static scratch)."""
        n = len(payload_ptr)
        if not len(payload_len) == len(kind) == len(hdr_idx) == n:
            raise ValueError("payload_ptr, payload_len, kind and hdr_idx must have one length")
        if len(hdr_off) != len(hdr_len):
            raise ValueError("hdr_off and hdr_len must have one length")
        if n and (int(np.max(hdr_idx)) >= len(hdr_off)
                  or int((np.asarray(hdr_off, dtype=np.uint64)
                          + np.asarray(hdr_len, dtype=np.uint64)).max()) > len(hdr_buf)):
            raise ValueError("a header index or range is out of bounds")
        out = np.empty((n, 32), dtype=np.uint8)
        if n == 0:
            return out, 0
        hb = np.frombuffer(bytes(hdr_buf) or b"\0", dtype=np.uint8)
        arrs = [np.ascontiguousarray(x, dtype=t) for x, t in (
            (hdr_off, np.uint64), (hdr_len, np.uint32), (hdr_idx, np.uint32),
            (payload_ptr, np.uint64), (payload_len, np.uint64), (kind, np.uint8))]
        fn = self._lib.pots_hash_leaves_noalloc if noalloc else self._lib.pots_hash_leaves
        bad = fn(n, _addr(hb), *map(_addr, arrs), _addr(out), max(1, int(threads)))
        if bad == _SIZE_MAX:
            raise NativeError(f"{fn.__name__} failed: " + self._lib.pots_last_error().decode())
        return out, int(bad)

    def all_finite(self, ptr: int, nbytes: int, kind: int, *, threads: int = 1) -> bool:
        """Whether every value of the ``nbytes`` bytes at ``ptr`` (host or device) is finite."""
        if nbytes < 0 or (ptr == 0 and nbytes > 0):
            raise ValueError(f"bad buffer: ptr={ptr}, nbytes={nbytes}")
        rc = self._lib.pots_all_finite(ptr, nbytes, kind, max(1, int(threads)))
        if rc < 0:
            self._check(rc, "pots_all_finite")
        return bool(rc)

    def merkle_tree(self, leaves: bytes, n: int) -> bytes:
        """The ``2n − 1`` pre-order node hashes of the RFC 6962 tree (native.py:319-327)."""
        if n < 1 or len(leaves) != 32 * n:
            raise ValueError(f"need n >= 1 and 32·n bytes of leaves, got n={n}, {len(leaves)}")
        out = ctypes.create_string_buffer(32 * (2 * n - 1))
        self._check(self._lib.pots_merkle_tree(n, bytes(leaves), out), "pots_merkle_tree")
        return out.raw

    # ---- device-resident entry points -----------------------------------------------------

    def merkle_tree_device(self, digests: torch.Tensor,
                           stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """The pre-order node buffer, uint8 ``[2n − 1, 32]`` on the digests' device, of the
        tree over ``digests`` (uint8 ``[n, 32]`` in HBM). Stream-ordered, no sync."""
        if digests.dtype != torch.uint8 or digests.dim() != 2 or digests.shape[1] != 32:
            raise ValueError("digests must be uint8 [n, 32]")
        if not digests.is_cuda or not digests.is_contiguous():
            raise ValueError("digests must be a contiguous GPU tensor")
        n = digests.shape[0]
        if n < 1:
            raise ValueError("a Merkle tree needs at least one leaf")
        nodes = torch.empty(2 * n - 1, 32, dtype=torch.uint8, device=digests.device)
        self._check(self._lib.pots_merkle_tree_async(n, digests.data_ptr(), nodes.data_ptr(),
                                                     _stream(stream)), "pots_merkle_tree_async")
        return nodes

    def challenge_matrices(self, h: bytes, ms: Sequence[int], k: int, width: int, *,
                           threads: int = 1, device: torch.device | str = "cuda"
                           ) -> torch.Tensor:
        """The protocol's ``challenge_matrices``, bit for bit: fp32 ``[len(ms), width, k]``
        on the GPU (native.py:263-284)."""
        if len(h) != 32:
            raise ValueError("h must be 32 bytes")
        if not 1 <= k <= 255:
            raise ValueError(f"k must be in [1, 255], got {k}")
        if not 1 <= width < 1 << 32:
            raise ValueError(f"width must be in [1, 2^32), got {width}")
        for m in ms:
            if not 1 <= m < 1 << 32:
                raise ValueError(f"m must be in [1, 2^32), got {m}")
        n = len(ms)
        out = torch.empty(n, width, k, dtype=torch.float32, device=device)
        if n == 0:
            return out
        msa = np.asarray(ms, dtype=np.uint32)
        widths = np.full(n, width, dtype=np.uint32)
        offs = np.arange(n, dtype=np.uint64) * np.uint64(width * k)
        self._check(self._lib.pots_challenges(bytes(h), k, n, _addr(msa), _addr(widths),
                                              _addr(offs), out.data_ptr(), 1),
                    "pots_challenges")
        return out

    def fv_plan(self, products: Sequence[FvProduct], k: int, guard: bool = True) -> FvPlan:
        """A Freivalds plan over GPU-resident products (``pots_fv_plan_*``)."""
        return FvPlan(self, products, k, guard)

    def verdicts(self, rows: torch.Tensor, specs: torch.Tensor, *, k: int, eps_in: float,
                 eps_acc: float, tau: float, guard: bool = True, judge: bool = True,
                 finished: bool = False, stream: torch.cuda.Stream | None = None
                 ) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
        """Per-product verdicts on the GPU: ``(codes int32 [n, 2], finished fp64 [n, 3] or
        None, first_fail int32 [1])``. ``specs`` is the packed per-product table of
        :func:`verdict_specs`."""
        import math
        n = rows.shape[0]
        dev = rows.device
        codes = torch.empty(n, 2, dtype=torch.int32, device=dev)
        fin = torch.empty(n, 3, dtype=torch.float64, device=dev) if finished else None
        first = torch.empty(1, dtype=torch.int32, device=dev)
        if n == 0:
            first.fill_(0)
            return codes, fin, first
        if rows.dtype != torch.float64 or not rows.is_contiguous() or rows.shape[1] != 5 + k:
            raise ValueError("rows must be contiguous fp64 [n, 5 + k]")
        self._check(self._lib.pots_verdicts_async(
            n, rows.data_ptr(), k, specs.data_ptr(), float(eps_in), float(eps_acc), float(tau),
            1.0 / math.sqrt(3.0), math.sqrt(2.0), int(bool(guard)), int(bool(judge)),
            codes.data_ptr(), fin.data_ptr() if fin is not None else None, first.data_ptr(),
            _stream(stream)), "pots_verdicts_async")
        return codes, fin, first

    def update_plan(self, weights: Sequence[UpdateWeight], eta: float, eps_w: float
                    ) -> UpdatePlan:
        """Check 6a's update-identity plan over GPU-resident weights (``pots_update_plan_*``)."""
        return UpdatePlan(self, weights, eta, eps_w)

    def leaf_plan(self, headers: Sequence[bytes], payloads: Sequence[torch.Tensor],
                  kinds: Sequence[int], fuse: FvPlan | None = None) -> LeafPlan:
        """A reusable hashing plan over GPU-resident payloads: leaf ``i`` is
        ``BLAKE3(0x00 ‖ headers[i] ‖ payload bytes of payloads[i])``. With ``fuse``, the
        leaves that are the P of a product of that Freivalds plan also have its P-pass sums
        taken by the chunk stage (``pots_leaf_plan_create_fused``)."""
        return LeafPlan(self, headers, payloads, kinds, fuse)

    def step_run(self, leaf: LeafPlan, fv: FvPlan, key: torch.Tensor, digests: torch.Tensor,
                 bad: torch.Tensor, rows: torch.Tensor,
                 stream: torch.cuda.Stream | None = None) -> None:
        """``pots_step_run``: fv stage 0, the leaf plan, fv stages 1-5, on one stream."""
        if digests.shape != (leaf.n, 32) or digests.dtype != torch.uint8:
            raise ValueError("digests must be uint8 [n, 32]")
        if rows.shape != (fv.n, 5 + fv.k) or rows.dtype != torch.float64:
            raise ValueError("rows must be fp64 [n, 5 + k]")
        self._check(self._lib.pots_step_run(leaf._h, fv._h, key.data_ptr(), digests.data_ptr(),
                                            bad.data_ptr(), rows.data_ptr(), _stream(stream)),
                    "pots_step_run")


class LeafPlan:
    """``pots_leaf_plan_*``: metadata uploaded once, then :meth:`run` enqueues the hashing of
    every leaf on a stream with no allocation and no host sync."""

    def __init__(self, lib: Native, headers: Sequence[bytes], payloads: Sequence[torch.Tensor],
                 kinds: Sequence[int], fuse: FvPlan | None = None) -> None:
        n = len(payloads)
        if not (len(headers) == len(kinds) == n) or n == 0:
            raise ValueError("one header and one kind per payload, at least one leaf")
        uniq: dict[bytes, int] = {}
        idx = np.empty(n, dtype=np.uint32)
        for i, h in enumerate(headers):
            idx[i] = uniq.setdefault(bytes(h), len(uniq))
        hdrs = list(uniq)
        hdr_len = np.array([len(h) for h in hdrs], dtype=np.uint32)
        hdr_off = np.zeros(len(hdrs), dtype=np.uint64)
        if len(hdrs) > 1:
            hdr_off[1:] = np.cumsum(hdr_len[:-1], dtype=np.uint64)
        ptr = np.empty(n, dtype=np.uint64)
        ln = np.empty(n, dtype=np.uint64)
        for i, t in enumerate(payloads):
            if not (t.is_cuda and t.is_contiguous()):
                raise ValueError(f"payload {i} must be a contiguous GPU tensor")
            ptr[i], ln[i] = t.data_ptr(), t.nbytes
        self._create(lib, b"".join(hdrs), hdr_off, hdr_len, idx, ptr, ln,
                     np.asarray(kinds, dtype=np.uint8), fuse, list(payloads),
                     payloads[0].device)

    @classmethod
    def from_arrays(cls, lib: Native, hdr_buf: bytes, hdr_off: np.ndarray, hdr_len: np.ndarray,
                    hdr_idx: np.ndarray, payload_ptr: np.ndarray, payload_len: np.ndarray,
                    kind: np.ndarray, device: torch.device,
                    fuse: FvPlan | None = None) -> LeafPlan:
        """A plan over ``pots_hash_leaves``'s arguments (every payload in device memory, or
        empty), fused with ``fuse`` if given. It keeps no tensor: the caller keeps the
        payloads alive and in place while its runs are in flight."""
        self = cls.__new__(cls)
        self._create(lib, hdr_buf, hdr_off, hdr_len, hdr_idx, payload_ptr, payload_len, kind,
                     fuse, [], device)
        return self

    def _create(self, lib: Native, hdr_buf: bytes, hdr_off: np.ndarray, hdr_len: np.ndarray,
                idx: np.ndarray, ptr: np.ndarray, ln: np.ndarray, kd: np.ndarray,
                fuse: FvPlan | None, keep: list[Any], device: torch.device) -> None:
        n = len(idx)
        if not (len(ptr) == len(ln) == len(kd) == n) or n == 0:
            raise ValueError("one header index, payload and kind per leaf, at least one leaf")
        self._lib = lib
        self._keep = keep
        hb = np.frombuffer(hdr_buf or b"\0", dtype=np.uint8)
        idx = np.ascontiguousarray(idx, dtype=np.uint32)
        hdr_off = np.ascontiguousarray(hdr_off, dtype=np.uint64)
        hdr_len = np.ascontiguousarray(hdr_len, dtype=np.uint32)
        ptr = np.ascontiguousarray(ptr, dtype=np.uint64)
        ln = np.ascontiguousarray(ln, dtype=np.uint64)
        kd = np.ascontiguousarray(kd, dtype=np.uint8)
        h = ctypes.c_void_p()
        if fuse is None:
            _create(lib, lambda: lib._lib.pots_leaf_plan_create(
                n, _addr(hb), _addr(hdr_off), _addr(hdr_len), _addr(idx), _addr(ptr), _addr(ln),
                _addr(kd), ctypes.byref(h)), "pots_leaf_plan_create")
        else:
            if fuse._fused_leaf is not None:
                raise ValueError("this Freivalds plan is already fused with a leaf plan")
            _create(lib, lambda: lib._lib.pots_leaf_plan_create_fused(
                n, _addr(hb), _addr(hdr_off), _addr(hdr_len), _addr(idx), _addr(ptr), _addr(ln),
                _addr(kd), fuse._h, ctypes.byref(h)), "pots_leaf_plan_create_fused")
            fuse._fused_leaf = weakref.ref(self)
        self._h = h
        _LIVE_PLANS.add(self)
        # The chunk stage of a fused plan writes into the Freivalds plan's records and reads
        # its challenges: the Freivalds plan lives at least as long.
        self._fv = fuse
        self.fused = int(lib._lib.pots_leaf_plan_fused(h))
        st = (ctypes.c_uint64 * 3)()
        lib._check(lib._lib.pots_leaf_plan_fused_stats(h, ctypes.byref(st, 0),
                                                       ctypes.byref(st, 8),
                                                       ctypes.byref(st, 16)),
                   "pots_leaf_plan_fused_stats")
        # the fused chunk kernel's message bytes, chunks and run records per run
        self.fused_bytes, self.fused_chunks, self.fused_records = (int(x) for x in st)
        self.n = n
        self.chunks = int(lib._lib.pots_leaf_plan_chunks(h))
        self.bytes = int(lib._lib.pots_leaf_plan_bytes(h))
        self.device = device

    def run(self, out: torch.Tensor | None = None, bad: torch.Tensor | None = None,
            stream: torch.cuda.Stream | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Enqueue the hashing: ``(digests uint8 [n, 32], first_bad int32 [1])`` on the GPU."""
        if out is None:
            out = torch.empty(self.n, 32, dtype=torch.uint8, device=self.device)
        if bad is None:
            bad = torch.empty(1, dtype=torch.int32, device=self.device)
        if out.shape != (self.n, 32) or out.dtype != torch.uint8 or not out.is_contiguous():
            raise ValueError("out must be contiguous uint8 [n, 32]")
        self._lib._check(self._lib._lib.pots_leaf_plan_run(self._h, out.data_ptr(),
                                                           bad.data_ptr(), _stream(stream)),
                         "pots_leaf_plan_run")
        return out, bad

    STAGES = ("stage", "chunks", "levels")
    # Stage 1's two kernels on their own (pots_leaf_plan_run_stage): the fused leaves' chunks
    # and the other leaves' chunks.
    FUSED_CHUNKS, PLAIN_CHUNKS = 3, 4

    def set_grid(self, max_blocks: int) -> None:
        """Limit the chunk kernel to ``max_blocks`` blocks (0: no limit); results are the same,
        the kernel just leaves the rest of the GPU to other streams."""
        if not 0 <= max_blocks < 1 << 32:
            raise ValueError(f"max_blocks must be in [0, 2^32), got {max_blocks}")
        self._lib._check(self._lib._lib.pots_leaf_plan_set_grid(self._h, max_blocks),
                         "pots_leaf_plan_set_grid")

    def run_stage(self, stage: int, out: torch.Tensor, bad: torch.Tensor,
                  stream: torch.cuda.Stream | None = None) -> None:
        """Enqueue one stage of :meth:`run` (``STAGES``: staging copies, the chunk kernel,
        the per-leaf tree levels); running all of them in order is :meth:`run`."""
        if out.shape != (self.n, 32) or out.dtype != torch.uint8 or not out.is_contiguous():
            raise ValueError("out must be contiguous uint8 [n, 32]")
        self._lib._check(self._lib._lib.pots_leaf_plan_run_stage(
            self._h, stage, out.data_ptr(), bad.data_ptr(), _stream(stream)),
            "pots_leaf_plan_run_stage")

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib._lib.pots_leaf_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


DT_F32, DT_BF16 = 0, 1
_DT = {torch.float32: DT_F32, torch.bfloat16: DT_BF16}


class _FvProductC(ctypes.Structure):
    _fields_ = [("a", _vp), ("b", _vp), ("p", _vp), ("bias", _vp), ("lda", _u64),
                ("ldb", _u64), ("ldp", _u64), ("n", _u32), ("q", _u32), ("w", _u32),
                ("m", _u32), ("a_dtype", _u32), ("b_dtype", _u32), ("p_dtype", _u32),
                ("a_trans", _u32)]


# _FvProductC as a numpy record, so a plan's table is filled column by column
_FV_RECORD = np.dtype([("a", "<u8"), ("b", "<u8"), ("p", "<u8"), ("bias", "<u8"),
                       ("lda", "<u8"), ("ldb", "<u8"), ("ldp", "<u8"), ("n", "<u4"),
                       ("q", "<u4"), ("w", "<u4"), ("m", "<u4"), ("a_dtype", "<u4"),
                       ("b_dtype", "<u4"), ("p_dtype", "<u4"), ("a_trans", "<u4")])
assert _FV_RECORD.itemsize == ctypes.sizeof(_FvProductC)


class FvProduct:
    """One checked product for :class:`FvPlan`: GPU tensors ``a`` [n, q], ``b`` [q, w], ``p``
    [n, w] (fp32 or bf16), an optional fp32 ``bias`` [w], and the challenge label ``m``.
    The kernels stream rows with unit column stride; an operand in another layout (a
    transposed view such as a linear layer's ``W.t()``, as captured operands are) is copied
    to that layout by the plan, once, when the plan is built."""

    __slots__ = ("a", "b", "p", "bias", "m")

    def __init__(self, a: torch.Tensor, b: torch.Tensor, p: torch.Tensor, m: int,
                 bias: torch.Tensor | None = None) -> None:
        self.a, self.b, self.p, self.m, self.bias = a, b, p, m, bias


def verdict_specs(qs: Sequence[int], ns: Sequence[int], biased: Sequence[bool],
                  kappa_max: Sequence[float], device: torch.device | str = "cuda"
                  ) -> torch.Tensor:
    """The per-product table ``pots_verdicts_async`` reads: 24-byte records
    ``{double kappa_max; uint32 q, n, biased, pad}``."""
    n = len(qs)
    rec = np.zeros(n, dtype=np.dtype([("kappa", "<f8"), ("q", "<u4"), ("n", "<u4"),
                                      ("biased", "<u4"), ("pad", "<u4")]))
    rec["kappa"] = np.asarray(kappa_max, dtype=np.float64)
    rec["q"] = np.asarray(qs, dtype=np.uint32)
    rec["n"] = np.asarray(ns, dtype=np.uint32)
    rec["biased"] = np.asarray(biased, dtype=np.uint32)
    return torch.from_numpy(rec.view(np.uint8).copy()).to(device)


def _row_major(t: torch.Tensor) -> torch.Tensor:
    """``t`` if its rows are contiguous and do not overlap, else a row-major copy."""
    if isinstance(t, torch.Tensor) and t.dim() == 2:
        s0, s1 = t.stride()
        if (s1 != 1 or s0 < t.shape[1]) and t.numel():
            return t.contiguous()
    return t


def _twin_mates(products: Sequence[FvProduct], k: int | None) -> dict[int, int]:
    """``{i: j}`` for each product ``i`` whose ``A`` is a transposed view of product ``j``'s
    row-major ``A`` (the same storage, shape swapped), where the plan's twin pass can read
    that operand once for both: bf16, ``k ≤ 4``, ``X = A_iᵀ`` with rows a multiple of 16 and
    columns of 128, 16-byte aligned rows. Each ``j`` is taken once."""
    if k is None or not 1 <= k <= 4:
        return {}
    rowmajor: dict[tuple[int, int, int, int], list[int]] = {}
    for j, pr in enumerate(products):
        a = pr.a
        if a.dim() == 2 and a.dtype == torch.bfloat16 and a.is_cuda and a.stride(1) == 1 \
                and a.stride(0) >= a.shape[1]:
            rowmajor.setdefault((a.data_ptr(), a.shape[0], a.shape[1], a.stride(0)),
                                []).append(j)
    mates: dict[int, int] = {}
    taken: set[int] = set()
    for i, pr in enumerate(products):
        a = pr.a
        if not (a.dim() == 2 and a.dtype == torch.bfloat16 and a.is_cuda and
                a.stride(0) == 1 and a.shape[0] > 1 and a.stride(1) >= a.shape[0]):
            continue
        n, q = a.shape            # A = Xᵀ: X is [q, n] with row stride ld
        ld = a.stride(1)
        if q % 16 or n % 128 or a.data_ptr() % 16 or (2 * ld) % 16:
            continue
        for j in rowmajor.get((a.data_ptr(), q, n, ld), ()):
            if j not in taken and j != i:
                mates[i] = j
                taken.add(j)
                break
    return mates


def fv_table(products: Sequence[FvProduct], k: int | None = None
             ) -> tuple[np.ndarray, list[torch.Tensor], dict[tuple[int, str], torch.Tensor]]:
    """The product table ``pots_fv_plan_create`` reads (one ``pots_fv_product`` per product),
    the tensors it points into, which must stay alive while a plan built on it runs, and the
    ones of those this call made, by ``(product index, field)``: a product's fp32 bias
    (``"bias"``) and row-major copies of operands in another layout (``"a"``, ``"b"``,
    ``"p"``).

    With ``k`` given, an ``A`` that is the transpose of another product's row-major ``A`` is
    passed as it lies (``a_trans``), for the plan's twin pass, where :func:`_twin_mates`
    allows it; any other transposed operand is copied to row-major."""
    table = []
    keep = []
    made: dict[tuple[int, str], torch.Tensor] = {}
    dts = _DT
    mates = _twin_mates(products, k)
    for i, pr in enumerate(products):
        a, b, p = pr.a, pr.b, pr.p
        a_trans = 0
        if i in mates:  # A = Xᵀ of its twin's X, read by the twin pass where it lies
            a_trans = 1
            x = a.t()
            keep.append(a)
            a = x
        sa, sb, sp = a.stride(), b.stride(), p.stride()
        ash, bsh, psh = a.shape, b.shape, p.shape
        # The common case (row-major 2-D GPU operands in fp32 or bf16) is read once;
        # anything else is made row-major and validated operand by operand.
        if not (len(sa) == len(sb) == len(sp) == 2 and sa[1] == sb[1] == sp[1] == 1 and
                sa[0] >= ash[1] and sb[0] >= bsh[1] and sp[0] >= psh[1] and
                a.is_cuda and b.is_cuda and p.is_cuda and a.dtype in dts and
                b.dtype in dts and p.dtype in dts):
            given = (a, b, p)
            a, b, p = (_row_major(t) for t in given)
            for name, t, t0 in (("a", a, given[0]), ("b", b, given[1]), ("p", p, given[2])):
                if t is not t0:
                    made[(i, name)] = t
                if not t.is_cuda or t.dim() != 2 or t.stride(1) != 1 or t.dtype not in dts:
                    raise ValueError(f"product {i}: {name} must be a 2-D GPU tensor in "
                                     f"fp32 or bf16")
            sa, sb, sp = a.stride(), b.stride(), p.stride()
            ash, bsh, psh = a.shape, b.shape, p.shape
        nn, q = ash
        if a_trans:
            nn, q = q, nn  # the product's A is [n, q] = Xᵀ
        q2, w = bsh
        if q2 != q or psh[0] != nn or psh[1] != w:
            raise ValueError(f"product {i}: shapes {(nn, q)}·{tuple(bsh)} vs "
                             f"{tuple(psh)}")
        if not 1 <= pr.m < 1 << 32:
            raise ValueError(f"m must be in [1, 2^32), got {pr.m}")
        bias = pr.bias
        if bias is not None:
            bias = bias.detach().to(device=a.device, dtype=torch.float32).contiguous()
            if bias.shape != (w,):
                raise ValueError(f"product {i}: bias of shape {tuple(bias.shape)}, "
                                 f"expected ({w},)")
            keep.append(bias)
            made[(i, "bias")] = bias
        table.append((a.data_ptr(), b.data_ptr(), p.data_ptr(),
                      bias.data_ptr() if bias is not None else 0, sa[0], sb[0], sp[0],
                      nn, q, w, pr.m, dts[a.dtype], dts[b.dtype], dts[p.dtype], a_trans))
        keep += [a, b, p]
    return np.array(table, dtype=_FV_RECORD), keep, made


class FvPlan:
    """``pots_fv_plan_*``: operand layout and workspace fixed once; :meth:`rows` enqueues the
    challenges, the three streaming passes and the reduction for every product."""

    def __init__(self, lib: Native, products: Sequence[FvProduct], k: int,
                 guard: bool = True,
                 table: tuple[np.ndarray, list[torch.Tensor], Any] | None = None) -> None:
        n = len(products)
        if n == 0:
            raise ValueError("a Freivalds plan needs at least one product")
        if not 1 <= k <= 255:
            raise ValueError(f"k must be in [1, 255], got {k}")
        arr, keep, _ = table if table is not None else fv_table(products, k)
        self._create(lib, arr, keep, k, guard, products[0].a.device)

    @classmethod
    def from_table(cls, lib: Native, table: np.ndarray, keep: list[torch.Tensor], k: int,
                   guard: bool, device: torch.device) -> FvPlan:
        """A plan over a product table already made (``fv_table``'s records); ``keep`` holds
        the tensors it points into while the plan's runs are in flight."""
        if len(table) == 0:
            raise ValueError("a Freivalds plan needs at least one product")
        if not 1 <= k <= 255:
            raise ValueError(f"k must be in [1, 255], got {k}")
        self = cls.__new__(cls)
        self._create(lib, np.ascontiguousarray(table, dtype=_FV_RECORD), keep, k, guard, device)
        return self

    def _create(self, lib: Native, arr: np.ndarray, keep: list[torch.Tensor], k: int,
                guard: bool, device: torch.device) -> None:
        n = len(arr)
        h = ctypes.c_void_p()
        _create(lib, lambda: lib._lib.pots_fv_plan_create(n, arr.ctypes.data, k,
                                                          int(bool(guard)), ctypes.byref(h)),
                "pots_fv_plan_create")
        self._lib, self._h, self._keep = lib, h, keep
        _LIVE_PLANS.add(self)
        self._fused_leaf = None  # weak reference to the leaf plan fused with this one
        self.n, self.k = n, k
        self.widths = [int(w) for w in arr["w"]]
        self.device = device
        self.bytes = int(lib._lib.pots_fv_plan_bytes(h))
        # pairs of products whose shared operand (A and Aᵀ) the twin pass reads once
        self.twins = int(lib._lib.pots_fv_plan_twins(h))
        self._key = torch.empty(32, dtype=torch.uint8, device=self.device)

    def rows(self, h: bytes | torch.Tensor, out: torch.Tensor | None = None,
             stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """fp64 ``[n, 5 + k]`` rows (``freivalds.ROW``), challenges keyed on ``h`` (32 bytes,
        host bytes or a GPU uint8 tensor). Stream-ordered, no sync."""
        if isinstance(h, torch.Tensor):
            key = h
        else:
            if len(h) != 32:
                raise ValueError("h must be 32 bytes")
            key = self._key
            key.copy_(torch.frombuffer(bytearray(h), dtype=torch.uint8), non_blocking=False)
        if out is None:
            out = torch.empty(self.n, 5 + self.k, dtype=torch.float64, device=self.device)
        self._lib._check(self._lib._lib.pots_fv_plan_run(self._h, key.data_ptr(), out.data_ptr(),
                                                         _stream(stream)), "pots_fv_plan_run")
        return out

    STAGES = ("challenges", "b_pass", "reduce", "a_pass", "p_pass", "rows")
    # Stage 4's two parts on their own: the row pass over the unfused products' P, and the
    # fused products' sums from the leaf plan's run records.
    P_PASS, P_FUSED = 6, 7
    # Stage 3's two parts on their own: the row pass over the A's of products with no twin,
    # and the twin pass over the twins' shared operands.
    A_ROWS, TWINS = 8, 9

    def run_stage(self, stage: int, key: torch.Tensor, out: torch.Tensor,
                  stream: torch.cuda.Stream | None = None) -> None:
        """Enqueue one stage of :meth:`rows` (``STAGES``) with the key already a GPU uint8
        tensor; running all of them in order is :meth:`rows`."""
        if out.shape != (self.n, 5 + self.k) or out.dtype != torch.float64:
            raise ValueError("out must be fp64 [n, 5 + k]")
        self._lib._check(self._lib._lib.pots_fv_plan_run_stage(
            self._h, stage, key.data_ptr(), out.data_ptr(), _stream(stream)),
            "pots_fv_plan_run_stage")

    def set_grid(self, stage: int, max_blocks: int) -> None:
        """Limit the row pass of ``stage`` (1 B, 3 A, 4 P) to ``max_blocks`` blocks (0: no
        limit); results are the same, the pass just leaves the rest of each CU to other
        streams."""
        if not 0 <= max_blocks < 1 << 32:
            raise ValueError(f"max_blocks must be in [0, 2^32), got {max_blocks}")
        self._lib._check(self._lib._lib.pots_fv_plan_set_grid(self._h, stage, max_blocks),
                         "pots_fv_plan_set_grid")

    def challenges(self) -> list[torch.Tensor]:
        """The last run's challenge matrices, fp32 ``[w_i, k]`` per product (GPU views)."""
        total = sum(self.widths) * self.k
        flat = torch.empty(total, dtype=torch.float32, device=self.device)
        self._lib._check(self._lib._lib.pots_fv_plan_copy_challenges(
            self._h, flat.data_ptr(), _stream(None)), "pots_fv_plan_copy_challenges")
        out, at = [], 0
        for w in self.widths:
            out.append(flat[at:at + w * self.k].view(w, self.k))
            at += w * self.k
        return out

    def close(self) -> None:
        leaf = self._fused_leaf() if getattr(self, "_fused_leaf", None) is not None else None
        if leaf is not None:  # its chunk stage writes into this plan's memory
            leaf.close()
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib._lib.pots_fv_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


UPDATE_MAX_PARTS = 8


class _UpdateWeightC(ctypes.Structure):
    _fields_ = [("w_t", _vp), ("w_next", _vp), ("parts", _vp * UPDATE_MAX_PARTS),
                ("part_dtype", _u32 * UPDATE_MAX_PARTS), ("n_parts", _u32), ("pad", _u32),
                ("n", _u64), ("tau_w", ctypes.c_double)]


class UpdateWeight:
    """One weight for :class:`UpdatePlan`: GPU tensors ``w_t``, ``w_next`` (fp32) and the
    gradient's ``parts`` (fp32 or bf16, each of ``w_t``'s shape, summed in order), and its
    band ``tau_w``."""

    __slots__ = ("w_t", "w_next", "parts", "tau_w")

    def __init__(self, w_t: torch.Tensor, w_next: torch.Tensor, parts: Sequence[torch.Tensor],
                 tau_w: float) -> None:
        self.w_t, self.w_next, self.parts, self.tau_w = w_t, w_next, tuple(parts), tau_w


class UpdatePlan:
    """``pots_update_plan_*``: check 6a's pass over every weight, enqueued per run; results
    land in a device array of ``(ρ_max bits, first non-finite, first over τ_W)`` per weight
    (``UINT64_MAX`` for none)."""

    NONE = (1 << 64) - 1

    def __init__(self, lib: Native, weights: Sequence[UpdateWeight], eta: float,
                 eps_w: float) -> None:
        n = len(weights)
        if n == 0:
            raise ValueError("an update plan needs at least one weight")
        arr = (_UpdateWeightC * n)()
        keep = []
        for i, w in enumerate(weights):
            ts = (w.w_t, w.w_next, *w.parts)
            for t in ts:
                if not (t.is_cuda and t.is_contiguous()):
                    raise ValueError(f"weight {i}: tensors must be contiguous GPU tensors")
                if t.shape != w.w_t.shape:
                    raise ValueError(f"weight {i}: shape {tuple(t.shape)} != "
                                     f"{tuple(w.w_t.shape)}")
            if w.w_t.dtype != torch.float32 or w.w_next.dtype != torch.float32:
                raise ValueError(f"weight {i}: W_t and W_t+1 must be fp32")
            if not 1 <= len(w.parts) <= UPDATE_MAX_PARTS:
                raise ValueError(f"weight {i}: 1..{UPDATE_MAX_PARTS} gradient parts")
            c = arr[i]
            c.w_t, c.w_next = w.w_t.data_ptr(), w.w_next.data_ptr()
            for j, p in enumerate(w.parts):
                if p.dtype not in (torch.float32, torch.bfloat16):
                    raise ValueError(f"weight {i}: gradient parts must be fp32 or bf16")
                c.parts[j] = p.data_ptr()
                c.part_dtype[j] = 1 if p.dtype == torch.bfloat16 else 0
            c.n_parts = len(w.parts)
            c.n = w.w_t.numel()
            c.tau_w = float(w.tau_w)
            keep += list(ts)
        h = ctypes.c_void_p()
        _create(lib, lambda: lib._lib.pots_update_plan_create(
            n, ctypes.addressof(arr), float(np.float32(eta)), float(np.float32(eps_w)),
            ctypes.byref(h)), "pots_update_plan_create")
        self._lib, self._h, self._keep = lib, h, keep
        _LIVE_PLANS.add(self)
        self.n = n
        self.device = weights[0].w_t.device
        self.bytes = int(lib._lib.pots_update_plan_bytes(h))

    def run(self, out: torch.Tensor | None = None,
            stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """Enqueue the pass: uint64 results ``[n, 3]`` (as int64) on the GPU, no sync."""
        if out is None:
            out = torch.empty(self.n, 3, dtype=torch.int64, device=self.device)
        self._lib._check(self._lib._lib.pots_update_plan_run(self._h, out.data_ptr(),
                                                             _stream(stream)),
                         "pots_update_plan_run")
        return out

    @staticmethod
    def decode(out: torch.Tensor) -> list[tuple[float, int | None, int | None]]:
        """Host view of :meth:`run`'s results: ``(ρ_max, first_nonfinite, first_over)`` per
        weight, the indices ``None`` where no entry qualifies."""
        raw = out.cpu().numpy().view(np.uint64)
        rho = raw[:, 0].copy().view(np.float64)
        res = []
        for i in range(raw.shape[0]):
            nf, ov = int(raw[i, 1]), int(raw[i, 2])
            res.append((float(rho[i]), None if nf == UpdatePlan.NONE else nf,
                        None if ov == UpdatePlan.NONE else ov))
        return res

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib._lib.pots_update_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


_LIB: Native | None = None
_LOCK = threading.Lock()


def get() -> Native:
    """The library, loaded once per process. Raises ``RuntimeError`` when it is missing or no
    GPU is visible: this build has no CPU fallback."""
    global _LIB
    with _LOCK:
        if _LIB is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                                   "`python pots-2.0_amd/build.py` (hipcc, gfx950)")
            if not torch.cuda.is_available():
                raise RuntimeError("libpots_mi355x needs a GPU and none is visible")
            torch.cuda.init()
            _LIB = Native(LIB_PATH)
        return _LIB


_disabled = 0
_disabled_lock = threading.Lock()


def enabled() -> bool:
    """False inside :func:`disabled`. Kept for the reference's callers, which read it. Unlike
    the reference (native.py:353-368), nothing switches on it: there is no CPU hashing path in
    the product, so the GPU library serves every call either way."""
    return _disabled == 0


@contextmanager
def disabled() -> Iterator[None]:
    """Make :func:`enabled` return False inside the block. Nestable. A flag only: calls
    inside the block still run on the GPU library."""
    global _disabled
    with _disabled_lock:
        _disabled += 1
    try:
        yield
    finally:
        with _disabled_lock:
            _disabled -= 1


def describe() -> dict[str, object]:
    """The library this process uses, for an environment record. Never builds."""
    out: dict[str, object] = {"enabled": enabled(), "library": None, "version": None,
                              "error": None}
    try:
        lib = _LIB
        if lib is None:
            if not LIB_PATH.exists():
                return out
            out["library"] = LIB_PATH.name
            return out
        out.update(library=Path(lib.path).name, version=lib.version)
    except Exception as e:
        out["error"] = f"{type(e).__name__}: {e}"
    return out
