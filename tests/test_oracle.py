"""The CPU oracle against the reference's known answers, BLAKE3's published vectors, an
independent second implementation, and the closed forms the mathematics fixes.

These pin the oracle before it is trusted as the GPU kernels' checker: a dropped flag, a
wrong permutation word, a tree split off by one, a byte-order slip in the label or the entry
map, or a transposed challenge matrix fails at least one test here.
"""

from __future__ import annotations

import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

import blake3_tree
import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
KA = json.loads((GOLDEN / "blake3_known_answers.json").read_text())


def seq(n: int) -> bytes:
    return bytes(i % 251 for i in range(n))


# ---- BLAKE3 --------------------------------------------------------------------------------

def test_reference_keyed_known_answer():
    ref = KA["reference"]["keyed_empty"]
    key = ref["key_ascii"].encode()
    assert O.blake3(b"", key=key).hex() == ref["digest"]
    assert blake3_tree.blake3(b"", key=key).hex() == ref["digest"]


def test_reference_xof_known_answer():
    ref = KA["reference"]["xof_label"]
    key, msg = bytes.fromhex(ref["key_hex"]), bytes.fromhex(ref["input_hex"])
    assert msg == O.encode_label(1, 1)
    assert O.blake3(msg, key=key, length=16).hex() == ref["xof16"]
    assert blake3_tree.blake3(msg, key=key, length=16).hex() == ref["xof16"]
    r = O.challenge_matrices(key, [1], 1, 4)[0, :, 0]
    assert r.tolist() == [x / 2**24 for x in ref["numerators"]]
    assert [f"{v:08x}" for v in r.numpy().view(np.uint32)] == ref["fp32_bits"]


def test_reference_merkle_abc_known_answer():
    ref = KA["reference"]["merkle_abc"]
    hs = [O.hash_leaf(x.encode()) for x in ref["leaves_ascii"]]
    assert O.merkle_root(hs).hex() == ref["root"]
    assert O.merkle_root_recursive(hs).hex() == ref["root"]
    assert O.hash_node(O.hash_node(hs[0], hs[1]), hs[2]).hex() == ref["root"]


@pytest.mark.parametrize("n", sorted(int(k) for k in KA["published"]))
def test_published_vectors(n):
    want = KA["published"][str(n)]
    assert O.blake3(seq(n)).hex() == want
    assert blake3_tree.blake3(seq(n)).hex() == want


LENGTHS = [0, 1, 63, 64, 65, 1023, 1024, 1025, 2047, 2048, 2049, 3072, 4096, 5000, 8193,
           16385, 40000]


@pytest.mark.parametrize("n", LENGTHS)
def test_two_implementations_agree(n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert O.blake3(data) == blake3_tree.blake3(data)
    key = bytes(range(32))
    assert O.blake3(data, key=key, length=100) == blake3_tree.blake3(data, key=key, length=100)


@pytest.mark.parametrize("seek", [0, 1, 63, 64, 65, 1000])
def test_xof_seek_is_a_window_of_the_stream(seek):
    key, msg = bytes(range(32)), O.encode_label(7, 3)
    whole = O.blake3(msg, key=key, length=seek + 200)
    assert O.blake3(msg, key=key, length=200, seek=seek) == whole[seek:]
    assert blake3_tree.blake3(msg, key=key, length=200, seek=seek) == whole[seek:]


def test_golden_leaf_digests_match_the_oracle():
    import sys
    sys.path.insert(0, str(GOLDEN))
    from payloads import DTYPES, payload
    for e in json.loads((GOLDEN / "leaf_digests.json").read_text()):
        t = payload(tuple(e["shape"]), DTYPES[e["dtype"]], e["seed"])
        assert O.tensor_leaf_hash(e["tag"], t).hex() == e["digest"], e


def test_hash_leaves_first_bad_and_kinds():
    ts = [torch.randn(300) for _ in range(10)]
    ts[6][17] = float("nan")
    ts[3][0] = float("-inf")
    items = [(O.tensor_leaf_header(3, t), t, 1) for t in ts]
    digests, bad = O.hash_leaves(items)
    assert bad == 3
    assert digests[:3] == [O.tensor_leaf_hash(3, t) for t in ts[:3]]
    # kind 0 (int32 leaves) never tests
    _, bad = O.hash_leaves([(b"", ts[3], 0)])
    assert bad == 1


def test_simd_leaf_hashing_equals_the_spec_hasher():
    """The bench's CPU baseline hashes with 16 chunks per AVX-512 instruction
    (``blake3_simd.c``); every digest must equal the spec hasher's: message lengths around one
    chunk, 16 chunks (one full batch) and 17 (a batch plus a partial chunk), whole batches with
    and without a tail, headers of 1 to 4 dimensions (the 0x00 ‖ header prefix shifts every
    chunk's start), and a leaf of over 2^16 chunks."""
    g = torch.Generator().manual_seed(8)
    items = []
    for hl_dims in (1, 2, 4):
        shape = (3,) * hl_dims
        hdr = O.tensor_leaf_header(O.TAG_PRODUCT, torch.zeros(shape))
        m0 = 1 + len(hdr)
        for msg in (m0, 1023, 1024, 1025, 2048, 2049, 16 * 1024, 16 * 1024 + 1, 17 * 1024 - 3,
                    32 * 1024, 33 * 1024 + 7, 100_000):
            p = torch.randint(0, 256, (msg - m0,), dtype=torch.uint8, generator=g)
            items.append((hdr, p, 0))
    items.append((b"", torch.randint(0, 256, ((1 << 26) + 5,), dtype=torch.uint8,
                                     generator=g), 0))
    want, bad_want = O.hash_leaves(items)
    got, bad_got = O.hash_leaves(items, simd=True)
    assert bad_got == bad_want == len(items)
    assert got == want


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_simd_leaf_hashing_finds_the_same_first_bad_leaf(dtype):
    """The SIMD path tests each payload for NaN/Inf before hashing it, 64 bytes per compare:
    a value in the vector body or in the scalar tail, in any leaf, gives the spec hasher's first
    bad index and the same digests before it."""
    kind = O.FINITE_KIND[dtype]
    for n, pos in ((1000, 3), (1000, 999), (40, 39), (5000, 2048)):
        ts = [torch.randn(n).to(dtype) for _ in range(6)]
        ts[4][pos] = float("nan")
        ts[2][pos] = float("-inf")
        items = [(O.tensor_leaf_header(3, t), t, kind) for t in ts]
        want, bad_want = O.hash_leaves(items)
        got, bad_got = O.hash_leaves(items, simd=True)
        assert bad_got == bad_want == 2
        assert got[:2] == want[:2]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_kinds_flag_either_half_of_a_word(dtype):
    kind = O.FINITE_KIND[dtype]
    for pos in (0, 1, 6, 7):
        t = torch.ones(8, dtype=dtype)
        t[pos] = float("inf")
        assert not O.all_finite(t)
        _, bad = O.hash_leaves([(b"", t, kind)])
        assert bad == 0
    t = torch.full((5,), -0.0, dtype=dtype)
    assert O.all_finite(t)


# ---- leaf encoding -------------------------------------------------------------------------

def test_encoding_literals():
    ref = KA["reference"]
    assert O.tensor_leaf_header(O.TAG_WEIGHT, torch.zeros(3, 70000)).hex() == \
        ref["header_3x70000_f32_weight_hex"]
    t = torch.tensor([1.0])
    assert (O.tensor_leaf_header(O.TAG_PRODUCT, t) + O.payload_bytes(t)).hex() == \
        ref["product_leaf_1p0_hex"]


def test_record_encoding_layout():
    ids = torch.tensor([1, 2, 3], dtype=torch.int32)
    b = O.encode_record(ids, ids + 1, torch.ones(3, dtype=torch.int32))
    assert b[:6] == bytes([0x01, 0x10, 0, 0, 0, 3]) and len(b) == 6 + 12 * 3
    assert struct.unpack("<3i", b[6:18]) == (1, 2, 3)


# ---- Merkle tree ---------------------------------------------------------------------------

def _leaves(n):
    return [O.hash_leaf(i.to_bytes(4, "big")) for i in range(n)]


@pytest.mark.parametrize("n", [*range(1, 71), 127, 128, 129, 1000])
def test_tree_matches_recursive_definition(n):
    hs = _leaves(n)
    nodes = O.merkle_tree(hs)
    assert len(nodes) == 32 * (2 * n - 1)
    assert nodes[:32] == O.merkle_root_recursive(hs)

    def walk(lo, hi, p):  # every pre-order slot holds its range's recursive root
        assert nodes[32 * p:32 * p + 32] == O.merkle_root_recursive(hs[lo:hi])
        if hi - lo > 1:
            k = 1 << ((hi - lo - 1).bit_length() - 1)
            walk(lo, lo + k, p + 1)
            walk(lo + k, hi, p + 2 * k)
    if n <= 70:
        walk(0, n, 0)


def test_promotion_not_duplication():
    a, b, c = _leaves(3)
    assert O.merkle_root([a, b, c]) == O.hash_node(O.hash_node(a, b), c)
    assert O.merkle_root([a, b, c]) != O.merkle_root([a, b, c, c])


@pytest.mark.parametrize("n", range(1, 41))
def test_audit_paths_verify(n):
    hs = _leaves(n)
    nodes = O.merkle_tree(hs)
    root = nodes[:32]

    def path(i):
        out, lo, hi, p = [], 0, n, 0
        while hi - lo > 1:
            k = 1 << ((hi - lo - 1).bit_length() - 1)
            if i < lo + k:
                out.append(nodes[32 * (p + 2 * k):32 * (p + 2 * k) + 32])
                p, hi = p + 1, lo + k
            else:
                out.append(nodes[32 * (p + 1):32 * (p + 1) + 32])
                p, lo = p + 2 * k, lo + k
        return out[::-1]
    for i in range(n):
        pth = path(i)
        assert O.verify_path(hs[i], i, n, pth, root)
        assert not O.verify_path(hs[(i + 1) % n] if n > 1 else b"\0" * 32, i, n, pth, root)
        for k in range(len(pth)):  # a flipped bit anywhere in the path fails
            bad = list(pth)
            bad[k] = bytes([bad[k][0] ^ 1]) + bad[k][1:]
            assert not O.verify_path(hs[i], i, n, bad, root)
        assert not O.verify_path(hs[i], i, n, pth + [hs[0]], root)
        if n > 1:
            assert not O.verify_path(hs[i], (i + 1) % n, n, pth, root)


# ---- challenges ----------------------------------------------------------------------------

def test_entry_map_exhaustive_grid():
    grid = 1 << 24
    a = np.arange(grid, dtype=np.uint32)
    low = np.random.default_rng(0).integers(0, 256, size=grid, dtype=np.uint32)
    r = O.entries((a << 8) | low)
    ref = (2 * a.astype(np.float64) + 1 - grid) / grid
    assert np.array_equal(r.astype(np.float64), ref)          # exact in fp32
    assert np.array_equal(r[grid - 1 - a.astype(np.int64)], -r)  # symmetric grid
    assert np.array_equal(O.entries(a << 8), r)               # the low byte is discarded


@pytest.mark.parametrize("width", [1, 5, 16, 17, 256, 257, 1000, 4096])
@pytest.mark.parametrize("k", [1, 3, 9])
def test_challenge_matrices_equal_per_vector_xof(width, k):
    h = bytes(range(32))
    ms = [1, 7, 2**32 - 1]
    R = O.challenge_matrices(h, ms, k, width)
    assert R.shape == (3, width, k) and R.dtype == torch.float32
    for i, m in enumerate(ms):
        assert torch.equal(R[i], O.challenge_matrix_xof(h, m, k, width))


def test_challenge_label_layout_and_python_twin():
    assert O.encode_label(0x01020304, 255) == b"\x10\x01\x02\x03\x04\xff"
    h = bytes(range(32))
    xof = blake3_tree.blake3(O.encode_label(9, 3), key=h, length=4 * 300)
    want = O.entries(np.frombuffer(xof, dtype="<u4"))
    got = O.challenge_matrices(h, [9], 3, 300)[0, :, 2].numpy()
    assert np.array_equal(got, want)


def test_challenge_moments():
    r = O.challenge_matrices(bytes(range(32)), [1], 8, 131_072).numpy().astype(np.float64)
    assert abs(r.mean()) < 3e-3 and abs(r.var() - 1 / 3) < 2e-3


# ---- sizing and finishing ------------------------------------------------------------------

def test_e_m_known_answers():
    fp32 = 2.0**-24
    assert O.e_m(64, fp32, fp32) == pytest.approx(5.6e-7, rel=1e-2)
    assert O.e_m(576, fp32, fp32) == pytest.approx(1.51e-6, rel=1e-2)
    assert O.e_m(1536, fp32, fp32) == pytest.approx(2.4e-6, rel=2e-2)
    assert O.e_m(49_152, fp32, fp32) == pytest.approx(1.330e-5, rel=1e-3)


def test_band_unit_branches():
    s = O.SIGMA_R
    assert O.band_unit(100, 2**-24, 2**-24, 0.0, 3.0) == s * 10 * 2**-24 * 3.0
    assert math.isnan(O.band_unit(100, 2**-24, 2**-24, 1.0, float("nan")))
    u = O.band_unit(100, 2**-8, 2**-24, 2.0, 1.0)  # U < ‖P‖: the pre-split unit
    assert u == s * (math.sqrt(2) * 2**-8 + 10 * 2**-24) * 2.0


def test_judge_order_and_nan():
    base = dict(nu=1.0, p_abs1=1.0, p_norm=1.0, u=1.0, unit=1.0, residuals=(0.5, 0.5))
    assert O.judge(base, tau=8, kappa_max=10) == (O.ACCEPT, 0)
    assert O.judge({**base, "residuals": (0.5, 9.0)}, tau=8, kappa_max=10) == (O.RESIDUAL, 2)
    assert O.judge({**base, "nu": 11.0}, tau=8, kappa_max=10) == (O.KAPPA, 0)
    assert O.judge({**base, "u": float("nan")}, tau=8, kappa_max=10) == (O.NONFINITE, 0)
    assert O.judge({**base, "nu": float("inf")}, tau=8, kappa_max=10,
                   guard=False) == (O.ACCEPT, 0)


# ---- Freivalds rows ------------------------------------------------------------------------

def _prod(n, q, w, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(n, q, generator=g).to(dtype).float()
    b = torch.randn(q, w, generator=g).to(dtype).float()
    p = (a @ b).to(dtype).float()
    return a, b, p


def test_forged_entry_stands_out():
    a, b, p = _prod(40, 24, 32, 0)
    r = O.challenge_matrices(bytes(32), [5], 4, 32)[0]
    honest = O.finish_row(O.measure_product_row(a, b, p, r), q=24, n=40, eps_in=2**-24,
                          eps_acc=2**-24)
    p2 = p.clone()
    p2[3, 7] += 1e-2 * p.abs().max()
    forged = O.finish_row(O.measure_product_row(a, b, p2, r), q=24, n=40, eps_in=2**-24,
                          eps_acc=2**-24)
    assert max(forged["normalized"]) > 100 * max(max(honest["normalized"]), 1e-3)


def test_bias_is_a_ones_column():
    a, b, _ = _prod(16, 12, 20, 1)
    bias = torch.randn(20)
    p = a @ b + bias
    r = O.challenge_matrices(bytes(32), [3], 2, 20)[0]
    row = O.measure_product_row(a, b, p, r, bias=bias)
    a1 = torch.cat([a, torch.ones(16, 1)], 1)
    b1 = torch.cat([b, bias[None]], 0)
    ref = O.measure_product_row(a1, b1, p, r)
    assert row[0] == pytest.approx(ref[0], rel=1e-6)  # nu
    f = O.finish_row(row, q=13, n=16, eps_in=2**-24, eps_acc=2**-24, biased=True)
    g = O.finish_row(ref, q=13, n=16, eps_in=2**-24, eps_acc=2**-24)
    assert f["u"] == pytest.approx(g["u"], rel=1e-6)


def test_u_is_the_term_frobenius_norm_and_below_nu():
    a, b, p = _prod(30, 17, 11, 2)
    r = O.challenge_matrices(bytes(32), [1], 1, 11)[0]
    row = O.measure_product_row(a, b, p, r)
    terms = (a[:, :, None] * b[None, :, :]).double()
    assert math.sqrt(row[3]) == pytest.approx(float(terms.square().sum().sqrt()), rel=1e-5)
    assert math.sqrt(row[3]) <= row[0] * (1 + 1e-6)


@pytest.mark.parametrize("row_fn", [O.measure_product_row, O.measure_row_f64])
@pytest.mark.parametrize("n,q,w", [(5, 7, 3), (16, 64, 40), (33, 9, 128)])
def test_all_ones_operands_give_the_closed_forms(row_fn, n, q, w):
    """A = 1[n,q], B = 1[q,w], P = A·B = q·1[n,w]: every row of |A|(|B|1) and of |P|·1 is
    q·w, so ν = ‖|P|·1‖ = √n·q·w; ‖P‖_F = q·√(n·w); U² = Σ A²(B²1) = n·q·w; the residuals
    are 0: exactly in fp64, and within fp32 rounding (below one fp32 band unit) in the fp32
    formulas. The other columns are small integers' sums: exact in both."""
    a, b = torch.ones(n, q), torch.ones(q, w)
    p = torch.full((n, w), float(q))
    r = O.challenge_matrices(bytes(32), [9], 3, w)[0]
    nu, p_abs1, p_norm, u2, bias_sq, *res = row_fn(a, b, p, r)
    assert nu == pytest.approx(math.sqrt(n) * q * w, rel=1e-7)
    assert p_abs1 == pytest.approx(math.sqrt(n) * q * w, rel=1e-7)
    assert p_norm == pytest.approx(q * math.sqrt(n * w), rel=1e-7)
    assert u2 == n * q * w and bias_sq == 0.0
    if row_fn is O.measure_row_f64:
        assert res == [0.0, 0.0, 0.0]
    else:
        unit = O.finish_row([nu, p_abs1, p_norm, u2, bias_sq, *res], q=q, n=n,
                            eps_in=2**-24, eps_acc=2**-24)["unit"]
        assert max(res) <= unit


def test_non_negative_operands_have_no_cancellation():
    """With A, B ≥ 0, |A|(|B|1) = A(B1) = P·1 = |P|·1, so κ = ν/‖|P|·1‖ = 1 to rounding; a
    sign flip in one entry of A lowers ‖|P|·1‖ below ν."""
    g = torch.Generator().manual_seed(4)
    a, b = torch.rand(24, 16, generator=g), torch.rand(16, 30, generator=g)
    p = (a.double() @ b.double()).float()
    r = O.challenge_matrices(bytes(32), [2], 1, 30)[0]
    for row_fn in (O.measure_product_row, O.measure_row_f64):
        mp = O.finish_row(row_fn(a, b, p, r), q=16, n=24, eps_in=2**-24, eps_acc=2**-24)
        assert mp["kappa"] == pytest.approx(1.0, abs=1e-6)
    a2 = a.clone()
    a2[:, 3] = -a2[:, 3]
    p2 = (a2.double() @ b.double()).float()
    mp = O.finish_row(O.measure_row_f64(a2, b, p2, r), q=16, n=24, eps_in=2**-24,
                      eps_acc=2**-24)
    assert mp["kappa"] > 1.0 + 1e-3


def test_planted_residual_is_delta_times_its_challenge_entry():
    """Integer operands make A·(B·r) − P·r exact in fp64, so an honest P has residual 0 and
    P + δ·e_i·e_jᵀ has residual |δ·r[j, col]| in column ``col``: a swapped column or a wrong
    sign fails it."""
    g = torch.Generator().manual_seed(6)
    a = torch.randint(-3, 4, (12, 10), generator=g).float()
    b = torch.randint(-3, 4, (10, 14), generator=g).float()
    p = a @ b
    r = O.challenge_matrices(bytes(range(32)), [11], 4, 14)[0]
    assert O.measure_row_f64(a, b, p, r)[5:] == [0.0] * 4
    p2 = p.clone()
    p2[7, 5] += 0.5
    res = O.measure_row_f64(a, b, p2, r)[5:]
    assert res == [abs(0.5 * float(r[5, col])) for col in range(4)]
    # the fp32 formulas agree to within their own rounding (one fp32 band unit)
    row32 = O.measure_product_row(a, b, p2, r)
    unit = O.finish_row(row32, q=10, n=12, eps_in=2**-24, eps_acc=2**-24)["unit"]
    assert row32[5:] == pytest.approx(res, rel=0, abs=unit)


def test_safe_norm_large_and_zero():
    x = torch.tensor([3e19, -3e19, 1.0])
    assert math.isfinite(float(O.safe_norm(x)))
    assert float(O.safe_norm(x)) == pytest.approx(math.sqrt(2) * 3e19, rel=1e-6)
    assert float(O.safe_norm(torch.zeros(5))) == 0.0
    assert math.isnan(float(O.safe_norm(torch.tensor([1.0, float("nan")]))))


def test_members_equal_single_products():
    a = torch.randn(3, 16, 12)
    b = torch.randn(3, 12, 20)
    p = a @ b
    h = bytes(range(32))
    R = O.challenge_matrices(h, [4, 5, 6], 2, 20)
    rows = O.measure_products_rows(a, b, p, R)
    for i in range(3):
        single = O.measure_product_row(a[i], b[i], p[i], R[i])
        assert rows[i][:3] == pytest.approx(single[:3], rel=1e-4)


def test_f64_yardstick_agrees_with_fp32_formulas():
    a, b, p = _prod(64, 48, 40, 3, torch.bfloat16)
    r = O.challenge_matrices(bytes(32), [2], 3, 40)[0]
    f32 = O.measure_product_row(a, b, p, r)
    f64 = O.measure_row_f64(a, b, p, r)
    assert f32[:4] == pytest.approx(f64[:4], rel=1e-5)


# ---- check 6a: the update identity ---------------------------------------------------------
# Pinned by exact cases (power-of-two entries make every fp32 operation exact, so R, scale and
# ρ have closed forms) and by the outcomes the reference's own tests state
# (tests/verification/verifier/test_update_identity.py).

EPS_W, TAU_W, ETA = 2.0**-24, 4.0, 1e-3


def _honest_update(shape, seed=0, eta=ETA):
    gen = torch.Generator().manual_seed(seed)
    w = torch.randn(shape, generator=gen)
    g = torch.randn(shape, generator=gen)
    return w, torch.add(w, g, alpha=-eta), g  # the optimizer's step


def _ulps(x, i, q):
    x = x.clone()
    for _ in range(q):
        x.view(-1)[i] = torch.nextafter(x.view(-1)[i], torch.tensor(math.inf))
    return x


def test_update_reference_rounding_gives_zero_rho():
    w, _, g = _honest_update((64, 32))
    out = O.update_identity(w, w - ETA * g, [g], ETA, EPS_W, TAU_W)
    assert out["rho_max"] == 0.0 and out["first_nonfinite"] is None and out["first_over"] is None


def test_update_closed_forms():
    # entry 0: R = 2^-20, scale = 2^-24 -> ρ = 16; entry 1: ηG = 1, W − ηG = 0, R = 2^-30,
    # scale = 2^-24·2 -> ρ = 2^-7; entry 2: 0/0 -> 0; entry 3: R > 0 over scale 0 -> inf;
    # entry 4: R = 0 -> 0.
    w = torch.tensor([1.0, 1.0, 0.0, 0.0, 2.0])
    g = torch.tensor([0.0, 1024.0, 0.0, 0.0, 0.0])
    wn = torch.tensor([1.0 + 2.0**-20, 2.0**-30, 0.0, 2.0**-100, 2.0])
    out = O.update_identity(w, wn, [g], 2.0**-10, EPS_W, TAU_W)
    r, s = out["r"].double(), out["scale"].double()
    assert r.tolist() == [2.0**-20, 2.0**-30, 0.0, 2.0**-100, 0.0]
    assert s.tolist() == [2.0**-24, 2.0**-23, 0.0, 0.0, 2.0**-23]
    assert out["rho_max"] == math.inf
    assert out["first_over"] == 0 and out["first_nonfinite"] is None
    out = O.update_identity(w[:2], wn[:2], [g[:2]], 2.0**-10, EPS_W, 100.0)
    assert out["rho_max"] == 16.0 and out["first_over"] is None


def test_update_chain_gradient_adds_in_order():
    # ((1 + 2^-24) + 2^-24) rounds to 1 in fp32; 1 + (2^-24 + 2^-24) would not
    parts = [torch.tensor([1.0]), torch.tensor([2.0**-24]), torch.tensor([2.0**-24])]
    assert O.chain_gradient([p.to(torch.bfloat16) for p in parts]).item() == 1.0
    assert O.chain_gradient([parts[0], parts[1] + parts[2]]).item() == 1.0 + 2.0**-23


def test_update_honest_step_accepts():
    for seed, shape in enumerate([(48, 40), (7, 3, 33), (300,)]):
        w, wn, g = _honest_update(shape, seed)
        out = O.update_identity(w, wn, [g], ETA, EPS_W, TAU_W)
        assert out["first_nonfinite"] is None and out["first_over"] is None
        assert out["rho_max"] <= TAU_W


def test_update_forged_and_tied_entries():
    w, _, g = _honest_update((40, 40), seed=3)
    wn = w - ETA * g
    for i in range(0, w.numel(), 7):
        wn = _ulps(wn, i, 1)
    assert 1.0 < O.update_identity(w, wn, [g], ETA, EPS_W, TAU_W)["rho_max"] <= 2.0
    w, wn, g = _honest_update((50, 30), seed=1)
    out = O.update_identity(w, _ulps(wn, 777, 9), [g], ETA, EPS_W, TAU_W)
    assert out["rho_max"] > TAU_W and out["first_over"] == 777
    # ρ exactly at τ accepts; the next double below rejects
    w, wn, g = _honest_update((20, 20), seed=2)
    forged = _ulps(wn, 5, 5)
    rho = O.update_identity(w, forged, [g], ETA, EPS_W, math.inf)["rho_max"]
    assert O.update_identity(w, forged, [g], ETA, EPS_W, rho)["first_over"] is None
    assert O.update_identity(w, forged, [g], ETA, EPS_W, math.nextafter(rho, 0.0))[
        "first_over"] == 5


@pytest.mark.parametrize("bad", [math.nan, math.inf, -math.inf])
def test_update_non_finite_inputs(bad):
    w, wn, g = _honest_update((30, 30), seed=4)
    g = g.clone()
    g.view(-1)[123] = bad
    assert O.update_identity(w, wn, [g], ETA, EPS_W, TAU_W)["first_nonfinite"] == 123
    w, wn, g = _honest_update((30, 30), seed=5)
    wn = wn.clone()
    wn.view(-1)[17] = math.nan
    out = O.update_identity(w, wn, [g], ETA, EPS_W, TAU_W)
    assert out["first_nonfinite"] == 17 and math.isnan(out["rho_max"])


def test_update_scale_overflow_and_underflowing_ratio():
    # |W_t| + |η·G| overflows while W_t − η·G = 0 and R stay finite
    w, wn, g = _honest_update((10, 10), seed=6, eta=1.0)
    w, wn, g = w.clone(), wn.clone(), g.clone()
    w.view(-1)[9] = g.view(-1)[9] = 3e38
    wn.view(-1)[9] = 0.0
    assert O.update_identity(w, wn, [g], 1.0, EPS_W, TAU_W)["first_nonfinite"] == 9
    # an fp32 quotient that underflows keeps its float64 value; 0/0 entries count as 0
    w, g, wn = torch.zeros(4, 4), torch.zeros(4, 4), torch.zeros(4, 4)
    w.view(-1)[9] = g.view(-1)[9] = 1e38
    wn.view(-1)[9] = 1.4e-45
    out = O.update_identity(w, wn, [g], 1.0, EPS_W, TAU_W)
    assert out["first_over"] is None and 0.0 < out["rho_max"] < 1e-70
