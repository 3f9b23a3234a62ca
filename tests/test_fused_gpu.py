"""P read once: the leaf hasher taking the Freivalds P pass of product leaves
(``pots_leaf_plan_create_fused``), against the unfused plans and the CPU oracle.

Each case is a small transcript of product leaves (2-D tensors, tag 0x03) with their A and B,
hashed and measured twice: by an unfused leaf plan plus an unfused Freivalds plan, and by a
Freivalds plan fused with the leaf plan and run through ``pots_step_run``. The shapes put row
boundaries inside 128-byte pairs and at chunk boundaries, the leaf's first bytes after the
header and its last bytes in the regions no chunk's interior pairs take, and include products
that must not be fused (rows under 1 KiB, a class padding over 1/16, a payload at an offset,
a P shared by two products, k outside 1, 2 and 4).

Tolerances: digests, first-bad and verdict codes bit for bit; the rows' non-negative columns
relative 1e-6 against the unfused plan and 1e-5 against the fp64 oracle; residuals against the
fp64 oracle within 2 band units when honest and relative 1e-4 (floor 2 band units) when a P
entry was changed, as the Freivalds tests do.
"""

from __future__ import annotations

import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
BF16, FP32 = 2.0**-8, 2.0**-24
KEY = bytes(range(32))


def _product(n, q, w, dt, seed, tamper=()):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(n, q, generator=g).to(dt)
    b = (torch.randn(q, w, generator=g) * q ** -0.5).to(dt)
    p = (a.double() @ b.double()).to(dt)
    for i, j, f in tamper:
        p[i, j] = (p[i, j].double() * f).to(dt)
    return a, b, p


def _run_case(lib, prods_cpu, k=4, expect_fused=None, extra_leaves=(), placed=None):
    """prods_cpu: [(a, b, p)] on the CPU. Returns (rows_fused, rows_unfused, digests) after
    checking digests and fusion counts. ``placed(i, p)``: product i's P on the GPU and its
    leaf, a view of the same memory (by default a fresh copy, the leaf P itself)."""
    from verification.commitment import native
    dev, leaves = [], []
    for i, (a, b, p) in enumerate(prods_cpu):
        pd, leaf = (p.cuda(), None) if placed is None else placed(i, p)
        dev.append((a.cuda(), b.cuda(), pd))
        leaves.append(pd if leaf is None else leaf)
    leaves += [t.cuda() for t in extra_leaves]
    hdrs = [O.tensor_leaf_header(O.TAG_PRODUCT, t) for t in leaves]
    kinds = [native.FINITE_KIND[t.dtype] for t in leaves]
    fvp = [native.FvProduct(a, b, p, i + 1) for i, (a, b, p) in enumerate(dev)]
    key = torch.tensor(list(KEY), dtype=torch.uint8, device="cuda")

    fv_u = lib.fv_plan(fvp, k)
    rows_u = fv_u.rows(key)
    leaf_u = lib.leaf_plan(hdrs, leaves, kinds)
    dig_u, bad_u = leaf_u.run()

    fv_f = lib.fv_plan(fvp, k)
    leaf_f = lib.leaf_plan(hdrs, leaves, kinds, fuse=fv_f)
    if expect_fused is not None:
        assert leaf_f.fused == expect_fused
    dig_f = torch.empty_like(dig_u)
    bad_f = torch.empty(1, dtype=torch.int32, device="cuda")
    rows_f = torch.empty_like(rows_u)
    for _ in range(2):  # a second run reuses the records
        lib.step_run(leaf_f, fv_f, key, dig_f, bad_f, rows_f)
    torch.cuda.synchronize()
    assert torch.equal(dig_f, dig_u)
    assert int(bad_f.item()) == int(bad_u.item()) == len(leaves)
    want = [O.tensor_leaf_hash(O.TAG_PRODUCT, t.cpu()) for t in leaves]
    assert [bytes(x) for x in dig_f.cpu().numpy()] == want
    if leaf_f.fused:
        with pytest.raises(ValueError):
            fv_f.rows(key)  # a fused plan runs only beside its leaf plan
    leaf_f.close()
    fv_f.close()
    return rows_f.cpu().tolist(), rows_u.cpu().tolist()


def _check_rows(prods_cpu, rows_f, rows_u, k=4, tampered=()):
    ms = list(range(1, len(prods_cpu) + 1))
    for i, (a, b, p) in enumerate(prods_cpu):
        r = O.challenge_matrices(KEY, [ms[i]], k, p.shape[1])[0]
        ref = O.measure_row_f64(a, b, p, r, None)
        eps_in = BF16 if p.dtype == torch.bfloat16 else FP32
        unit = O.finish_row(ref, q=a.shape[1], n=a.shape[0], eps_in=eps_in,
                            eps_acc=FP32)["unit"]
        for col in range(5):
            assert rows_f[i][col] == pytest.approx(rows_u[i][col], rel=1e-6, abs=1e-300), (i, col)
            assert rows_f[i][col] == pytest.approx(ref[col], rel=1e-5, abs=1e-300), (i, col)
        for x, y in zip(rows_f[i][5:], ref[5:]):
            if i in tampered:
                assert x == pytest.approx(y, rel=1e-4, abs=2 * unit), i
            else:
                assert abs(x - y) <= 2 * unit, (i, x, y, unit)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_fused_rows_equal_unfused_and_oracle(lib, dt):
    esz = 2 if dt == torch.bfloat16 else 4
    shapes = [(64, 96, 1024 // esz),    # 1 KiB rows: one class
              (128, 64, 2560 // esz),   # 2.5 KiB rows: 5 classes, rows end mid-pair
              (256, 80, 4096 // esz),   # 4 KiB rows
              (64, 48, 3072 // esz)]    # 3 KiB rows
    prods = [_product(n, q, w, dt, seed=s) for s, (n, q, w) in enumerate(shapes)]
    rows_f, rows_u = _run_case(lib, prods, expect_fused=len(prods))
    _check_rows(prods, rows_f, rows_u)


@pytest.mark.parametrize("k", [1, 2])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_fused_rows_for_one_and_two_challenges(lib, k, dt):
    """The fused kernel for plans of k = 1 and 2 (R rows of 4 and 8 bytes): rows ending mid-pair
    and on a chunk boundary, many classes, and a changed entry, against the unfused plan and
    the fp64 oracle."""
    esz = 2 if dt == torch.bfloat16 else 4
    shapes = [(64, 96, 1024 // esz), (128, 64, 2560 // esz), (64, 48, 3072 // esz),
              (128, 32, 8960 * 2 // esz)]
    prods = [_product(n, q, w, dt, seed=40 + s) for s, (n, q, w) in enumerate(shapes)]
    n, q, w = shapes[1]
    prods[1] = _product(n, q, w, dt, seed=41, tamper=[(77, w - 1, 3.0)])
    rows_f, rows_u = _run_case(lib, prods, k=k, expect_fused=len(prods))
    _check_rows(prods, rows_f, rows_u, k=k, tampered=(1,))


def test_fused_leaves_of_every_header_length(lib):
    """A product leaf's header is 4(1 + ndim) bytes, so its 128-byte pairs start at columns
    ≡ −2(1 + ndim) (mod 8). The fused kernel reads a leaf whose payload sits 4 bytes past
    (a 16-byte boundary + its header length), so each P is placed at the byte offset that
    makes its leaf, a view with 1, 2, 3 or 4 dims, one the kernel fuses: the pairs' elements
    then start at every even column offset modulo 8. Rows of 516 columns (8,192 of them: 129
    chunk classes, 64 periods, no class padding) put the pairs at offsets that change from
    row to row. Rows end mid-pair, and one entry is changed."""
    shapes = [(128, 40, 1280), (128, 40, 1280), (128, 40, 1280), (128, 40, 1280),
              (8192, 40, 516)]
    prods = [_product(n, q, w, torch.bfloat16, seed=60 + s) for s, (n, q, w) in enumerate(shapes)]
    n, q, w = shapes[2]
    prods[2] = _product(n, q, w, torch.bfloat16, seed=62, tamper=[(33, 700, 3.0)])
    dims = [1, 2, 3, 4, 2]
    bufs = []

    def placed(i, p):
        nd = dims[i]
        off = ((4 * (1 + nd) + 4) % 16) // 2  # elements: payload ≡ header + 4 (mod 16)
        buf = torch.zeros(p.numel() + 8, dtype=p.dtype, device="cuda")
        assert buf.data_ptr() % 16 == 0
        bufs.append(buf)
        pd = buf[off:off + p.numel()].view(p.shape)
        pd.copy_(p)
        leaf = pd.reshape((1,) * (nd - 2) + tuple(p.shape)) if nd >= 2 else pd.view(-1)
        assert leaf.dim() == nd and leaf.data_ptr() == pd.data_ptr()
        return pd, leaf

    rows_f, rows_u = _run_case(lib, prods, expect_fused=len(prods), placed=placed)
    _check_rows(prods, rows_f, rows_u, tampered=(2,))


def test_fused_large_rows_and_many_classes(lib):
    # 17.5 KiB rows (35 classes) and a header-only last chunk
    prods = [_product(128, 64, 8960, torch.bfloat16, seed=7)]
    rows_f, rows_u = _run_case(lib, prods, expect_fused=1)
    _check_rows(prods, rows_f, rows_u)


def test_fused_head_shaped_rows(lib):
    """The tied head's row length: 151,936 bf16 columns, 303,872-byte rows, 1,187 chunk
    classes with no class padding (the C4 logits and dF leaves have it), with changed
    entries on a row end and deep inside a row. At this width two changed entries sit below
    the honest rounding noise, so the rows are compared, not the verdicts."""
    w = 151936
    a, b, p = _product(256, 64, w, torch.bfloat16, seed=31)
    tampered = _product(256, 64, w, torch.bfloat16, seed=32,
                        tamper=[(3, w - 1, 2.0), (200, 77777, -1.0)])
    rows_f, rows_u = _run_case(lib, [(a, b, p), tampered], expect_fused=2)
    _check_rows([(a, b, p), tampered], rows_f, rows_u, tampered=(1,))


def test_fused_changed_entries_in_every_region(lib):
    n, q, w = 128, 64, 1280  # 2560-byte rows
    # row 0's first elements lie before the first 128-byte boundary (12-byte header), the last
    # row's last ones after the last boundary, others at row ends inside pairs and at chunk
    # boundaries
    tamper = [(0, 0, 1.5), (0, 57, -2.0), (n - 1, w - 1, 3.0), (n - 1, w - 5, 0.5),
              (5, w - 1, 1.25), (6, 0, 1.25), (40, 506, -1.0), (77, 640, 2.0)]
    prods = [_product(n, q, w, torch.bfloat16, seed=11, tamper=tamper),
             _product(n, q, w, torch.bfloat16, seed=12, tamper=[(0, 0, 1.0 + 2**-7)]),
             _product(n, q, w, torch.bfloat16, seed=13)]
    rows_f, rows_u = _run_case(lib, prods, expect_fused=3)
    _check_rows(prods, rows_f, rows_u, tampered=(0, 1))
    # eight changed entries stand well above the bf16 rounding of an honest P
    assert max(rows_f[0][5:]) > 2 * max(rows_f[2][5:])


def test_fused_squares_of_tiny_and_huge_entries(lib):
    """Rows whose squares leave fp32's normal range (entries near 1e-22, or 1e25 whose squares
    overflow fp32) are marked by the chunk kernel and their Σx² taken in fp64 from P; the
    norms equal the unfused pass's and the fp64 oracle's."""
    n, q, w = 64, 32, 1024
    base = [_product(n, q, w, torch.bfloat16, seed=s) for s in (21, 22, 23)]
    tiny = (base[0][0], base[0][1], (base[0][2].float() * 1e-22).to(torch.bfloat16))
    huge = (base[1][0], base[1][1], (base[1][2].float() * 1e25).to(torch.bfloat16))
    mixed_p = base[2][2].clone()
    mixed_p[10] = (mixed_p[10].float() * 1e-30).to(torch.bfloat16)  # one row of tiny entries
    mixed = (base[2][0], base[2][1], mixed_p)
    prods = [tiny, huge, mixed]
    rows_f, rows_u = _run_case(lib, prods, expect_fused=3)
    ms = [1, 2, 3]
    for i, (a, b, p) in enumerate(prods):
        r = O.challenge_matrices(KEY, [ms[i]], 4, w)[0]
        ref = O.measure_row_f64(a, b, p, r, None)
        for col in (1, 2):  # ‖|P|1‖ and ‖P‖_F
            assert rows_f[i][col] == pytest.approx(rows_u[i][col], rel=1e-6), (i, col)
            assert rows_f[i][col] == pytest.approx(ref[col], rel=1e-5), (i, col)


def test_products_that_are_not_fused(lib):
    dt = torch.bfloat16
    small = _product(64, 32, 256, dt, seed=1)        # 512-byte rows
    padded = _product(100, 32, 1000, dt, seed=2)     # 125 classes for 196 chunks
    shared = _product(64, 32, 512, dt, seed=3)
    prods = [small, padded, shared, (shared[0], shared[1], shared[2]),
             _product(64, 32, 512, dt, seed=4)]      # only this one qualifies
    from verification.commitment import native
    dev = [(a.cuda(), b.cuda(), p.cuda()) for a, b, p in prods]
    dev[3] = (dev[3][0], dev[3][1], dev[2][2])  # the same P tensor as product 3
    leaves = [dev[0][2], dev[1][2], dev[2][2], dev[4][2]]
    hdrs = [O.tensor_leaf_header(O.TAG_PRODUCT, t) for t in leaves]
    kinds = [native.FINITE_KIND[dt]] * 4
    fvp = [native.FvProduct(a, b, p, i + 1) for i, (a, b, p) in enumerate(dev)]
    key = torch.tensor(list(KEY), dtype=torch.uint8, device="cuda")
    rows_u = lib.fv_plan(fvp, 4).rows(key).cpu().tolist()
    fv_f = lib.fv_plan(fvp, 4)
    leaf_f = lib.leaf_plan(hdrs, leaves, kinds, fuse=fv_f)
    assert leaf_f.fused == 1
    dig = torch.empty(4, 32, dtype=torch.uint8, device="cuda")
    bad = torch.empty(1, dtype=torch.int32, device="cuda")
    rows = torch.empty(5, 9, dtype=torch.float64, device="cuda")
    lib.step_run(leaf_f, fv_f, key, dig, bad, rows)
    rows = rows.cpu().tolist()
    assert [bytes(x) for x in dig.cpu().numpy()] == [
        O.tensor_leaf_hash(O.TAG_PRODUCT, t.cpu()) for t in leaves]
    for i in range(4):  # unfused products: the same kernels, the same bits
        assert rows[i] == rows_u[i]
    assert rows[4][:5] == pytest.approx(rows_u[4][:5], rel=1e-6)
    # k of 3 (R rows of 12 bytes): nothing is fused
    fv3 = lib.fv_plan(fvp, 3)
    assert lib.leaf_plan(hdrs, leaves, kinds, fuse=fv3).fused == 0
    # a plan is fused once
    with pytest.raises(ValueError):
        lib.leaf_plan(hdrs, leaves, kinds, fuse=fv_f)


def test_payload_at_an_offset_is_not_fused(lib):
    from verification.commitment import native
    a, b, p = _product(64, 32, 256, torch.float32, seed=5)
    buf = torch.zeros(p.numel() + 1, dtype=torch.float32, device="cuda")
    buf[1:] = p.reshape(-1).cuda()
    pv = buf[1:].view(64, 256)  # 4 bytes past a 16-byte boundary
    fvp = [native.FvProduct(a.cuda(), b.cuda(), pv, 1)]
    hdr = [O.tensor_leaf_header(O.TAG_PRODUCT, pv)]
    fv = lib.fv_plan(fvp, 4)
    assert lib.leaf_plan(hdr, [pv], [native.FINITE_KIND[torch.float32]], fuse=fv).fused == 0


def test_non_finite_product_leaf_is_still_reported(lib):
    from verification.commitment import native
    prods = [_product(64, 32, 512, torch.bfloat16, seed=s) for s in range(3)]
    dev = [(a.cuda(), b.cuda(), p.cuda()) for a, b, p in prods]
    dev[1][2][30, 100] = float("nan")
    leaves = [p for _, _, p in dev]
    hdrs = [O.tensor_leaf_header(O.TAG_PRODUCT, t) for t in leaves]
    fv = lib.fv_plan([native.FvProduct(a, b, p, i + 1) for i, (a, b, p) in enumerate(dev)], 4)
    leaf = lib.leaf_plan(hdrs, leaves, [native.FINITE_KIND[torch.bfloat16]] * 3, fuse=fv)
    assert leaf.fused == 3
    key = torch.tensor(list(KEY), dtype=torch.uint8, device="cuda")
    dig = torch.empty(3, 32, dtype=torch.uint8, device="cuda")
    bad = torch.empty(1, dtype=torch.int32, device="cuda")
    rows = torch.empty(3, 9, dtype=torch.float64, device="cuda")
    lib.step_run(leaf, fv, key, dig, bad, rows)
    assert int(bad.item()) == 1


def test_device_step_verifier_fused_equals_unfused(lib):
    from verification.computation.instances.decoder import DecoderComputation
    from verification.prover.synthetic import synthetic_step
    from verification.verifier.step import DeviceStepVerifier
    c = DecoderComputation(L=1, d=512, d_f=1024, n_h=4, n_kv=2, n_v=1024, n_s=2, n=256,
                           qkv_bias=True, compute_dtype=torch.bfloat16)
    step = synthetic_step(c, seed=3, operands=True)
    fused = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=4)
    plain = DeviceStepVerifier(c, step.leaves, lambda s: step.operands[s.m], k=4, fuse=False)
    assert fused.fused > 0 and plain.fused == 0
    d, _ = plain.hasher.digests()
    claimed = bytes(lib.merkle_tree_device(d)[0].cpu().numpy())
    for _ in range(2):
        a, b = fused.run(claimed), plain.run(claimed)
        assert a.root == b.root == claimed
        assert (a.first_bad, a.first_fail, a.check) == (b.first_bad, b.first_fail, b.check)
        assert torch.equal(a.codes, b.codes)
        ra, rb = a.rows.cpu(), b.rows.cpu()
        assert torch.allclose(ra[:, :5], rb[:, :5], rtol=1e-6, atol=0)


def test_stages_apart_and_grid_limits_equal_one_call(lib):
    """The fused pair's stages enqueued one at a time (the leaf plan's two chunk kernels and
    the P stage's two parts apart) and row passes limited to a few blocks give the rows and
    digests of pots_step_run bit for bit."""
    from verification.commitment import native
    prods = [_product(128, 64, 1280, torch.bfloat16, seed=31),
             _product(64, 32, 256, torch.bfloat16, seed=32),      # not fused (512-byte rows)
             _product(64, 48, 768, torch.float32, seed=33)]
    dev = [(a.cuda(), b.cuda(), p.cuda()) for a, b, p in prods]
    leaves = [p for _, _, p in dev]
    hdrs = [O.tensor_leaf_header(O.TAG_PRODUCT, t) for t in leaves]
    kinds = [native.FINITE_KIND[t.dtype] for t in leaves]
    fvp = [native.FvProduct(a, b, p, i + 1) for i, (a, b, p) in enumerate(dev)]
    key = torch.tensor(list(KEY), dtype=torch.uint8, device="cuda")

    def fresh():
        fv = lib.fv_plan(fvp, 4)
        leaf = lib.leaf_plan(hdrs, leaves, kinds, fuse=fv)
        assert leaf.fused == 2
        return fv, leaf, (torch.empty(3, 32, dtype=torch.uint8, device="cuda"),
                          torch.empty(1, dtype=torch.int32, device="cuda"),
                          torch.empty(3, 9, dtype=torch.float64, device="cuda"))

    fv, leaf, (dig1, bad1, rows1) = fresh()
    lib.step_run(leaf, fv, key, dig1, bad1, rows1)
    fv2, leaf2, (dig2, bad2, rows2) = fresh()
    for st, n in ((1, 3), (3, 5), (4, 2)):
        fv2.set_grid(st, n)
    LP, FP = native.LeafPlan, native.FvPlan
    fv2.run_stage(0, key, rows2)
    for st in (0, LP.PLAIN_CHUNKS, LP.FUSED_CHUNKS, 2):
        leaf2.run_stage(st, dig2, bad2)
    for st in (1, 2, FP.P_PASS, FP.A_ROWS, FP.TWINS, FP.P_FUSED, 5):
        fv2.run_stage(st, key, rows2)
    torch.cuda.synchronize()
    assert torch.equal(dig1, dig2) and int(bad2.item()) == 3
    assert torch.equal(rows1.view(torch.int64), rows2.view(torch.int64))
    with pytest.raises(ValueError):
        fv2.run_stage(FP.TWINS + 1, key, rows2)
    with pytest.raises(ValueError):
        fv2.set_grid(2, 4)  # only the row passes take a grid limit
    with pytest.raises(ValueError):
        leaf2.run_stage(LP.PLAIN_CHUNKS + 1, dig2, bad2)


def test_fused_stats_count_what_the_kernel_moves(lib):
    """pots_leaf_plan_fused_stats: the fused leaves' message bytes, chunks, and one record per
    (row, chunk) pair whose 128-byte interior windows hold elements of the row."""
    from verification.commitment import native
    n, w = 128, 1280
    a, b, p = (t.cuda() for t in _product(n, 32, w, torch.bfloat16, seed=41))
    fv = lib.fv_plan([native.FvProduct(a, b, p, 1)], 4)
    hdr = O.tensor_leaf_header(O.TAG_PRODUCT, p)
    leaf = lib.leaf_plan([hdr], [p], [native.FINITE_KIND[torch.bfloat16]], fuse=fv)
    H, rb = 1 + len(hdr), 2 * w
    L = H + n * rb
    hc, lf = -(-H // 128) * 128, L // 128 * 128
    records = 0
    for i in range(n):  # chunks each row's interior bytes fall in
        fs, fe = max(H + i * rb, hc), min(H + (i + 1) * rb, lf)
        records += (fe - 1) // 1024 - fs // 1024 + 1
    assert (leaf.fused_bytes, leaf.fused_chunks, leaf.fused_records) == (L, -(-L // 1024),
                                                                         records)
