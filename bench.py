"""Benchmark: one verified step of the hot path on a resident transcript, on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--no-cpu-baseline]

A step is the verifier's whole hot path over one training step's transcript, already in HBM
(check 2 and check 5 of the reference, verification/verifier/checks.py:204-272,576-658):
hash every leaf (BLAKE3 chunks, per-leaf trees, NaN/Inf test fused) and build the Merkle
root; expand the claimed root into every product's challenge matrix; run the three
Freivalds passes over every product's B, A and P; reduce to one fp64 row per product; judge
every product. One host read at the end of the step (root, first non-finite leaf, first
rejected product). Each product's P is a leaf, and the hashing kernel takes the P pass of the
product leaves it streams (pots_leaf_plan_create_fused), so those P are read from HBM once.

Prints one JSON line (the driver's contract): `value` is the step's verified throughput,
(bytes hashed + bytes Freivalds-checked) / step time, in GB/s, every P counted in both (it is
hashed and Freivalds-checked) though the fused kernel reads it once; `parts` splits it by
stage and gives the HBM bytes the step actually reads;
`roofline` is the dominant kernel against MI355X's 8 TB/s; `cpu_baseline` times the CPU
oracle on a bounded sample of the same transcript on the host's cores.

Only one GPU is used; --gpus above 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "pots-2.0_amd", ROOT / "oracle"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBPS = 8000.0
# Whole-GPU 32-bit VALU issue rate: 256 CUs x 4 SIMDs x 16 lanes per clock at the 2.4 GHz peak
# engine clock, in lane operations per second.
VALU_PEAK_OPS = 256 * 4 * 16 * 2.4e9
# VALU instructions per byte of message on the chunk kernels' interior path (two 64-byte blocks
# per 128-byte pair), from a static count of this build's gfx950 assembly: two compressions
# and the NaN/Inf test, 1,438 per pair; with the fused P sums of a k = 4 plan, 1,903 per pair
# of bf16 and 1,704 of fp32 products. Edge blocks and the tree levels are left out.
VALU_OPS_PER_BYTE = {"plain": 1438 / 128, "fused_bf16": 1903 / 128, "fused_fp32": 1704 / 128}
METRIC = "Freivalds-verified GB/s + BLAKE3 Merkle GB/s (% HBM roofline); step verify ms"
CONFIGS = {
    "c1": ("SmolLM2-135M step, 4x256 tokens, fp32, k=1", "smollm2_135m", 1),
    "c3": ("Qwen2-0.5B-shaped step, 8x1024 tokens, bf16, k=2", "qwen2_0_5b_shape", 2),
    "c4": ("Qwen2-1.5B-shaped step, 4x2048 tokens, bf16, k=4", "qwen2_1_5b_shape", 4),
    "c5": ("Qwen2-1.5B-shaped step, 4x2048 tokens, bf16, adversarial: a seeded 1% of the "
           "products perturbed (one entry each, relative size log-uniform in [1e-6, 1]), "
           "re-rooted, k=16", "qwen2_1_5b_shape", 16),
}
# the perturbation of config 5: which products and entries (prover.synthetic.perturb_products)
C5_FRACTION, C5_SEED = 0.01, 5


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cores() -> int:
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()
        if quota != "max":
            n = min(n, max(1, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    return n


def product_inputs(step):
    """(a, b, p, bias fp32 or None, m) of every product, operands as the prover used them."""
    import torch
    c = step.c
    out = []
    for spec in c.products:
        a, b = step.operands[spec.m]
        bias = None
        if spec.bias is not None:
            bias = step.w_t(spec.bias).to(c.operand_dtype).to(torch.float32)
        out.append((a, b, step.product(spec.m), bias, spec.m))
    return out


def cpu_baseline(step, items, fv_budget_s: float = 3.0, runs: int = 3) -> dict:
    """The CPU oracle on a bounded sample of the same transcript, on the host's cores, each
    part timed as the median of ``runs`` runs after a warm-up: leaf hashing with the pthread
    restatement of the reference's native.c over SIMD BLAKE3 (16 chunks per AVX-512
    instruction, as the reference's BLAKE3 library hashes on such a CPU; scalar where AVX-512
    is missing), and the reference's Freivalds formulas (torch-CPU fp32, challenges included)
    on products spread over the inventory."""
    import statistics

    import torch

    import oracle as O
    c = step.c
    threads = cores()
    torch.set_num_threads(threads)
    # hashing sample: product leaves spread over the step, about 4 GB
    simd = O.simd_degree()
    hs, hbytes = [], 0
    prod = list(range(c.n_s + c.n_w, c.n_s + c.n_w + c.M))
    for i in prod[::3]:
        t = step.leaves[i].cpu()
        hs.append((O.tensor_leaf_header(O.TAG_PRODUCT, t), t, O.FINITE_KIND[t.dtype]))
        hbytes += 1 + len(hs[-1][0]) + t.nbytes
        if hbytes > 4e9:
            break
    O.hash_leaves(hs[:4], threads, simd=simd > 1)
    t_hash = []
    for _ in range(runs):
        t0 = time.perf_counter()
        O.hash_leaves(hs, threads, simd=simd > 1)
        t_hash.append(time.perf_counter() - t0)
    # Freivalds sample: every 11th product in canonical order, until about fv_budget_s
    key = bytes(range(32))
    sample, spent = [], 0.0
    for it in items[::11]:
        a, b, p, bias, m = it
        cpu = (a.cpu(), b.cpu(), p.cpu(), None if bias is None else bias.cpu(), m)
        t0 = time.perf_counter()
        r = O.challenge_matrices(key, [m], step.k, cpu[2].shape[1], threads)[0]
        O.measure_product_row(cpu[0], cpu[1], cpu[2], r, cpu[3])
        spent += time.perf_counter() - t0
        sample.append(cpu)
        if spent > fv_budget_s:
            break
    fbytes = sum(x[0].nbytes + x[1].nbytes + x[2].nbytes for x in sample)
    t_fv = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for a, b, p, bias, m in sample:
            r = O.challenge_matrices(key, [m], step.k, p.shape[1], threads)[0]
            O.measure_product_row(a, b, p, r, bias)
        t_fv.append(time.perf_counter() - t0)
    th, tf = statistics.median(t_hash), statistics.median(t_fv)
    value = (hbytes + fbytes) / (th + tf) / 1e9
    return {"value": round(value, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"median of {runs} runs after a warm-up: hashing {len(hs)} product leaves "
                      f"(every 3rd, {hbytes / 1e9:.2f} GB, {hbytes / th / 1e9:.2f} GB/s, "
                      + (f"BLAKE3 with {simd} chunks per AVX-512 instruction"
                         if simd > 1 else "portable scalar BLAKE3")
                      + f" on {threads} pthreads) + Freivalds rows of "
                      f"{len(sample)} products (every 11th, {fbytes / 1e9:.2f} GB, "
                      f"{fbytes / tf / 1e9:.3f} GB/s, torch-CPU fp32 with {threads} threads, "
                      f"challenges included)"}


# The committed counter summaries whose fenced JSON blocks hold each kernel's HBM bytes per
# launch, by configuration (a configuration with none reports traffic as null).
TRAFFIC_FILES = {"c4": ROOT / "profiles" / "c4_kernel_counters.md",
                 "c5": ROOT / "profiles" / "c5_kernel_counters.md"}


def kernel_label(name: str) -> str:
    """A kernel's name as the bench reports it: the chunk kernels by name, a row pass by the
    pass its template arguments make it (``row_pass<XT, WEIGHTED, SQ64, NJG, VS>``: B is
    unweighted, A weighted, P takes its squares in fp64; VS, whether the block shares V, is
    the launch's and not the pass's)."""
    base = name.split("(")[0].replace("void ", "").strip()
    short = base.split("::")[-1]
    if short.startswith("row_pass<"):
        xt, weighted, sq64 = (x.strip().rstrip("u") for x in short[9:-1].split(",")[:3])
        dt = "bf16" if xt == "1" else "fp32"
        if weighted == "true":
            return f"row_pass<{dt}, weighted> (A pass)"
        if sq64 == "true":
            return f"row_pass<{dt}, fp64 squares> (P pass)"
        return f"row_pass<{dt}> (B pass)"
    if short == "twin_pass":
        return "twin_pass (A pass of twins)"
    return short.split("<")[0]  # chunk_kernel_fused<K>: one name for every K


def counter_summary(d: Path, copy_mib: int) -> int:
    """Mean value per dispatch of each counter for each kernel in a rocprofv3 --pmc CSV run;
    for FETCH_SIZE and WRITE_SIZE (KiB) also the bytes per launch, scaled by the same
    counter's reading for the calibration copy (two copies of ``copy_mib`` MiB, each read and
    written once), as JSON lines for the committed profile."""
    import collections
    import csv
    sums: dict = collections.defaultdict(float)
    disp: dict = collections.defaultdict(set)
    for f in d.rglob("*counter_collection.csv"):
        for r in csv.DictReader(f.open()):
            raw = r["Kernel_Name"]
            key = ("copyBuffer" if "copyBuffer" in raw else kernel_label(raw), r["Counter_Name"])
            sums[key] += float(r["Counter_Value"])
            disp[key].add(r["Dispatch_Id"])
    if not sums:
        print(f"no counter_collection.csv under {d}", file=sys.stderr)
        return 1
    print("| kernel | counter | dispatches | mean per dispatch | total |")
    print("|---|---|---|---|---|")
    for (k, cn), v in sorted(sums.items()):
        n = len(disp[(k, cn)])
        print(f"| `{k}` | {cn} | {n} | {v / n:.2f} | {v:.1f} |")
    if copy_mib:
        for cn in sorted({cn for _, cn in sums} & {"FETCH_SIZE", "WRITE_SIZE"}):
            copy_kib = sums.get(("copyBuffer", cn), 0.0)
            if not copy_kib:
                continue
            factor = 2 * copy_mib * 1024 / copy_kib  # true KiB per reported KiB
            print(f"\n{cn}: calibration copy reports {copy_kib:.0f} KiB for "
                  f"{2 * copy_mib * 1024} KiB moved, factor {factor:.3f}")
            for (k, c2), v in sorted(sums.items()):
                if c2 == cn and k != "copyBuffer":
                    n = len(disp[(k, c2)])
                    print(json.dumps({"kernel": k, "counter": cn,
                                      "bytes_per_launch": round(v / n * factor * 1024),
                                      "factor": round(factor, 3)}))
    return 0


def trace_summary(d: Path, steps: int, warmup: int) -> int:
    """Per-kernel dispatch durations of a rocprofv3 --kernel-trace CSV run of this bench, and
    the chunk kernel's launches split by phase: the claimed root and the warm-up steps, the
    timed steps (overlapped with the Freivalds passes), and the serialised stage leg whose
    mean is the roofline's ``launch_ms``."""
    import collections
    import csv
    rows = []
    for f in d.rglob("*kernel_trace.csv"):
        for r in csv.DictReader(f.open()):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                         r["Kernel_Name"].split("(")[0].replace("void ", "")))
    if not rows:
        print(f"no kernel_trace.csv under {d}", file=sys.stderr)
        return 1
    rows.sort()
    by = collections.defaultdict(list)
    for t0, t1, k in rows:
        by[k].append((t1 - t0) / 1e6)
    print("| kernel | calls | mean ms | min ms | max ms |")
    print("|---|---|---|---|---|")
    for k, ds in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        if k.startswith("pots::") or k.startswith("__amd"):
            print(f"| `{k}` | {len(ds)} | {sum(ds) / len(ds):.3f} | {min(ds):.3f} | "
                  f"{max(ds):.3f} |")
    chunk = next((k for k in by if k.startswith("pots::chunk_kernel_fused")),
                 "pots::chunk_kernel")
    # (kernel, launches before the warm-up steps: the claimed root's hashing), then its
    # launches in the warm-up steps, the timed steps and the serialised stage leg
    print()
    for name, n_root, beside in ((chunk, 1, "the Freivalds passes"),
                                 ("pots::row_pass<1u, true, false, 1u, false>", 0,
                                  "the chunk kernels")):
        ck = by.get(name, [])
        n_pre = n_root + warmup
        n_leg = max(3, min(steps, 5))  # the stage leg's runs, as main() makes them
        timed, leg = ck[n_pre:n_pre + steps], ck[n_pre + steps:n_pre + steps + n_leg]
        if timed and leg:
            print(f"{name[6:]}: {len(timed)} launches in the timed steps, mean "
                  f"{sum(timed) / len(timed):.3f} ms (beside {beside}); {len(leg)} launches "
                  f"in the serialised stage leg, mean {sum(leg) / len(leg):.3f} ms")
    return 0


def traffic_from_profile(kernel: str, config: str) -> int | None:
    """HBM bytes per launch of ``kernel`` (read + written) in configuration ``config`` from its
    committed counter summary (the fenced JSON block of TRAFFIC_FILES[config], one object per
    kernel and counter), or None when there is none or it holds no figure for that kernel."""
    if config not in TRAFFIC_FILES:
        return None
    try:
        text = TRAFFIC_FILES[config].read_text()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        rows = [json.loads(line) for line in block.splitlines() if line.strip()]
    except (OSError, IndexError, ValueError):
        return None
    got = {r["counter"]: int(r["bytes_per_launch"]) for r in rows if r.get("kernel") == kernel}
    if {"FETCH_SIZE", "WRITE_SIZE"} <= set(got):
        return got["FETCH_SIZE"] + got["WRITE_SIZE"]
    return None


def disk_leg(root: Path, c, step, k: int, claimed: bytes, v) -> dict:
    """The stored-step path: write the transcript as the on-disk store does (one torch.save
    file per leaf, meta.json, leaf_hashes.bin; plus the captured operands), then bring it back
    into HBM twice with the native loader (pread into pinned staging, DMA into one arena), and
    once with the reference's reader (torch.load of each leaf, then a copy to the GPU); verify
    the loaded copy with the device step verifier. The files were just written, so the reads
    come from the host's page cache: this measures the loader, not a disk."""
    import shutil

    import torch

    from verification.commitment import native
    from verification.commitment.merkle import MerkleTree
    from verification.transcript.loader import StepLoader, write_operands
    from verification.transcript.store import DiskStore
    from verification.verifier.step import DeviceStepVerifier

    d = root / "step"
    nodes = native.get().merkle_tree_device(v.digests)
    tree = MerkleTree.from_nodes(nodes.cpu().numpy().tobytes(), c.n_leaves)
    t0 = time.perf_counter()
    disk = DiskStore.write(d, c, step.leaves, tree)
    write_operands(d, step.operands)
    write_s = time.perf_counter() - t0
    files = sum(1 for _ in d.rglob("*.pt"))
    log(f"[bench] disk leg: {files} files written under {d} in {write_s:.1f} s")
    loader = StepLoader(threads=8, staging_mib=256)
    ms = [s.m for s in c.products]
    loads = []
    res = None
    try:
        for _ in range(2):
            res = None
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            res = loader.load(disk, c.n_leaves, ms)
            loads.append((time.perf_counter() - t0, dict(res.times)))
        best_s, times = min(loads, key=lambda x: x[0])
        moved, fallback = res.bytes, res.fallback
        log(f"[bench] disk leg: {moved / 1e9:.2f} GB in {best_s:.2f} s "
            f"({moved / best_s / 1e9:.1f} GB/s); " +
            ", ".join(f"{key} {t:.2f} s" for key, t in times.items()))
        out = DeviceStepVerifier(c, res.leaves, lambda s: res.operands[s.m], k=k).run(disk.root)
        assert out.root == claimed and out.check is None, out.detail
        # the reference's reader over the same leaves: torch.load, then a copy to the GPU
        dev = torch.device("cuda", torch.cuda.current_device())
        t0 = time.perf_counter()
        n_ref = 0
        for i in range(c.n_leaves):
            obj = disk.leaf(i)
            if isinstance(obj, torch.Tensor):
                obj.to(dev)
                n_ref += obj.nbytes
        torch.cuda.synchronize()
        ref_s = time.perf_counter() - t0
        log(f"[bench] disk leg: the reference's reader took {ref_s:.2f} s for the leaves "
            f"({n_ref / ref_s / 1e9:.2f} GB/s)")
    finally:
        res = None
        shutil.rmtree(d, ignore_errors=True)
    return {"files": files, "fallback_files": fallback, "bytes": moved,
            "write_s": round(write_s, 2),
            "load_s": [round(x[0], 3) for x in loads],
            "load_parts_s": {key: round(t, 3) for key, t in times.items()},
            "gbps": round(moved / best_s / 1e9, 2),
            "native_copy_gbps": round(moved / times["load"] / 1e9, 2),
            "threads": loader.threads, "staging_mib": 256,
            "reference_reader_s": round(ref_s, 3),
            "reference_reader_gbps": round(n_ref / ref_s / 1e9, 2),
            "verified": True, "source": "page cache (files written just before)"}


def prover_leg(widths=(4096, 8192, 8192, 4096), n_s: int = 2048, k: int = 2) -> dict:
    """The device-resident prover on an MLP step: the training pass with and without the
    capture, the labeling and SGD step, the commit of every leaf in HBM (the reference copies
    each product to the host as it is produced and hashes there: the bytes it would move are
    timed as a device-to-host copy into pinned memory), and the verify step with every operand
    rebuilt from the committed leaves by the replay."""
    import torch

    from verification.computation.instances.mlp import (MLPComputation, MLPReplay,
                                                        init_weights, synthetic_dataset)
    from verification.prover.step import commit, prove_step
    from verification.verifier.step import DeviceStepVerifier

    c = MLPComputation(widths, n_s=n_s, eta=1e-3)
    with torch.device("cuda"):
        model = c.build_model()
    w0 = init_weights(widths, 0, "cuda")
    records = synthetic_dataset(widths, n_s, 7)

    def timed(fn, reps=3):
        best, out = math.inf, None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = fn()
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
        return best * 1e3, out

    def plain():
        from verification.computation.interface import load_weights
        load_weights(c, model, w0)
        model.zero_grad(set_to_none=True)
        c.loss(model, records).backward()

    plain_ms, _ = timed(plain)
    prove_ms, step = timed(lambda: prove_step(c, model, w0, records))
    commit_ms, tree = timed(lambda: commit(c, step))
    leaves = step.leaves()
    leaf_bytes = sum(x.nbytes for x in leaves)
    moved = [*step.products, *step.w_next.values()]
    host = [torch.empty(x.shape, dtype=x.dtype, pin_memory=True) for x in moved]

    def offload():
        for h, x in zip(host, moved):
            h.copy_(x, non_blocking=True)

    d2h_ms, _ = timed(offload)
    d2h_bytes = sum(x.nbytes for x in moved)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    replay = MLPReplay(c, leaves)
    v = DeviceStepVerifier(c, leaves, lambda s: replay.operands(s.m), k=k)
    torch.cuda.synchronize()
    setup_ms = (time.perf_counter() - t0) * 1e3
    verify_ms, verdict = timed(lambda: v.run(tree.root))
    assert verdict.check is None and verdict.root == tree.root, verdict.detail
    log(f"[bench] prover leg: MLP {widths} x {n_s}: training pass {plain_ms:.1f} ms, under "
        f"capture with labeling and SGD {prove_ms:.1f} ms; commit of {leaf_bytes / 1e9:.2f} GB "
        f"in HBM {commit_ms:.2f} ms; the host copy it avoids: {d2h_bytes / 1e9:.2f} GB in "
        f"{d2h_ms:.1f} ms; replay and plans {setup_ms:.1f} ms, verify {verify_ms:.1f} ms")
    return {"model": f"MLP widths {list(widths)}, {n_s} records, fp32", "k": k,
            "products": c.M, "leaf_bytes": leaf_bytes,
            "training_pass_ms": round(plain_ms, 2), "prove_step_ms": round(prove_ms, 2),
            "commit_ms": round(commit_ms, 3),
            "commit_gbps": round(leaf_bytes / (commit_ms * 1e-3) / 1e9, 1),
            "avoided_d2h_bytes": d2h_bytes, "avoided_d2h_ms": round(d2h_ms, 2),
            "replay_and_plans_ms": round(setup_ms, 2), "verify_ms": round(verify_ms, 2),
            "verified": True}


def capture_leg_qwen2(batch: int = 4, seq: int = 2048, layers: int = 28, k: int = 4) -> dict:
    """A real training step of a Qwen2-1.5B-shaped model, proved, committed and verified on
    the GPU: transformers' Qwen2ForCausalLM at C4's shapes (all 28 decoder layers, random
    init, bf16 under autocast over fp32 masters, the build's attention core) runs under the
    device-resident capture; the products are labeled into the declared computation's
    canonical slots, SGD steps the weights, every leaf is hashed in HBM, and the device step
    verifier checks the step with the captured operands; then ``Verifier.verify_step`` checks
    it again from the committed leaves alone (the decoder replay). The reference copies each
    product to pinned host memory as it is made (``_offload``) and hashes on the host; that
    copy is timed on a sample."""
    import torch

    from setup.records import Record
    from verification.computation.instances.decoder import DecoderComputation
    from verification.computation.interface import snapshot_weights
    from verification.prover.step import commit, prove_step
    from verification.verifier.step import DeviceStepVerifier

    c = DecoderComputation(L=layers, d=1536, d_f=8960, n_h=12, n_kv=2, n_v=151936, n_s=batch,
                           n=seq, d_h=128, tied=True, qkv_bias=True,
                           compute_dtype=torch.bfloat16)
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = c.build_model()
    w0 = snapshot_weights(c, model)
    g = torch.Generator().manual_seed(1)
    records = []
    for _ in range(batch):
        ids = torch.randint(0, c.n_v, (seq,), generator=g, dtype=torch.int32)
        records.append(Record(ids, torch.roll(ids, -1), torch.ones(seq, dtype=torch.int32)))

    def plain():
        from verification.computation.interface import load_weights
        load_weights(c, model, w0)
        model.zero_grad(set_to_none=True)
        c.loss(model, records).backward()

    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        plain()
        torch.cuda.synchronize()
        plain_ms = (time.perf_counter() - t0) * 1e3
    model.zero_grad(set_to_none=True)
    t0 = time.perf_counter()
    step = prove_step(c, model, w0, records, keep_operands=True)
    torch.cuda.synchronize()
    prove_ms = (time.perf_counter() - t0) * 1e3
    t0 = time.perf_counter()
    tree = commit(c, step)
    torch.cuda.synchronize()
    commit_ms = (time.perf_counter() - t0) * 1e3
    leaves = step.leaves()
    leaf_bytes = sum(x.nbytes for x in leaves[c.n_s:])
    product_bytes = sum(p.nbytes for p in step.products)
    t0 = time.perf_counter()
    v = DeviceStepVerifier(c, leaves, lambda s: step.operands[s.m], k=k)
    torch.cuda.synchronize()
    setup_ms = (time.perf_counter() - t0) * 1e3
    verdict = v.run(tree.root)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    verdict = v.run(tree.root)
    torch.cuda.synchronize()
    verify_ms = (time.perf_counter() - t0) * 1e3
    assert verdict.check is None and verdict.root == tree.root, verdict.detail
    # What the check-level leg does not read goes before it: the device verifier's plans,
    # the prover's kept operands and model (the replay builds its own).
    v.close()
    del v, verdict, model
    step.operands.clear()
    import gc
    gc.collect()
    torch.cuda.empty_cache()
    # The reference-shaped path on the same step: Verifier.verify_step in the reference's
    # order, every operand and check 6b's glue gradients from the decoder replay of the
    # committed leaves; the first run builds the plans, the second finds them cached.
    from verification.commitment.leaves import leaf_hashes_of
    from verification.commitment.merkle import merkle_root
    from verification.transcript.store import InMemoryStore
    from verification.verifier.bands import Bands
    from verification.verifier.driver import Verifier
    recs = [leaves[c.record_index(i)] for i in range(c.n_s)]
    h_d = merkle_root(leaf_hashes_of(c, ((0, r) for r in recs)))
    cl_ms, cl_slots, cache = [], [], None
    for _ in range(2):
        cv = Verifier(c, h_D=h_d, n_records=c.n_s, k=k, n_steps=1, bands=Bands.provisional(),
                      seed=0, w0={n: leaves[c.w_t_index(n)] for n in c.weight_names},
                      schedule=lambda t: list(range(c.n_s)), allow_provisional=True)
        if cache is not None:
            cv.plans = cache
        assert cv.start_run(recs) is None
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rej = cv.verify_step(1, InMemoryStore(leaves, tree))
        cl_ms.append((time.perf_counter() - t0) * 1e3)
        cl_slots.append({s_: round(t_ * 1e3, 2) for s_, t_ in cv.timings[1].items()})
        assert rej is None, rej
        cache = cv.plans
    overlapped = cv.overlapped == [1]
    declined = cache.overlap.declined if cache.overlap is not None else None
    cache.close()
    log(f"[bench] qwen2 check-level Verifier.verify_step (decoder replay, check 6b on "
        f"{len(c.glue_gradient_weights)} glue weights; "
        f"{'overlapped' if overlapped else f'serial: {declined}'}): {cl_ms[0]:.0f} ms "
        f"building its plans, {cl_ms[1]:.0f} ms with them cached; " +
        ", ".join(f"{s_} {t_:.1f}" for s_, t_ in cl_slots[1].items()))
    # the reference's per-product copy to pinned host memory, on every 8th product
    sample = list(step.products[::8])
    host = [torch.empty(p.shape, dtype=p.dtype, pin_memory=True) for p in sample]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for h, p in zip(host, sample):
        h.copy_(p, non_blocking=True)
    torch.cuda.synchronize()
    d2h_gbps = sum(p.nbytes for p in sample) / (time.perf_counter() - t0) / 1e9
    summary = step.capture
    log(f"[bench] qwen2 prover leg: training step {plain_ms:.0f} ms, proved (capture, "
        f"labeling, SGD) {prove_ms:.0f} ms; {c.M} products ({summary['calls']} calls), "
        f"{product_bytes / 1e9:.2f} GB in HBM; commit of {leaf_bytes / 1e9:.2f} GB "
        f"{commit_ms:.0f} ms (root {tree.root.hex()[:16]}…); verifier plans {setup_ms:.0f} ms, "
        f"verify {verify_ms:.1f} ms (accepted); the host copy it avoids runs at "
        f"{d2h_gbps:.1f} GB/s ({product_bytes / d2h_gbps / 1e9:.2f} s for the products)")
    return {"model": f"Qwen2-1.5B-shaped, {layers} of 28 layers (transformers "
                     f"Qwen2ForCausalLM, random init, bf16 autocast over fp32 masters), "
                     f"{batch}x{seq} tokens",
            "k": k, "products": c.M, "calls": summary["calls"],
            "product_bytes": product_bytes, "leaf_bytes": leaf_bytes,
            "training_step_ms": round(plain_ms, 1), "prove_step_ms": round(prove_ms, 1),
            "commit_ms": round(commit_ms, 1), "verifier_setup_ms": round(setup_ms, 1),
            "verify_ms": round(verify_ms, 2), "verified": True,
            "check_level": {"verify_step_first_ms": round(cl_ms[0], 1),
                            "verify_step_ms": round(cl_ms[1], 1), "slots_ms": cl_slots[1],
                            "overlapped": overlapped, "declined": declined,
                            "glue_weights": len(c.glue_gradient_weights)},
            "avoided_d2h_gbps": round(d2h_gbps, 1),
            "avoided_d2h_s": round(product_bytes / d2h_gbps / 1e9, 3)}


def check_level_leg(c, step, k: int, claimed: bytes, runs: int = 4) -> dict:
    """``Verifier.verify_step`` on the resident transcript, as a caller of the reference's
    driver runs it: checks 7, 2, 6a, 5, 6b and 2.root, host judging included (operands from
    the synthetic capture, so trusted; 6b needs the replay's glue and is not run). The first
    run builds the verifier's plans (a run's first step); the later ones find them in the plan
    cache, as every later step of a run whose transcript keeps its layout does."""
    import torch

    from verification.commitment.leaves import leaf_hashes_of
    from verification.commitment.merkle import merkle_root
    from verification.transcript.store import InMemoryStore
    from verification.verifier.bands import Bands
    from verification.verifier.driver import Verifier
    c.use_operands(step.replay())
    records = [step.leaves[c.record_index(i)] for i in range(c.n_s)]
    h_d = merkle_root(leaf_hashes_of(c, ((0, r) for r in records)))
    times, slots = [], []
    cache = None
    for _ in range(runs):
        v = Verifier(c, h_D=h_d, n_records=c.n_s, k=k, n_steps=1, bands=Bands.provisional(),
                     seed=0, w0={n: step.leaves[c.w_t_index(n)] for n in c.weight_names},
                     schedule=lambda t: list(range(c.n_s)), allow_provisional=True,
                     trust_prover_operands=True)
        if cache is not None:
            v.plans = cache
        assert v.start_run(records) is None
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rej = v.verify_step(1, InMemoryStore(step.leaves, claimed_root=claimed))
        times.append((time.perf_counter() - t0) * 1e3)
        slots.append(v.timings[1])
        assert rej is None, rej
        cache = v.plans
    ov = cache.overlap
    hits, builds = (ov.hits, ov.builds) if ov is not None else (cache.hits, cache.builds)
    overlapped = len(v.overlapped) == 1
    declined = ov.declined if ov is not None else None
    grid_ms = ov.entry.grid_times if ov is not None and ov.entry is not None else {}
    cache.close()
    best = min(range(1, runs), key=lambda i: times[i])
    c.use_operands(None)
    log(f"[bench] check-level Verifier.verify_step ({'overlapped' if overlapped else 'serial'}"
        f" path): {times[0]:.1f} ms building its plans, {times[best]:.1f} ms with them cached "
        f"(best of {runs - 1}; {builds} built, {hits} reused); "
        + ", ".join(f"{s} {t * 1e3:.1f}" for s, t in slots[best].items()))
    return {"verify_step_ms": round(times[best], 1), "overlapped": overlapped,
            "declined": declined,
            "a_pass_grid_ms": {str(g): round(t, 2) for g, t in grid_ms.items()},
            "verify_step_first_ms": round(times[0], 1),
            "slots_ms": {s: round(t * 1e3, 2) for s, t in slots[best].items()},
            "first_slots_ms": {s: round(t * 1e3, 2) for s, t in slots[0].items()},
            "runs_ms": [round(t, 1) for t in times]}


def measure_step(c, step, k: int, args, desc: str, config: str):
    """The headline measurement of one configuration on its resident transcript: the plans,
    the claimed root (the root of the transcript as it is), the timed overlapped steps, the
    serialised stage leg, check 6a, and every kernel's roofline; returns the JSON line's dict
    (without the legs), the step verifier, the claimed root and the product inputs."""
    import torch

    from verification.commitment import native
    from verification.verifier.step import DeviceStepVerifier

    lib = native.get()
    stream = torch.cuda.current_stream()
    items = product_inputs(step)
    t0 = time.perf_counter()
    v = DeviceStepVerifier(c, step.leaves, lambda spec: step.operands[spec.m], k=k,
                           a_grid=args.a_grid, b_grid=args.b_grid,
                           hash_after_b=not args.hash_first, plain_early=args.plain_early)
    torch.cuda.synchronize()
    plan_build_ms = (time.perf_counter() - t0) * 1e3
    log(f"[bench] plans built in {plan_build_ms:.1f} ms (leaf plan "
        f"{'fused with' if v.fused else 'beside'} the Freivalds plan, verdict table; A-stage "
        f"grid {v.a_grid})")
    # The claimed root: the honest root of this transcript, as the prover would send it.
    v.hasher.digests(v.digests, v.bad, stream)
    claimed = lib.merkle_tree_device(v.digests, stream)[0].clone()
    torch.cuda.synchronize()
    claimed_b = bytes(claimed.cpu().numpy())
    hash_bytes, fv_bytes = v.hash_bytes, v.freivalds_bytes
    log(f"[bench] claimed root {claimed_b.hex()[:16]}…; hash {hash_bytes / 1e9:.2f} GB, "
        f"Freivalds {fv_bytes / 1e9:.2f} GB")

    def one_step(events=None):
        nodes, codes, first = v.enqueue(claimed, events)
        flags = torch.cat([nodes[0].view(torch.int32), v.bad, first])
        return flags.cpu(), codes

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    evs: list = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        flags, codes = one_step(evs)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = wall / args.steps * 1e3
    hashed_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    measured_ms = sum(e[0].elapsed_time(e[2]) for e in evs) / args.steps
    # the chunk kernel inside the timed steps, on its own (side) stream, beside the Freivalds
    chunks_in_step_ms = sum(e[4].elapsed_time(e[5]) for e in evs) / args.steps
    # the A pass inside the timed steps, beside the chunk kernels
    a_in_step_ms = sum(e[6].elapsed_time(e[7]) for e in evs) / args.steps
    root = flags[:8].numpy().tobytes()
    first_bad, first_fail = int(flags[8]), int(flags[9])
    assert root == claimed_b, "recomputed root differs from the claim"
    assert first_bad == c.n_leaves, "a synthetic leaf was reported non-finite"
    n_rej = int((codes[:, 0] != 0).sum())
    log(f"[bench] step {ms:.2f} ms (streams overlapped: hashing done at {hashed_ms:.2f} ms, "
        f"Freivalds rows at {measured_ms:.2f} ms); {n_rej} rejected (first {first_fail})")

    # Stage leg: the same work serialised on one stream, every stage bracketed by events on
    # that stream, for the per-kernel figures and the roofline.
    # (The challenges come first: a fused chunk kernel reads them.)
    # The chunk stage's two kernels are timed apart: the fused leaves' and the others'.
    fv_stages = native.FvPlan.STAGES
    leaf_stages = [(0, "hash.stage"), (native.LeafPlan.FUSED_CHUNKS, "hash.chunks_fused"),
                   (native.LeafPlan.PLAIN_CHUNKS, "hash.chunks"), (2, "hash.levels")]
    # the Freivalds stages after the challenges; the A pass as its two kernels
    fv_parts = [(1, "freivalds.b_pass"), (2, "freivalds.reduce"),
                (native.FvPlan.A_ROWS, "freivalds.a_pass"),
                (native.FvPlan.TWINS, "freivalds.twin_pass"), (4, "freivalds.p_pass"),
                (5, "freivalds.rows")]
    names = ([f"freivalds.{fv_stages[0]}"] + [nm for _, nm in leaf_stages] +
             ["tree"] + [nm for _, nm in fv_parts] + ["verdicts"])

    def staged(ev):
        i = 0
        ev[i].record(stream)
        v.key.copy_(claimed)
        v.plan.run_stage(0, v.key, v.rows, stream)
        i += 1
        ev[i].record(stream)
        for st, _ in leaf_stages:
            v.hasher.plan.run_stage(st, v.digests, v.bad, stream)
            i += 1
            ev[i].record(stream)
        lib.merkle_tree_device(v.digests, stream)
        i += 1
        ev[i].record(stream)
        for st, _ in fv_parts:
            v.plan.run_stage(st, v.key, v.rows, stream)
            i += 1
            ev[i].record(stream)
        lib.verdicts(v.rows, v.specs, k=k, eps_in=v.eps_in, eps_acc=v.eps_acc, tau=v.bands.tau,
                     stream=stream)
        i += 1
        ev[i].record(stream)

    n_stage_runs = max(3, min(args.steps, 5))
    sev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
           for _ in range(n_stage_runs)]
    for ev in sev:
        staged(ev)
    torch.cuda.synchronize()
    stage_ms = {nm: sum(ev[i].elapsed_time(ev[i + 1]) for ev in sev) / n_stage_runs
                for i, nm in enumerate(names)}
    serial_ms = sum(stage_ms.values())
    log("[bench] serialised stages (ms): " +
        ", ".join(f"{nm} {t:.3f}" for nm, t in stage_ms.items()) + f"; total {serial_ms:.2f}")

    # Check 6a (the update identity of every linear weight) beside the headline step: it is
    # part of the reference's verify_step but not of the metric's bytes, so it is timed on its
    # own and reported in parts.
    check_6a = None
    if c.linear_weights:
        uw = [native.UpdateWeight(step.leaves[c.w_t_index(nm)], step.leaves[c.w_next_index(nm)],
                                  [step.leaves[c.product_index(m)] for m in ms], 4.0)
              for nm, ms in c.linear_weights.items()]
        uplan = lib.update_plan(uw, c.eta, 2.0**-24)
        uout = uplan.run(stream=stream)
        torch.cuda.synchronize()
        n_over = sum(r[2] is not None or r[1] is not None for r in native.UpdatePlan.decode(uout))
        ue = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ue[0].record(stream)
        for _ in range(n_stage_runs):
            uplan.run(uout, stream)
        ue[1].record(stream)
        torch.cuda.synchronize()
        u_ms = ue[0].elapsed_time(ue[1]) / n_stage_runs
        check_6a = {"ms": round(u_ms, 4), "bytes": uplan.bytes,
                    "gbps": round(uplan.bytes / (u_ms * 1e-3) / 1e9, 1),
                    "weights": len(uw), "rejected": n_over}
        log(f"[bench] check 6a: {len(uw)} linear weights, {uplan.bytes / 1e9:.2f} GB in "
            f"{u_ms:.3f} ms ({check_6a['gbps']:.0f} GB/s), {n_over} rejected")
        uplan.close()

    # Algorithmic bytes of each single-kernel stage, per the survey's measurement plan: the
    # message bytes (1 + header + payload) of the leaves a chunk kernel hashes, or the operand
    # a row pass reads (A, B, or the P of the products the chunk kernel did not take), each
    # element once. Writes (chaining values, run records, partial sums) are not counted.
    a_bytes = sum(a.nbytes for a, _, _, _, _ in items)
    b_bytes = sum(b.nbytes for _, b, _, _, _ in items)
    p_bytes = sum(p.nbytes for _, _, p, _, _ in items)
    # Twins: products whose A is another product's A transposed (the same tensor); the twin
    # pass reads that operand once for both, the row pass the A's of the other products.
    mates = native._twin_mates([native.FvProduct(a, b, p, m) for a, b, p, _, m in items], k)
    twin_x_bytes = sum(items[j][0].nbytes for j in mates.values())
    twinned = set(mates) | set(mates.values())
    a_row_bytes = sum(items[i][0].nbytes for i in range(len(items)) if i not in twinned)
    assert v.plan.twins == len(mates), (v.plan.twins, len(mates))
    hp = v.hasher.plan
    fused_p_bytes = hp.fused_bytes - 12 * v.fused  # payload: 0x00 || 11-byte 2-D header off
    kernels = {
        "hash.chunks": ("chunk_kernel", hash_bytes - hp.fused_bytes),
        "freivalds.a_pass": ("row_pass<bf16, weighted> (A pass)", a_row_bytes),
        "freivalds.b_pass": ("row_pass<bf16> (B pass)", b_bytes),
    }
    if twin_x_bytes:
        kernels["freivalds.twin_pass"] = ("twin_pass (A pass of twins)", twin_x_bytes)
    if v.fused:
        kernels["hash.chunks_fused"] = ("chunk_kernel_fused", hp.fused_bytes)
    if p_bytes - fused_p_bytes > 0:
        kernels["freivalds.p_pass"] = ("row_pass<bf16, fp64 squares> (P pass)",
                                       p_bytes - fused_p_bytes)
    dom = max(kernels, key=lambda nm: stage_ms[nm])
    # The chunk kernels are bound by 32-bit VALU issue, not HBM: their fraction of it.
    fused_key = "fused_bf16" if c.product_dtype == torch.bfloat16 else "fused_fp32"
    valu = {}
    # (the fused kernel's count is its k = 4 instantiation's; other k leave it out)
    for nm, (kname, nbytes), per in (
            ("hash.chunks", kernels["hash.chunks"], VALU_OPS_PER_BYTE["plain"]),
            ("hash.chunks_fused", kernels.get("hash.chunks_fused", ("", 0)) if k == 4
             else ("", 0), VALU_OPS_PER_BYTE[fused_key])):
        if nbytes and stage_ms[nm] > 0:
            ops = per * nbytes
            valu[kname] = {"ops_per_byte": round(per, 2), "ops": int(ops),
                           "achieved_tops": round(ops / (stage_ms[nm] * 1e-3) / 1e12, 2),
                           "peak_tops": round(VALU_PEAK_OPS / 1e12, 2),
                           "frac": round(ops / (stage_ms[nm] * 1e-3) / VALU_PEAK_OPS, 4)}
    # the kernels the step's events bracket
    in_step = {"hash.chunks_fused" if v.fused else "hash.chunks": chunks_in_step_ms}
    if not mates:  # else the step's A-pass events bracket the row pass and the twin pass
        in_step["freivalds.a_pass"] = a_in_step_ms
    dom_name, dom_bytes = kernels[dom]
    achieved = dom_bytes / (stage_ms[dom] * 1e-3) / 1e9

    def kernel_roofline(nm: str) -> dict:
        kname, nbytes = kernels[nm]
        gbps = nbytes / (stage_ms[nm] * 1e-3) / 1e9
        out = {"bound": "valu" if nm.startswith("hash.") else "hbm",
               "achieved": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
               "algorithmic_bytes": nbytes, "launch_ms": round(stage_ms[nm], 4),
               "launch_ms_in_step": (round(in_step[nm], 4) if nm in in_step else None),
               "traffic": traffic_from_profile(kname, config)}
        if kname in valu:
            out["valu_frac"] = valu[kname]["frac"]
        return out
    hash_ms = sum(stage_ms[nm] for _, nm in leaf_stages)
    fv_ms = stage_ms[f"freivalds.{fv_stages[0]}"] + sum(stage_ms[nm] for _, nm in fv_parts)
    total = hash_bytes + fv_bytes
    value = total / (ms * 1e-3) / 1e9
    # P of a fused product is read once, by the hashing kernel (its leaf message is the
    # 12-byte 0x00 || header of a 2-D tensor, then P)
    # and a twin's shared A once, by the twin pass
    read_bytes = hash_bytes + a_row_bytes + twin_x_bytes + b_bytes + p_bytes - fused_p_bytes
    # the bytes the Freivalds stages read themselves: A, B, and the P the hash did not take
    fv_read_bytes = a_row_bytes + twin_x_bytes + b_bytes + p_bytes - fused_p_bytes
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u32 (BLAKE3) + bf16 operands with fp32 accumulation (Freivalds)",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: {desc}; whole verify step (check 2 hashing + "
                               "Merkle root, check 5 challenges + Freivalds + verdicts) on a "
                               "transcript resident in HBM",
                   "leaves": c.n_leaves, "products": c.M, "k": k,
                   "hash_bytes": hash_bytes, "freivalds_bytes": fv_bytes,
                   "p_pass_fused_products": v.fused,
                   "p_pass_fused_leaf_bytes": v.hasher.plan.fused_bytes,
                   "p_pass_fused_records": v.hasher.plan.fused_records,
                   "twins": len(mates), "twin_shared_bytes": twin_x_bytes,
                   "a_pass_blocks": v.a_grid,
                   "a_pass_grid_ms": {str(g): round(t, 2) for g, t in v.grid_times.items()}},
        "parts": {"step_verify_ms": round(ms, 3),
                  "step_frac_hbm": round(value / HBM_PEAK_GBPS, 4),
                  # bytes the step reads once each: every leaf, and the A and B operands
                  "step_read_bytes": read_bytes,
                  "step_read_gbps": round(read_bytes / (ms * 1e-3) / 1e9, 1),
                  "overlap": {"hashed_at_ms": round(hashed_ms, 3),
                              "rows_at_ms": round(measured_ms, 3),
                              "a_pass_in_step_ms": round(a_in_step_ms, 3),
                              "chunks_in_step_ms": round(chunks_in_step_ms, 3),
                              "serial_ms": round(serial_ms, 3)},
                  "hash_ms": round(hash_ms, 3),
                  "hash_gbps": round(hash_bytes / (hash_ms * 1e-3) / 1e9, 1),
                  "freivalds_ms": round(fv_ms, 3),
                  "freivalds_read_bytes": fv_read_bytes,
                  "freivalds_gbps": round(fv_read_bytes / (fv_ms * 1e-3) / 1e9, 1),
                  "plan_build_ms": round(plan_build_ms, 1),
                  "stages_ms": {nm: round(t, 4) for nm, t in stage_ms.items()},
                  "rejected": n_rej,
                  "check_6a": check_6a},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_from_profile(dom_name, config),
                     "kernel": dom_name,
                     "algorithmic_bytes": dom_bytes, "launch_ms": round(stage_ms[dom], 4),
                     "launch_ms_in_step": (round(in_step[dom], 4) if dom in in_step else None),
                     "valu": valu,
                     # every kernel of the step with its own roofline: the chunk kernels are
                     # bound by 32-bit VALU issue ("valu_frac"), the row passes by HBM
                     "kernels": {kernels[nm][0]: kernel_roofline(nm) for nm in
                                 sorted(kernels, key=lambda nm: -stage_ms[nm])}},
    }
    return out, v, claimed_b, items


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--hash-first", action="store_true",
                    help="start the fused chunk kernel after the challenges, not the B pass")
    ap.add_argument("--plain-early", action="store_true",
                    help="hash the unfused leaves while the B pass runs")
    ap.add_argument("--b-grid", type=int, default=0,
                    help="blocks of the B pass (0: one per tile)")
    ap.add_argument("--a-grid", type=int, default=None,
                    help="blocks of the A pass (default when fused: the fastest of 1, 1.5 "
                         "and 2 blocks per CU and one per tile, timed on the step when the "
                         "plan is built; unfused: one per tile); see pots_fv_plan_set_grid")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="copy this many MiB device to device twice before timing, so a "
                         "counter run sees a plain copy kernel of known size")
    ap.add_argument("--disk-leg", metavar="DIR",
                    help="also write the transcript under DIR in the on-disk store's format "
                         "(with the captured operands), load it back into HBM with the native "
                         "loader, verify the loaded copy, report parts.disk_load, and delete it")
    ap.add_argument("--prover-leg", nargs="?", const="mlp", choices=("mlp", "qwen2"),
                    help="also run the device-resident prover and report parts.prover: 'mlp' "
                         "proves an MLP step (capture, labeling, SGD), commits it in HBM and "
                         "verifies it with the replay; 'qwen2' proves a Qwen2-1.5B-shaped "
                         "training step (transformers, random init, bf16 autocast over fp32 "
                         "masters, 28 layers, 4x2048 tokens), commits it in HBM and verifies "
                         "it, with the prover's operands and then from the leaves alone")
    ap.add_argument("--c5-leg", action=argparse.BooleanOptionalAction, default=True,
                    help="after the C4 headline and its legs, perturb the resident transcript "
                         "as config 5 does and time it at k=16 (parts.c5)")
    ap.add_argument("--check-level", action=argparse.BooleanOptionalAction, default=True,
                    help="time Verifier.verify_step (the reference's check-level entry point) "
                         "on the same transcript, beside the step")
    ap.add_argument("--counter-summary", metavar="DIR",
                    help="summarise rocprofv3 --pmc CSV output under DIR and exit")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="summarise rocprofv3 --kernel-trace CSV output under DIR of a run "
                         "with the same --steps/--warmup, and exit")
    args = ap.parse_args()
    if args.counter_summary:
        return counter_summary(Path(args.counter_summary), args.calibration_copy_mib)
    if args.trace_summary:
        return trace_summary(Path(args.trace_summary), args.steps, args.warmup)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); sharding "
              "across GPUs is designed but not built or measured.", file=sys.stderr)
        return 2

    import torch

    from verification.commitment import native
    from verification.computation.instances import decoder
    from verification.prover.synthetic import perturb_products, synthetic_step

    native.get()
    # The prover legs build their own model and step; they run first, on an empty GPU, so
    # that the resident C4 transcript need not share HBM with them.
    prover = None
    if args.prover_leg:
        prover = prover_leg() if args.prover_leg == "mlp" else capture_leg_qwen2()
        import gc
        gc.collect()
        torch.cuda.empty_cache()
    desc, ctor, k = CONFIGS[args.config]
    c = getattr(decoder, ctor)()
    log(f"[bench] {args.config}: {c.M} products, {c.n_leaves} leaves, k={k}")
    t0 = time.perf_counter()
    step = synthetic_step(c, seed=0, operands=True)
    step.k = k
    if args.config == "c5":
        perturb_products(step, C5_FRACTION, seed=C5_SEED)
    torch.cuda.synchronize()
    log(f"[bench] transcript built in {time.perf_counter() - t0:.1f} s, "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB resident")

    if args.calibration_copy_mib:
        src = torch.ones(args.calibration_copy_mib << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    out, v, claimed_b, items = measure_step(c, step, k, args, desc, args.config)
    if args.check_level:
        out["parts"]["check_level"] = check_level_leg(c, step, k, claimed_b)
    if args.disk_leg:
        out["parts"]["disk_load"] = disk_leg(Path(args.disk_leg), c, step, k, claimed_b, v)
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline")
        out["cpu_baseline"] = cpu_baseline(step, items)
    if prover is not None:
        out["parts"]["prover"] = prover
    if args.c5_leg and args.config == "c4":
        v.close()
        del v
        out["parts"]["c5"] = c5_leg(c, step, args)
    print(json.dumps(out), flush=True)
    return 0


def c5_leg(c, step, args) -> dict:
    """Config 5 on the resident C4 transcript, beside the headline: a seeded 1% of the
    products perturbed in place (one entry each, relative size log-uniform in [1e-6, 1]), the
    transcript re-rooted as the forging prover would commit it, and the step timed at k = 16
    with every kernel's roofline. Runs last: it changes the transcript."""
    import torch

    from verification.prover.synthetic import perturb_products
    forged = perturb_products(step, C5_FRACTION, seed=C5_SEED)
    log(f"[bench] c5 leg: {len(forged)} products perturbed, k=16")
    sub = argparse.Namespace(**{**vars(args), "steps": max(3, min(args.steps, 5)),
                                "warmup": 1, "a_grid": None})
    out, v, _, _ = measure_step(c, step, 16, sub, CONFIGS["c5"][0], "c5")
    v.close()
    torch.cuda.synchronize()
    parts = out["parts"]
    return {"k": 16, "perturbed": len(forged), "rejected": parts["rejected"],
            "ms_per_step": out["ms_per_step"], "value": out["value"], "unit": "GB/s",
            "step_frac_hbm": parts["step_frac_hbm"],
            "hash_bytes": out["config"]["hash_bytes"],
            "freivalds_bytes": out["config"]["freivalds_bytes"],
            "twins": out["config"]["twins"], "a_pass_blocks": out["config"]["a_pass_blocks"],
            "p_pass_fused_products": out["config"]["p_pass_fused_products"],
            "overlap": parts["overlap"], "stages_ms": parts["stages_ms"],
            "dominant": {key: out["roofline"][key] for key in
                         ("kernel", "bound", "achieved", "frac", "launch_ms")},
            "kernels": out["roofline"]["kernels"]}


if __name__ == "__main__":
    sys.exit(main())
