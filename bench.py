"""Benchmark: one verified step of the hot path on a resident transcript, on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--no-cpu-baseline]

A step is the verifier's whole hot path over one training step's transcript, already in HBM
(check 2 and check 5 of the reference, verification/verifier/checks.py:204-272,576-658):
hash every leaf (BLAKE3 chunks, per-leaf trees, NaN/Inf test fused) and build the Merkle
root; expand the claimed root into every product's challenge matrix; run the three
Freivalds passes over every product's B, A and P; reduce to one fp64 row per product; judge
every product. One host read at the end of the step (root, first non-finite leaf, first
rejected product).

Prints one JSON line (the driver's contract): `value` is the step's verified throughput,
(bytes hashed + bytes Freivalds-checked) / step time, in GB/s; `parts` splits it by stage;
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
METRIC = "Freivalds-verified GB/s + BLAKE3 Merkle GB/s (% HBM roofline); step verify ms"
CONFIGS = {
    "c1": ("SmolLM2-135M step, 4x256 tokens, fp32, k=1", "smollm2_135m", 1),
    "c3": ("Qwen2-0.5B-shaped step, 8x1024 tokens, bf16, k=2", "qwen2_0_5b_shape", 2),
    "c4": ("Qwen2-1.5B-shaped step, 4x2048 tokens, bf16, k=4", "qwen2_1_5b_shape", 4),
}


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


def cpu_baseline(step, items, budget_s: float = 20.0) -> dict:
    """The CPU oracle on a bounded sample of the same transcript, on the host's cores:
    leaf hashing with the pthread restatement of the reference's native.c, and the
    reference's Freivalds formulas (torch-CPU fp32) on products of layer 1."""
    import torch

    import oracle as O
    c = step.c
    threads = cores()
    torch.set_num_threads(threads)
    # hashing sample: product leaves until ~1.5 GB
    hs, hbytes = [], 0
    for i in range(c.n_s + c.n_w, c.n_s + c.n_w + c.M):
        t = step.leaves[i].cpu()
        hs.append((O.tensor_leaf_header(O.TAG_PRODUCT, t), t, O.FINITE_KIND[t.dtype]))
        hbytes += 1 + len(hs[-1][0]) + t.nbytes
        if hbytes > 1.5e9:
            break
    O.hash_leaves(hs[:2], threads)
    t0 = time.perf_counter()
    O.hash_leaves(hs, threads)
    t_hash = time.perf_counter() - t0
    # Freivalds sample: the first products in canonical order, until ~budget/2 seconds
    fbytes, t_fv, nprod = 0, 0.0, 0
    key = bytes(range(32))
    for a, b, p, bias, m in items:
        if t_fv > budget_s / 2:
            break
        a_c, b_c, p_c = a.cpu(), b.cpu(), p.cpu()
        t0 = time.perf_counter()
        r = O.challenge_matrices(key, [m], step.k, p_c.shape[1], threads)[0]
        O.measure_product_row(a_c, b_c, p_c, r, None if bias is None else bias.cpu())
        t_fv += time.perf_counter() - t0
        fbytes += a_c.nbytes + b_c.nbytes + p_c.nbytes
        nprod += 1
    value = (hbytes + fbytes) / (t_hash + t_fv) / 1e9
    return {"value": round(value, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"hash {len(hs)} product leaves ({hbytes / 1e9:.2f} GB, "
                      f"{hbytes / t_hash / 1e9:.2f} GB/s, portable scalar BLAKE3 on {threads} "
                      f"pthreads) + Freivalds rows of the first {nprod} products "
                      f"({fbytes / 1e9:.2f} GB, {fbytes / t_fv / 1e9:.3f} GB/s, torch-CPU "
                      f"fp32 with {threads} threads, challenges included), one run each"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding is a design in DESIGN.md, not a measured path.", file=sys.stderr)
        return 2

    import torch

    from verification.commitment import native
    from verification.computation.instances import decoder
    from verification.prover.synthetic import synthetic_step
    from verification.verifier.step import DeviceStepVerifier

    lib = native.get()
    desc, ctor, k = CONFIGS[args.config]
    c = getattr(decoder, ctor)()
    log(f"[bench] {args.config}: {c.M} products, {c.n_leaves} leaves, k={k}")
    t0 = time.perf_counter()
    step = synthetic_step(c, seed=0, operands=True)
    step.k = k
    torch.cuda.synchronize()
    log(f"[bench] transcript built in {time.perf_counter() - t0:.1f} s, "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB resident")

    stream = torch.cuda.current_stream()
    items = product_inputs(step)
    v = DeviceStepVerifier(c, step.leaves, lambda spec: step.operands[spec.m], k=k)
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
    root = flags[:8].numpy().tobytes()
    first_bad, first_fail = int(flags[8]), int(flags[9])
    assert root == claimed_b, "recomputed root differs from the claim"
    assert first_bad == c.n_leaves, "a synthetic leaf was reported non-finite"
    n_rej = int((codes[:, 0] != 0).sum())
    log(f"[bench] step {ms:.2f} ms (streams overlapped: hashing done at {hashed_ms:.2f} ms, "
        f"Freivalds rows at {measured_ms:.2f} ms); {n_rej} rejected (first {first_fail})")

    # Stage leg: the same work serialised on one stream, every stage bracketed by events on
    # that stream, for the per-kernel figures and the roofline.
    names = ([f"hash.{s}" for s in native.LeafPlan.STAGES] + ["tree"] +
             [f"freivalds.{s}" for s in native.FvPlan.STAGES] + ["verdicts"])

    def staged(ev):
        i = 0
        ev[i].record(stream)
        for st in range(len(native.LeafPlan.STAGES)):
            v.hasher.plan.run_stage(st, v.digests, v.bad, stream)
            i += 1
            ev[i].record(stream)
        lib.merkle_tree_device(v.digests, stream)
        i += 1
        ev[i].record(stream)
        v.key.copy_(claimed)
        for st in range(len(native.FvPlan.STAGES)):
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

    # Algorithmic HBM bytes of each single-kernel stage: the operand every element of which
    # the kernel reads once (A, B or P of every product; every leaf's message bytes plus one
    # 32-byte chaining value written per 1 KiB chunk).
    a_bytes = sum(a.nbytes for a, _, _, _, _ in items)
    b_bytes = sum(b.nbytes for _, b, _, _, _ in items)
    p_bytes = sum(p.nbytes for _, _, p, _, _ in items)
    kernels = {
        "hash.chunks": ("chunk_kernel", hash_bytes + 32 * v.hasher.plan.chunks),
        "freivalds.a_pass": ("row_pass<bf16, weighted> (A pass)", a_bytes),
        "freivalds.p_pass": ("row_pass<bf16, fp64 squares> (P pass)", p_bytes),
        "freivalds.b_pass": ("row_pass<bf16> (B pass)", b_bytes),
    }
    dom = max(kernels, key=lambda nm: stage_ms[nm])
    dom_name, dom_bytes = kernels[dom]
    achieved = dom_bytes / (stage_ms[dom] * 1e-3) / 1e9
    hash_ms = sum(stage_ms[f"hash.{s}"] for s in native.LeafPlan.STAGES)
    fv_ms = sum(stage_ms[f"freivalds.{s}"] for s in native.FvPlan.STAGES)
    total = hash_bytes + fv_bytes
    value = total / (ms * 1e-3) / 1e9
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
                   "hash_bytes": hash_bytes, "freivalds_bytes": fv_bytes},
        "parts": {"step_verify_ms": round(ms, 3),
                  "step_frac_hbm": round(value / HBM_PEAK_GBPS, 4),
                  "overlap": {"hashed_at_ms": round(hashed_ms, 3),
                              "rows_at_ms": round(measured_ms, 3),
                              "serial_ms": round(serial_ms, 3)},
                  "hash_ms": round(hash_ms, 3),
                  "hash_gbps": round(hash_bytes / (hash_ms * 1e-3) / 1e9, 1),
                  "freivalds_ms": round(fv_ms, 3),
                  "freivalds_gbps": round(fv_bytes / (fv_ms * 1e-3) / 1e9, 1),
                  "stages_ms": {nm: round(t, 4) for nm, t in stage_ms.items()},
                  "rejected": n_rej},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": None, "kernel": dom_name,
                     "algorithmic_bytes": dom_bytes, "launch_ms": round(stage_ms[dom], 4)},
    }
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline")
        out["cpu_baseline"] = cpu_baseline(step, items)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
