"""Benchmark of the scoring-and-selection hot path on one MI355X.

Default workload: the metric's filtered top-100 over the 30M x 512 int8 table. Items are
per-row int8 quantizations of N(0,1) float32 rows (scale = max|x| / 127), queries likewise
(B = 16); every item carries the 8 categorical attributes of the filtered-kNN configuration
(cardinalities 16 .. 1000, Zipf(1.1) values) and a 64-bit, 3-hash Bloom signature over its
(attribute, value) tokens; each query is an AND over 1-3 attributes of OR over value sets, tuned
to 10 % selectivity. A step is the filtered forward over one query batch, inputs resident in
HBM: the Bloom pre-filter (plans prepared once, outside the timed region, as the reference's
prepare_queries), the exact clause post-check on the Bloom survivors, and the int8 scan with the
fused exact top-100 (ties to the lower index). ``--filter none`` times the plain scan.

Prints one JSON line with the whole-job throughput (queries/s), the dominant kernel's (the int8
scan's) roofline fraction measured live with HIP events on its launch stream, and the
reference's CPU path (torch.mm over item chunks + the filter + top-k) timed on a bounded sample
on this host.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
CARDINALITIES = (16, 32, 64, 128, 256, 512, 1000, 1000)
BLOOM_BITS, BLOOM_K, HASH_K = 64, 3, 7


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def quantize_rows(x: torch.Tensor) -> torch.Tensor:
    """Per-row symmetric int8 (the reference's quantize_int8 codes) for synthetic tables."""
    a = x.abs().amax(dim=1, keepdim=True).clamp_min(1e-8)
    return ((x.double() / a.double()).float() * 127.0).round().clamp(-128, 127).to(torch.int8)


def int8_table(n: int, d: int, seed: int, dev: torch.device, chunk: int = 1 << 20) -> torch.Tensor:
    gen = torch.Generator(device=dev).manual_seed(seed)
    out = torch.empty((n, d), dtype=torch.int8, device=dev)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        out[s : s + m] = quantize_rows(torch.randn((m, d), generator=gen, device=dev))
    return out


def zipf(card: int, s: float = 1.1) -> torch.Tensor:
    p = 1.0 / torch.arange(1, card + 1, dtype=torch.float64) ** s
    return p / p.sum()


def attr_table(n: int, seed: int, dev: torch.device, chunk: int = 1 << 22) -> torch.Tensor:
    """[N, 8, 1] int16 attribute values, Zipf(1.1) over each attribute's cardinality."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    out = torch.empty((n, len(CARDINALITIES), 1), dtype=torch.int16, device=dev)
    for c, card in enumerate(CARDINALITIES):
        p = zipf(card).to(dev)
        for s in range(0, n, chunk):
            m = min(chunk, n - s)
            out[s : s + m, c, 0] = torch.multinomial(p, m, replacement=True, generator=gen).to(
                torch.int16)
    return out


def query_sets(attrs: torch.Tensor, b: int, selectivity: float, seed: int) -> np.ndarray:
    """[B, 8, V] value sets (-1 pads): row r ANDs 1 + r % 3 random attributes, each an OR of its
    most frequent values from rank 0 or 1 on (small sets), grown until the attribute's mass reaches
    selectivity ** (1 / attributes) (attributes are independent, so the row's selectivity is
    about the target; the bench measures it exactly)."""
    g = np.random.default_rng(seed)
    freq = [torch.bincount(attrs[:, c, 0].long(), minlength=card).double().cpu().numpy()
            for c, card in enumerate(CARDINALITIES)]
    freq = [f / f.sum() for f in freq]
    rows = []
    for r in range(b):
        n_attr = 1 + r % 3
        chosen = g.choice(len(CARDINALITIES), n_attr, replace=False)
        target = selectivity ** (1.0 / n_attr)
        row = [[] for _ in CARDINALITIES]
        for c in chosen:
            order = np.argsort(-freq[c], kind="stable")
            order = np.roll(order, -int(g.integers(0, 2)))
            mass = 0.0
            for v in order:
                if mass >= target:
                    break
                row[c].append(int(v))
                mass += freq[c][v]
        rows.append(row)
    v = max(len(x) for row in rows for x in row)
    out = np.full((b, len(CARDINALITIES), v), -1, np.int64)
    for r, row in enumerate(rows):
        for c, vals in enumerate(row):
            out[r, c, : len(vals)] = vals
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--n", type=int, default=30_000_000)
    ap.add_argument("--d", type=int, default=512)
    ap.add_argument("--k", type=int, default=100)
    ap.add_argument("--filter", choices=("bloom", "none"), default="bloom",
                    help="bloom: Bloom pre-filter + exact clause post-check (the metric's "
                         "filtered top-100); none: the plain scan")
    ap.add_argument("--selectivity", type=float, default=0.1)
    ap.add_argument("--cpu-sample", type=int, default=2_000_000,
                    help="items of the CPU baseline's bounded sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 2 GiB device copy three times (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against a known byte count)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one GPU per box); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import retrieve_amd.hip  # noqa: F401  (registers torch.ops.retrieve.*)
    import retrieve_amd.st as st
    from retrieve_amd import _native
    from retrieve_amd import bloom as bl

    dev = torch.device("cuda:0")
    b, n, d, k = args.batch, args.n, args.d, args.k
    filtered = args.filter == "bloom"
    log(f"generating items {n}x{d} int8 and queries {b}x{d}")
    items = int8_table(n, d, 1234, dev)
    queries = int8_table(b, d, 99, dev)
    torch.cuda.synchronize()

    rev = words = offs = blob = sets_t = attrs = None
    plan_count = max_stack = 0
    measured_sel = None
    if filtered:
        log("generating attributes, Bloom index and query plans")
        attrs = attr_table(n, 4321, dev)
        sets = query_sets(attrs, b, args.selectivity, 77)
        fid, fo, fv = st.attrs_to_features(attrs.long())
        words, offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, BLOOM_BITS, BLOOM_K)
        del fid, fo, fv
        blob, plan_count, max_stack = st.prepare_plans(bl.sets_to_expressions(sets), HASH_K, dev)
        rev = torch.zeros(len(CARDINALITIES), dtype=torch.bool, device=dev)
        sets_t = torch.from_numpy(sets).to(dev)
        exact = torch.ops.retrieve.clause_bits(attrs, rev, sets_t)
        counts = torch.ops.retrieve.mask_compact(exact, n)[1]
        measured_sel = (counts.double() / n).cpu().numpy()
        del exact
        torch.cuda.synchronize()
        log(f"selectivity per row: mean {measured_sel.mean():.4f}, "
            f"min {measured_sel.min():.4f}, max {measured_sel.max():.4f}")

    def step():
        mask = None
        if filtered:
            pre = torch.ops.st.bloom_index_search_batch_prepared(
                words, offs, blob, plan_count, max_stack, BLOOM_K, HASH_K)
            mask = torch.ops.retrieve.clause_bits(attrs, rev, sets_t, pre)
        return torch.ops.retrieve.int8_scan_topk(queries, items, k, mask)

    if args.copy_probe:
        src = torch.empty(2 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy probe: 3 x 2 GiB device copies")
        del src, dst

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    lib = _native.lib()
    _native.check(lib.rt_profile_enable(1))
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = ctypes.c_double()
    launches = ctypes.c_int64()
    _native.check(lib.rt_profile_collect(ctypes.byref(total_ms), ctypes.byref(launches)))
    _native.check(lib.rt_profile_enable(0))
    ms_step = wall * 1e3 / args.steps
    kernel_ms = total_ms.value / max(1, launches.value)
    scan_bytes = n * d + b * d  # the item table once + the query block
    achieved = scan_bytes / (kernel_ms * 1e-3) / 1e9
    # the whole step's algorithmic bytes: + Bloom words, the int16 attributes, the masks
    step_bytes = scan_bytes
    if filtered:
        step_bytes += n * BLOOM_BITS // 8 + n * len(CARDINALITIES) * 2 + 3 * b * n // 8
    log(f"ms/step {ms_step:.3f}; main scan {kernel_ms:.3f} ms ({achieved:.0f} GB/s)")

    cpu = None
    if not args.no_cpu:
        from oracle import baseline

        ns = min(args.cpu_sample, n)
        log(f"cpu baseline on {ns} items")
        q_cpu = queries.cpu()
        it_cpu = items[:ns].cpu()
        valid_fn = None
        if filtered:
            valid_fn = baseline.clause_sets_valid(attrs[:ns].cpu().long(), sets_t.cpu())
        t_s, threads = baseline.time_int8(q_cpu, it_cpu, k, valid_fn=valid_fn)
        t_full = t_s * (n / ns)
        what = "torch.mm over 2M-row chunks + topk + lowest-id merge"
        if filtered:
            what = "the exact value-set filter (torch.isin) gating " + what
        cpu = {
            "value": b / t_full,
            "unit": "queries/s",
            "cores": threads,
            "kind": "port",
            "sample": f"B={b} queries x first {ns} of {n} items ({what}), median of 3, scaled "
                      f"x{n / ns:.1f} to the full table; host has {os.cpu_count()} logical CPUs",
        }

    workload = f"int8 scan top-{k}: N={n} D={d} B={b}"
    if filtered:
        workload = (f"filtered int8 top-{k}: N={n} D={d} B={b}; Bloom {BLOOM_BITS} bits/item, "
                    f"{BLOOM_K} hashes pre-filter + exact AND-of-OR clause post-check over 8 "
                    f"attributes at {args.selectivity:.0%} target selectivity")
    line = {
        "metric": "queries/sec + achieved HBM GB/s, filtered top-100 over 30Mx512 int8 items",
        "value": b * args.steps / wall,
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: per-row int8 of N(0,1) float32 rows (torch generator seeds 1234 / "
                "99); attributes Zipf(1.1) (seed 4321), query sets numpy seed 77",
        "config": {
            "workload": workload,
            "global_batch": b,
            "achieved_hbm_gbs_whole_step": step_bytes / (ms_step * 1e-3) / 1e9,
            "measured_selectivity": None if measured_sel is None else float(measured_sel.mean()),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
