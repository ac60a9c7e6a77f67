"""Benchmark of the scoring-and-selection hot path on one MI355X.

Default workload (``--workload filtered``): the metric's filtered top-100 over the 30M x 512
int8 table. Items are per-row int8 quantizations of N(0,1) float32 rows (scale = max|x| / 127),
queries likewise (B = 16); every item carries the 8 categorical attributes of the filtered-kNN
configuration (cardinalities 16 .. 1000, Zipf(1.1) values) and a 64-bit, 3-hash Bloom signature
over its (attribute, value) tokens; each query is an AND over 1-3 attributes of OR over value
sets, tuned to 10 % selectivity. A step is the filtered forward over one query batch, inputs
resident in HBM: the Bloom pre-filter (plans prepared once, outside the timed region, as the
reference's prepare_queries), then the int8 scan with the fused exact top-100 (ties to the lower
index) and the exact clause post-check inside it: an item is checked against its query's clauses
where its score beats the query's running bound and its Bloom bit is set, as st::search's scorer
checks each Bloom-passing doc (``--unfused-filter``: the clause kernel writes the post-checked
mask first, and the scan reads it).

Other workloads (the remaining configurations, same JSON line):
  int8     the plain int8 scan top-k (configuration 4; ``--batch`` 1 / 16 / 256 / 1024)
  dense    bf16 top-100 over 10M x 128 clustered, L2-normalised items (configuration 2), with
           recall@100 against exact float32 scoring of the unrounded items
  filtered-dense  the same items under the Bloom pre-filter + exact clause post-check at 10 %,
           B = 256 (configuration 3)
  binary   1-bit retrieval: SimHash codes (sign of a Gaussian projection, 512 bits) scanned by
           Hamming score for the top-1000 under the Bloom + exact filter at 10 %, re-ranked by
           the int8 codes of the same vectors to the top-100 (configuration 5, B = 256)
  hamming  the plain 1-bit Hamming top-k over the same 30M SimHash codes (B = 16 by default)

Prints one JSON line with the whole-job throughput (queries/s), the dominant kernel's roofline
fraction measured live with HIP events on its launch stream, and the reference's CPU path timed
on a bounded sample on this host.
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
# HBM bytes per launch of the main scan (FETCH_SIZE x 2 + WRITE_SIZE, calibrated against a plain
# 2 GiB device copy), measured with rocprofv3 --pmc for these exact workloads; keyed by
# (workload, N, D, B, k). The profiles/ summaries named below give the counts and commands.
MEASURED_TRAFFIC: dict = {
    ("filtered", 30_000_000, 512, 16, 100): 15_399_664_224,  # filtered_int8_30Mx512_b16.md
    ("int8", 30_000_000, 512, 16, 100): 15_361_455_360,  # int8_scan_30Mx512_b16.md
    ("int8", 30_000_000, 512, 256, 100): 15_365_323_008,  # int8_scan_30Mx512_b256.md
    ("int8", 30_000_000, 512, 1024, 100): 44_373_443_584,  # int8_scan_30Mx512_b1024.md
    ("dense", 10_000_000, 128, 64, 100): 2_566_548_500,  # dense_bf16_10Mx128_b64.md
    ("dense", 10_000_000, 128, 1024, 100): 7_655_515_443,  # dense_bf16_10Mx128_b1024.md
    ("dense", 10_000_000, 128, 4096, 100): 14_667_483_648,  # dense_bf16_10Mx128_b4096.md
    # filtered_dense_bf16_10Mx128_b256.md, binary_30Mx512bit_b256.md
    ("filtered-dense", 10_000_000, 128, 256, 100): 2_886_129_572,
    ("binary", 30_000_000, 512, 256, 100): 2_909_370_266,
    ("hamming", 30_000_000, 512, 16, 100): 1_921_363_968,  # hamming_30Mx512bit_b16.md
}
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


def dense_table(n: int, d: int, centres: torch.Tensor, seed: int, dev: torch.device,
                chunk: int = 1 << 20) -> torch.Tensor:
    """[N, D] float32 rows centre[u] + 0.3 N(0,1), u uniform over the centres, L2-normalised."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    out = torch.empty((n, d), dtype=torch.float32, device=dev)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        u = torch.randint(0, centres.shape[0], (m,), generator=gen, device=dev)
        x = centres[u] + 0.3 * torch.randn((m, d), generator=gen, device=dev)
        out[s : s + m] = torch.nn.functional.normalize(x, dim=1)
    return out


def simhash_tables(n: int, d: int, proj: torch.Tensor, seed: int, dev: torch.device,
                   chunk: int = 1 << 20, with_codes: bool = True):
    """N(0,1) rows x: their SimHash codes (bit b of word w = (x @ proj.T)[64 w + b] > 0, the
    reference's LSB-first packing) and their per-row int8 codes (None without with_codes)."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    bits_out = torch.empty((n, proj.shape[0] // 64), dtype=torch.int64, device=dev)
    codes = torch.empty((n, d), dtype=torch.int8, device=dev) if with_codes else None
    shifts = torch.arange(64, device=dev, dtype=torch.int64)
    for s in range(0, n, chunk):
        m = min(chunk, n - s)
        x = torch.randn((m, d), generator=gen, device=dev)
        signs = (x @ proj.t() > 0).view(m, -1, 64).long()
        bits_out[s : s + m] = (signs << shifts).sum(-1)
        if codes is not None:
            codes[s : s + m] = quantize_rows(x)
    return bits_out, codes


class Filter:
    """The filtered-kNN configuration's attributes, Bloom index and query plans for B rows."""

    def __init__(self, n: int, b: int, selectivity: float, dev: torch.device):
        import retrieve_amd.st as st
        from retrieve_amd import bloom as bl

        log("generating attributes, Bloom index and query plans")
        self.attrs = attr_table(n, 4321, dev)
        sets = query_sets(self.attrs, b, selectivity, 77)
        fid, fo, fv = st.attrs_to_features(self.attrs.long())
        self.words, self.offs = torch.ops.st.bloom_index_build_fixed(fid, fo, fv, BLOOM_BITS,
                                                                     BLOOM_K)
        del fid, fo, fv
        # the row view the scans' per-candidate probe reads, built once beside the index
        self.doc_bits = torch.ops.retrieve_amd.bloom_doc_bits(self.words, self.offs, n)
        self.blob, self.plan_count, self.max_stack = st.prepare_plans(
            bl.sets_to_expressions(sets), HASH_K, dev)
        self.rev = torch.zeros(len(CARDINALITIES), dtype=torch.bool, device=dev)
        self.sets = torch.from_numpy(sets).to(dev)
        exact = torch.ops.retrieve_amd.clause_bits(self.attrs, self.rev, self.sets)
        counts = torch.ops.retrieve_amd.mask_compact(exact, n)[1]
        self.selectivity = (counts.double() / n).cpu().numpy()
        torch.cuda.synchronize()
        log(f"selectivity per row: mean {self.selectivity.mean():.4f}, "
            f"min {self.selectivity.min():.4f}, max {self.selectivity.max():.4f}")

    def bloom(self) -> torch.Tensor:
        """One batch's Bloom pre-filter: [B, ceil(N/64)] words."""
        return torch.ops.st.bloom_index_search_batch_prepared(
            self.words, self.offs, self.blob, self.plan_count, self.max_stack, BLOOM_K, HASH_K)

    def bloom_t(self) -> torch.Tensor:
        """The same words stored transposed (``st.bloom_search_t``): the blocked scans of large
        batches read them without a transpose per call."""
        import retrieve_amd.st as st

        return st.bloom_search_t(self.words, self.offs, self.blob, self.plan_count,
                                 self.max_stack, BLOOM_K, HASH_K)

    def scan(self, queries: torch.Tensor, items: torch.Tensor, k: int):
        """One batch's filtered top-k with the Bloom plans probed per candidate inside the scan,
        then the exact clauses (``scan_topk_bloom_clauses``): no Bloom mask is written."""
        return torch.ops.retrieve_amd.scan_topk_bloom_clauses(
            queries, items, k, self.attrs, self.rev, self.sets, self.doc_bits, self.words,
            self.offs, self.blob, self.plan_count, self.max_stack, BLOOM_K, HASH_K)

    def mask(self) -> torch.Tensor:
        """One batch's filter: Bloom pre-filter, then the exact post-check of its survivors."""
        return torch.ops.retrieve_amd.clause_bits(self.attrs, self.rev, self.sets, self.bloom())

    def bytes(self, n: int, b: int, fused: bool = False, probed: bool = False) -> int:
        """Algorithmic bytes of one batch's filter: the Bloom words and the Bloom mask written;
        unfused, also the int16 attributes, the Bloom mask read and the clause mask written
        (the scan's mask words, and fused its attribute reads, are sparse: candidates only);
        probed, nothing but the candidates' row bits and attributes (sparse)."""
        if probed:
            return 0
        if fused:
            return n * BLOOM_BITS // 8 + b * n // 8
        return n * BLOOM_BITS // 8 + n * len(CARDINALITIES) * 2 + 3 * b * n // 8

    def valid_fn(self, ns: int):
        from oracle import baseline

        return baseline.clause_sets_valid(self.attrs[:ns].cpu().long(), self.sets.cpu())


def _time_calls(fn, n: int) -> tuple[list, float]:
    """Per-call ms from an event pair around each call on the current stream, and the window's
    wall seconds."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s, e in ev:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in ev], time.perf_counter() - t0


def window_stats(ms: list, wall_s: float, bs: int) -> dict:
    """One window's summary with the reference harness's fields
    (evaluation/bench/measure.py:248-273): linear-interpolated quantiles, the mean trimmed by
    n // 10 calls at each end, closed-loop queries/s."""
    t = np.asarray(ms, dtype=np.float64)
    n = t.size
    q1, med, q3, p95, p99 = np.percentile(t, [25, 50, 75, 95, 99])
    mean, std = float(t.mean()), float(t.std())
    iqr = q3 - q1
    cut = n // 10
    return {
        "n": n,
        "median_ms": float(med),
        "mean_ms": mean,
        "trimmed_mean_ms": float(np.sort(t)[cut : n - cut].mean()),
        "p95_ms": float(p95),
        "p99_ms": float(p99),
        "min_ms": float(t.min()),
        "iqr_ms": float(iqr),
        "qps": n * bs / wall_s if wall_s > 0 else None,
        "host_gap_ms": wall_s * 1e3 / n - mean,
        "outliers_std": int((np.abs(t - mean) > 3 * std).sum()),
        "outliers_tukey": int(((t < q1 - 1.5 * iqr) | (t > q3 + 1.5 * iqr)).sum()),
        "load": "closed_loop",
    }


def latency_windows(step, windows: int, calls: int, b: int, mode: str, warmup: int = 50,
                    target_s: float = 2.0, n_min: int = 1000, n_max: int = 5000) -> dict:
    """The reference harness's latency protocol (evaluation/bench/measure.py:281-345), after
    the timed steps: `warmup` calls, a 20-call estimate, then `windows` windows of
    clamp(target_s / median, n_min, n_max) calls (or `calls`), the window with the median
    median reported with its spread over windows. Not part of ``value``."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    est, _ = _time_calls(step, 20)
    med = max(float(np.median(est)), 1e-6)
    n = calls if calls > 0 else int(min(max(target_s * 1e3 / med, n_min), n_max))
    runs = [_time_calls(step, n) for _ in range(windows)]
    medians = [float(np.median(ms)) for ms, _ in runs]
    pick = sorted(range(windows), key=medians.__getitem__)[windows // 2]
    d = window_stats(*runs[pick], b)
    d.update(mode=mode, bs=b, windows=windows,
             spread=(max(medians) - min(medians)) / medians[pick] if medians[pick] > 0 else 0.0,
             window_medians_ms=medians)
    d["unstable"] = d["spread"] > 0.05
    return d


GRAPH_LAUNCH_EVENTS = ("cudaGraphLaunch", "hipGraphLaunch")


class NotCapturable(RuntimeError):
    """The step does not compile to one graph launch per call."""


def mark_static(fn) -> None:
    """Mark the device tensors a step closure reads (directly, or as attributes of an object it
    holds) as static addresses, so the compiled graph reads them in place instead of copying
    them into its input buffers before every replay (a module's buffers, as the reference's
    tables are, are static already)."""
    seen: set[int] = set()

    def visit(obj, depth):
        if isinstance(obj, torch.Tensor):
            if obj.is_cuda and id(obj) not in seen:
                seen.add(id(obj))
                torch._dynamo.mark_static_address(obj)
        elif depth == 0 and hasattr(obj, "__dict__") and not isinstance(obj, torch.nn.Module):
            for v in vars(obj).values():
                visit(v, 1)

    for cell in getattr(fn, "__closure__", None) or ():
        visit(cell.cell_contents, 0)


def graph_callable(fn, *example_args, warmup: int = 5):
    """The reference harness's ``graph`` mode (``evaluation/bench/measure.py:348-373``):
    ``torch.compile(fn, mode="reduce-overhead", dynamic=False, fullgraph=True)`` warmed on
    ``example_args`` under ``inference_mode``; raises ``NotCapturable`` unless the warm-up
    caused no cudagraph skip and one call is exactly one graph launch. Call the result under
    ``torch.inference_mode()`` too (the mode it was captured in)."""
    from torch._dynamo.utils import counters
    from torch.profiler import ProfilerActivity, profile

    mark_static(fn)
    skips_before = int(counters["inductor"]["cudagraph_skips"])
    compiled = torch.compile(fn, mode="reduce-overhead", dynamic=False, fullgraph=True)
    with torch.inference_mode():
        for _ in range(warmup):
            compiled(*example_args)
        torch.cuda.synchronize()
        skips = int(counters["inductor"]["cudagraph_skips"]) - skips_before
        if skips:
            raise NotCapturable(f"cudagraph_skips={skips}")
        with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
            compiled(*example_args)
            torch.cuda.synchronize()
    events = prof.key_averages()
    launches = sum(e.count for e in events if e.key in GRAPH_LAUNCH_EVENTS)
    if launches != 1:
        seen = sorted({e.key for e in events if "raph" in e.key})
        raise NotCapturable(f"graph launches per call = {launches}, expected 1 ({seen})")
    return compiled


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload",
                    choices=("filtered", "int8", "dense", "filtered-dense", "binary", "hamming",
                             "exact"),
                    default="filtered")
    ap.add_argument("--batch", type=int, default=None,
                    help="query batch (default: 16 filtered / int8 / hamming, 64 dense, 256 "
                         "filtered-dense / binary)")
    ap.add_argument("--n", type=int, default=None,
                    help="items (default: 30M, dense 10M)")
    ap.add_argument("--d", type=int, default=None, help="dimensions (default 512, dense 128)")
    ap.add_argument("--k", type=int, default=100)
    ap.add_argument("--filter", choices=("bloom", "none"), default=None,
                    help="kept for older command lines: none = --workload int8")
    ap.add_argument("--selectivity", type=float, default=0.1)
    ap.add_argument("--unfused-bits", action="store_true",
                    help="binary: write the clause mask before the 1-bit scan (default: the "
                         "clauses are tested inside the scan, for the candidates only)")
    ap.add_argument("--unfused-filter", action="store_true",
                    help="filtered workloads: write the clause-checked mask before the scan "
                         "instead of checking the clauses inside it")
    ap.add_argument("--bloom-search", action="store_true",
                    help="filtered: search the Bloom index for the batch's mask first, then "
                         "scan under it (default: the Bloom plans are probed per candidate "
                         "inside the scan)")
    ap.add_argument("--cpu-sample", type=int, default=None,
                    help="items of the CPU baseline's bounded sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--windows", type=int, default=3,
                    help="latency windows after the timed steps, the reference harness's "
                         "protocol (0: none)")
    ap.add_argument("--window-calls", type=int, default=0,
                    help="calls per latency window (default: 2 s worth, clamped to 1000-5000)")
    ap.add_argument("--mode", choices=("eager", "graph"), default="eager",
                    help="graph: time calls of the step compiled with torch.compile("
                         "mode='reduce-overhead', fullgraph=True), gated as the reference "
                         "harness gates it (no cudagraph skip, one graph launch per call)")
    ap.add_argument("--jsonl", default=None,
                    help="append the latency record (reference harness fields) to this file")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 2 GiB device copy three times (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against a known byte count)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one GPU per box); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if args.filter == "none":
        args.workload = "int8"

    import retrieve_amd.hip  # noqa: F401  (registers torch.ops.retrieve.* / retrieve_amd.*)
    import retrieve_amd.st  # noqa: F401  (registers torch.ops.st.*)
    from retrieve_amd import _native

    dev = torch.device("cuda:0")
    wl = args.workload
    b = args.batch or {"filtered": 16, "int8": 16, "dense": 64, "filtered-dense": 256,
                       "binary": 256, "hamming": 16, "exact": 1024}[wl]
    dense_wl = wl in ("dense", "filtered-dense", "exact")
    n = args.n or {"exact": 100_000}.get(wl, 10_000_000 if dense_wl else 30_000_000)
    d = args.d or (128 if dense_wl else 512)
    k = args.k
    extra: dict = {}
    cpu_fn = None

    if wl in ("filtered", "int8"):
        log(f"generating items {n}x{d} int8 and queries {b}x{d}")
        items = int8_table(n, d, 1234, dev)
        queries = int8_table(b, d, 99, dev)
        flt = Filter(n, b, args.selectivity, dev) if wl == "filtered" else None

        def step():
            if flt is None:
                return torch.ops.retrieve_amd.int8_scan_topk(queries, items, k)
            if args.unfused_filter:
                return torch.ops.retrieve_amd.int8_scan_topk(queries, items, k, flt.mask())
            if args.bloom_search:
                return torch.ops.retrieve_amd.int8_scan_topk_clauses(
                    queries, items, k, flt.attrs, flt.rev, flt.sets, flt.bloom())
            return flt.scan(queries, items, k)

        scan_bytes = n * d + b * d  # the item table once + the query block
        table = items  # the streamed table (the read ceiling is measured over it)
        scan_ops = 2 * b * n * d
        probed = not (args.unfused_filter or args.bloom_search)
        step_bytes = scan_bytes + (flt.bytes(n, b, not args.unfused_filter, probed) if flt else 0)
        bound = "hbm" if 2 * b < 625 else "mfma"  # int8 ridge: 625 OP/B
        dtype = "int8"
        data = ("synthetic: per-row int8 of N(0,1) float32 rows (torch generator seeds 1234 / "
                "99)" + ("; attributes Zipf(1.1) (seed 4321), query sets numpy seed 77"
                         if flt else ""))
        workload = f"int8 scan top-{k}: N={n} D={d} B={b}"
        if flt:
            workload = (f"filtered int8 top-{k}: N={n} D={d} B={b}; Bloom {BLOOM_BITS} bits/item, "
                        f"{BLOOM_K} hashes pre-filter + exact AND-of-OR clause post-check over 8 "
                        f"attributes at {args.selectivity:.0%} target selectivity"
                        + ("; the clause mask written before the scan" if args.unfused_filter
                           else "; the Bloom search's mask, the clauses checked inside the scan"
                           if args.bloom_search else
                           "; the Bloom plans probed and the clauses checked inside the scan, "
                           "per candidate"))
            extra["measured_selectivity"] = float(flt.selectivity.mean())
        metric = ("queries/sec + achieved HBM GB/s, filtered top-100 over 30Mx512 int8 items"
                  if flt else "queries/sec + achieved HBM GB/s, int8 top-100 over 30Mx512 items")

        def cpu_fn():
            from oracle import baseline

            ns = min(args.cpu_sample or 2_000_000, n)
            valid_fn = flt.valid_fn(ns) if flt else None
            t_s, threads = baseline.time_int8(queries.cpu(), items[:ns].cpu(), k,
                                              valid_fn=valid_fn)
            what = "torch.mm over 2M-row chunks + topk + lowest-id merge"
            if flt:
                what = "the exact value-set filter (torch.isin) gating " + what
            return t_s * (n / ns), threads, f"B={b} queries x first {ns} of {n} items ({what})"

    elif wl == "filtered-dense":
        log(f"generating {n}x{d} clustered items (1024 centres) and {b} queries")
        gen = torch.Generator(device=dev).manual_seed(2024)
        centres = torch.randn((1024, d), generator=gen, device=dev)
        items = dense_table(n, d, centres, 2025, dev).bfloat16()
        queries = dense_table(b, d, centres, 2026, dev).bfloat16()
        flt = Filter(n, b, args.selectivity, dev)
        blocked = retrieve_amd.hip._use_blocked(b, 2 * d, k)

        def step():
            if args.unfused_filter:
                return torch.ops.retrieve_amd.dense_scan_topk(queries, items, k, flt.mask())
            # (the blocked scan of a large batch reads the transposed words directly)
            words = flt.bloom_t() if blocked else flt.bloom()
            return torch.ops.retrieve_amd.dense_scan_topk_clauses(queries, items, k, flt.attrs,
                                                             flt.rev, flt.sets, words)

        scan_bytes = n * d * 2 + b * d * 2
        table = items  # the streamed table (the read ceiling is measured over it)
        scan_ops = 2 * b * n * d
        step_bytes = scan_bytes + flt.bytes(n, b, not args.unfused_filter)
        bound = "hbm" if b < 312 else "mfma"  # bf16 ridge: 312.5 FLOP/B
        dtype = "bf16"
        data = ("synthetic: 1024 N(0,1) centres (seed 2024), items centre + 0.3 N(0,1) "
                "L2-normalised (seed 2025), queries likewise (seed 2026), stored bf16; attributes "
                "Zipf(1.1) (seed 4321), query sets numpy seed 77")
        workload = (f"filtered dense bf16 top-{k}: N={n} D={d} B={b}; Bloom {BLOOM_BITS} "
                    f"bits/item, {BLOOM_K} hashes pre-filter + exact AND-of-OR clause post-check "
                    f"over 8 attributes at {args.selectivity:.0%} target selectivity"
                    + ("; the clause mask written before the scan" if args.unfused_filter
                       else "; the clauses checked inside the scan"))
        extra["measured_selectivity"] = float(flt.selectivity.mean())
        metric = "queries/sec + achieved HBM GB/s, filtered bf16 top-100 over 10Mx128 items"

        def cpu_fn():
            from oracle import baseline

            ns = min(args.cpu_sample or 1_000_000, n)
            t_s, threads = baseline.time_topk(queries.cpu().float(), items[:ns].cpu().float(), k,
                                              valid_fn=flt.valid_fn(ns))
            return (t_s * (n / ns), threads,
                    f"B={b} queries x first {ns} of {n} items (the exact value-set filter "
                    "(torch.isin) gating float32 torch.mm over 2M-row chunks + topk + lowest-id "
                    "merge)")

    elif wl == "exact":
        log(f"generating {n}x{d} and {b}x{d} N(0,1) rows, L2-normalised, fp32")
        gen = torch.Generator(device=dev).manual_seed(11)
        items = torch.randn((n, d), generator=gen, device=dev)
        items = items / items.norm(dim=1, keepdim=True)
        queries = torch.randn((b, d), generator=gen, device=dev)
        queries = queries / queries.norm(dim=1, keepdim=True)

        def step():
            return torch.ops.retrieve_amd.dense_scan_topk(queries, items, k)

        # recall@k against torch's own fp32 product and top-k on the GPU (ties aside, the same)
        torch.backends.cuda.matmul.allow_tf32 = False
        ref = torch.topk(queries @ items.t(), k, dim=1).indices
        got = step()[0]
        extra["recall_at_k_vs_fp32"] = (
            (got.unsqueeze(2) == ref.unsqueeze(1)).any(2).sum().item() / (b * k))
        scan_bytes = n * d * 4 + b * d * 4
        table = items  # the streamed table (the read ceiling is measured over it)
        scan_ops = 2 * b * n * d
        step_bytes = scan_bytes
        bound = "fp32"
        dtype = "fp32"
        data = ("synthetic: N(0,1) rows and queries, L2-normalised (torch generator seed 11), "
                "fp32")
        workload = f"exact fp32 inner-product top-{k}: N={n} D={d} B={b} (configuration 1)"
        metric = "queries/sec, exact fp32 top-100 over 100kx128 items"

        def cpu_fn():
            from oracle import baseline

            t_s, threads = baseline.time_topk(queries.cpu(), items.cpu(), k)
            return (t_s, threads, f"B={b} queries x all {n} items (float32 torch.mm + topk + "
                    "lowest-id merge), full size")

    elif wl == "dense":
        log(f"generating {n}x{d} clustered items (1024 centres) and {b} queries")
        gen = torch.Generator(device=dev).manual_seed(2024)
        centres = torch.randn((1024, d), generator=gen, device=dev)
        items32 = dense_table(n, d, centres, 2025, dev)
        q32 = dense_table(b, d, centres, 2026, dev)
        items = items32.bfloat16()
        queries = q32.bfloat16()

        def step():
            return torch.ops.retrieve_amd.dense_scan_topk(queries, items, k)

        # recall@k against exact float32 scoring of the unrounded rows (chunked torch.mm)
        torch.backends.cuda.matmul.allow_tf32 = False
        best_s = torch.full((b, k), float("-inf"), device=dev)
        best_i = torch.full((b, k), -1, dtype=torch.int64, device=dev)
        for s0 in range(0, n, 1 << 21):
            sc = q32 @ items32[s0 : s0 + (1 << 21)].t()
            top = torch.topk(sc, min(k, sc.shape[1]), dim=1)
            cs = torch.cat([best_s, top.values], 1)
            ci = torch.cat([best_i, top.indices + s0], 1)
            t2 = torch.topk(cs, k, dim=1)
            best_s, best_i = t2.values, ci.gather(1, t2.indices)
        got = step()[0]
        hits = (got.unsqueeze(2) == best_i.unsqueeze(1)).any(2).sum().item()
        extra["recall_at_k_vs_fp32"] = hits / (b * k)
        log(f"recall@{k} vs exact fp32: {extra['recall_at_k_vs_fp32']:.4f}")
        # the same with fp16 storage (the reference module's dtype), outside the timed region
        items_h = items32.half()
        del items32
        got = torch.ops.retrieve_amd.dense_scan_topk(q32.half(), items_h, k)[0]
        hits = (got.unsqueeze(2) == best_i.unsqueeze(1)).any(2).sum().item()
        extra["recall_at_k_vs_fp32_fp16_storage"] = hits / (b * k)
        log(f"recall@{k} vs exact fp32, fp16 storage: "
            f"{extra['recall_at_k_vs_fp32_fp16_storage']:.4f}")
        del items_h

        scan_bytes = n * d * 2 + b * d * 2
        table = items  # the streamed table (the read ceiling is measured over it)
        scan_ops = 2 * b * n * d
        step_bytes = scan_bytes
        bound = "hbm" if b < 312 else "mfma"  # bf16 ridge: 312.5 FLOP/B
        dtype = "bf16"
        data = ("synthetic: 1024 N(0,1) centres (seed 2024), items centre + 0.3 N(0,1) "
                "L2-normalised (seed 2025), queries likewise (seed 2026), stored bf16")
        workload = f"dense bf16 top-{k}: N={n} D={d} B={b} (clustered, L2-normalised)"
        metric = "queries/sec + achieved HBM GB/s, bf16 top-100 over 10Mx128 items"

        def cpu_fn():
            from oracle import baseline

            ns = min(args.cpu_sample or 1_000_000, n)
            t_s, threads = baseline.time_topk(queries.cpu().float(), items[:ns].cpu().float(), k)
            return (t_s * (n / ns), threads,
                    f"B={b} queries x first {ns} of {n} items (float32 torch.mm over 2M-row "
                    "chunks + topk + lowest-id merge)")

    elif wl == "hamming":
        log(f"generating {n} SimHash codes ({d} bits), {b} queries")
        gen = torch.Generator(device=dev).manual_seed(555)
        proj = torch.randn((d, d), generator=gen, device=dev)
        item_bits, _ = simhash_tables(n, d, proj, 556, dev, with_codes=False)
        q_bits, _ = simhash_tables(b, d, proj, 557, dev, with_codes=False)

        def step():
            return torch.ops.retrieve_amd.hamming_scan_topk(q_bits, item_bits, k)

        scan_bytes = n * d // 8 + b * d // 8
        step_bytes = scan_bytes
        table = item_bits  # the streamed table (the read ceiling is measured over it)
        # 512-bit codes are scored on the fp4 matrix cores (2 ops per bit, item and query);
        # other widths by XOR + popcount. The fp4 ridge is 10.1 PFLOP/s / 8 TB/s = 1262 ops a
        # byte, 2 b d / (d / 8) = 16 b: HBM-bound up to 78 queries.
        scan_ops = 2 * b * n * d
        bound = "mfma" if d == 512 and 16 * b >= 1262 else "hbm"
        dtype = "fp4" if d == 512 else "u64"
        data = ("synthetic: N(0,1) rows (seed 556) and queries (seed 557), SimHash over a "
                "N(0,1) 512x512 projection (seed 555)")
        workload = f"1-bit Hamming top-{k}: N={n} bits={d} B={b}"
        metric = "queries/sec + achieved HBM GB/s, 1-bit Hamming top-k over 30M 512-bit codes"

        def cpu_fn():
            from oracle import baseline

            ns = min(args.cpu_sample or 1_000_000, n)
            t0 = time.perf_counter()
            baseline.hamming_topk_cpu(q_bits.cpu().numpy(), item_bits[:ns].cpu().numpy(), k)
            t_s = time.perf_counter() - t0
            return (t_s * (n / ns), 1,
                    f"B={b} queries x first {ns} of {n} items (numpy XOR + bitwise_count in "
                    "32K-item chunks, top-k by (score, id)), one run, scaled")

    else:  # binary
        k1 = 1000
        log(f"generating {n} SimHash codes ({d} bits) + int8 rerank codes, {b} queries")
        gen = torch.Generator(device=dev).manual_seed(555)
        proj = torch.randn((d, d), generator=gen, device=dev)
        item_bits, item_codes = simhash_tables(n, d, proj, 556, dev)
        q_bits, q_codes = simhash_tables(b, d, proj, 557, dev)
        flt = Filter(n, b, args.selectivity, dev)

        # the 1-bit stage pads a row past its candidates with -1, which the candidate scan skips
        # (ids outside the table are never read): each row's count is the full width
        full_counts = torch.full((b,), k1, dtype=torch.int64, device=dev)

        def step():
            ids1, _ = torch.ops.retrieve_amd.hamming_scan_topk_clauses(
                q_bits, item_bits, k1, flt.attrs, flt.rev, flt.sets,
                flt.bloom_t() if b >= 8 and k1 <= 1024 else flt.bloom(),
                fused=not args.unfused_bits)
            return torch.ops.retrieve_amd.int8_candidates_topk(q_codes, item_codes, ids1,
                                                               full_counts, k)

        scan_bytes = n * d // 8 + b * d // 8
        table = item_bits  # the streamed table (the read ceiling is measured over it)
        # 512-bit codes from 8 queries on are scored on the fp4 matrix cores, one multiply-add
        # per bit (bits as {0, 1.0} and {-2.0, +2.0} e2m1 values): 2 ops per bit, item and query
        mfma_scan = d == 512 and b >= 8
        scan_ops = 2 * b * n * d if mfma_scan else 2 * b * n * (d // 32)
        step_bytes = scan_bytes + flt.bytes(n, b, not args.unfused_bits) + b * k1 * d
        bound = "mfma" if mfma_scan else "hbm"
        dtype = "fp4" if mfma_scan else "u64"
        data = ("synthetic: N(0,1) rows (seed 556) and queries (seed 557), SimHash over a "
                "N(0,1) 512x512 projection (seed 555), int8 codes of the same rows; attributes "
                "Zipf(1.1) (seed 4321), query sets numpy seed 77")
        workload = (f"binary top-{k1} + int8 rerank top-{k}: N={n} bits={d} B={b}; Bloom + exact "
                    f"filter at {args.selectivity:.0%} target selectivity"
                    + ("; the clause mask written before the scan" if args.unfused_bits
                       else "; the clauses checked inside the scan"))
        extra["measured_selectivity"] = float(flt.selectivity.mean())
        metric = ("queries/sec + achieved HBM GB/s, filtered 1-bit top-1000 + int8 rerank "
                  "top-100 over 30M items")

        def cpu_fn():
            from oracle import baseline

            ns = min(args.cpu_sample or 200_000, n)
            valid = flt.valid_fn(ns)(0, ns).numpy()
            t0 = time.perf_counter()
            baseline.hamming_rerank_cpu(q_bits.cpu().numpy(), q_codes.cpu().numpy(),
                                        item_bits[:ns].cpu().numpy(),
                                        item_codes[:ns].cpu().numpy(), k1, k, valid)
            t_s = time.perf_counter() - t0
            return (t_s * (n / ns), 1,
                    f"B={b} queries x first {ns} of {n} items (numpy XOR + bitwise_count in "
                    "32K-item chunks, exact filter, top-1000 by (score, id), int8 re-rank of "
                    "the candidates), one run, scaled")

    torch.cuda.synchronize()
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
    eager_step = step

    lib = _native.lib()
    total_ms = ctypes.c_double()
    launches = ctypes.c_int64()
    if args.mode == "graph":
        # the timed steps are calls of the compiled step, one graph launch each (the reference
        # harness's gate); the main scan's HIP-event time comes from as many eager steps right
        # after (events are not recorded inside the graph)
        log("compiling the step: torch.compile(mode='reduce-overhead', fullgraph=True)")
        compiled = graph_callable(step)

        def step():
            with torch.inference_mode():
                return compiled()

        for _ in range(max(args.warmup, 3)):  # the compiled calls' own first-call costs
            step()
        torch.cuda.synchronize()
        log(f"timing {args.steps} compiled calls")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        _native.check(lib.rt_profile_enable(1))
        for _ in range(args.steps):
            eager_step()
        torch.cuda.synchronize()
    else:
        _native.check(lib.rt_profile_enable(1))
        log(f"timing {args.steps} steps")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    _native.check(lib.rt_profile_collect(ctypes.byref(total_ms), ctypes.byref(launches)))
    _native.check(lib.rt_profile_enable(0))
    extra["mode"] = args.mode
    ms_step = wall * 1e3 / args.steps
    kernel_ms = total_ms.value / max(1, launches.value)
    if bound == "hbm":
        achieved = scan_bytes / (kernel_ms * 1e-3) / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    elif bound == "fp32":
        # fp32 FMAs on the vector units, priced against MI355X's fp32 matrix peak
        achieved = scan_ops / (kernel_ms * 1e-3) / 1e12
        peak, unit = 157.3, "TFLOP/s"
        bound = "mfma"
    else:
        achieved = scan_ops / (kernel_ms * 1e-3) / 1e12
        peak = {"int8": 5000.0, "bf16": 2500.0, "fp4": 10100.0}[dtype]  # dense MFMA peaks
        unit = "TFLOP/s"
    log(f"ms/step {ms_step:.3f}; main scan {kernel_ms:.3f} ms ({achieved:.0f} {unit})")
    if bound == "mfma" and dtype in ("int8", "bf16"):
        # what the matrix cores sustain on random operands at the clock they hold under that
        # load (register-fed chains, no memory traffic): context for the spec-peak fraction
        rate, mhz = ctypes.c_double(), ctypes.c_double()
        _native.check(lib.rt_mfma_ceiling(0 if dtype == "int8" else 1, 200_000,
                                          ctypes.byref(rate), ctypes.byref(mhz), None))
        extra["mfma_sustained_random_operands"] = {
            "value": rate.value / 1e12, "unit": unit, "clock_mhz": mhz.value,
            "main_scan_frac_of_it": achieved / (rate.value / 1e12),
        }
        log(f"matrix cores sustain {rate.value / 1e12:.0f} {unit} at {mhz.value:.0f} MHz")
    if bound == "hbm":
        # what one plain streaming kernel reads over the same table: the practical ceiling the
        # scan's HBM fraction is to be read against
        rate = ctypes.c_double()
        _native.check(lib.rt_read_ceiling(table.data_ptr(), table.numel() * table.element_size(),
                                          5, ctypes.byref(rate), None))
        extra["hbm_read_ceiling"] = {"value": rate.value / 1e9, "unit": "GB/s",
                                     "main_scan_frac_of_it": achieved / (rate.value / 1e9)}
        log(f"a plain streaming read of the table: {rate.value / 1e9:.0f} GB/s")
    if args.windows > 0:
        rec = latency_windows(step, args.windows, args.window_calls, b, args.mode)
        extra["latency"] = {k: rec[k] for k in ("mode", "n", "windows", "median_ms", "p95_ms",
                                                "p99_ms", "qps", "spread")}
        if args.jsonl:
            rec.update(workload=wl, n_items=n, d=d, k=k, dtype=dtype)
            with open(args.jsonl, "a") as f:
                f.write(json.dumps(rec) + "\n")
    if wl == "binary":
        extra["hamming_path"] = ("fp4 matrix cores (bits as e2m1 nibbles)" if bound == "mfma"
                                 else "XOR + popcount")
        extra["hamming_hbm_gbs"] = scan_bytes / (kernel_ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        log("cpu baseline")
        t_full, threads, sample = cpu_fn()
        cpu = {
            "value": b / t_full,
            "unit": "queries/s",
            "cores": threads,
            "kind": "port",
            "sample": sample + f"; host has {os.cpu_count()} logical CPUs",
        }

    traffic = MEASURED_TRAFFIC.get((wl, n, d, b, k))
    line = {
        "metric": metric,
        "value": b * args.steps / wall,
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": data,
        "config": {
            "workload": workload,
            "global_batch": b,
            "main_kernel_ms": kernel_ms,
            "achieved_hbm_gbs_whole_step": step_bytes / (ms_step * 1e-3) / 1e9,
            **extra,
        },
        "roofline": {
            "bound": bound,
            "achieved": achieved,
            "peak": peak,
            "unit": unit,
            "frac": achieved / peak,
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
