"""Block-selection latency sweep: the reference's selection benchmark on this library.

    python -m nlogn_pisa_amd.benchmark [--lengths 4096 ... 262144] [--head-dims 64 128]
                                       [--providers fused q4 bsa] [--output-dir DIR]

Workload of ``pisa/benchmarks/flash_sparse_attn/top_k_pyramid/benchmark.py``:
B = 1, Hq = 32, Hkv = 2, bf16, block 64, Top-K 8, method ``pisa`` (LSE),
forced first + 2 recent blocks, the pyramid rebuilt in every call, no attention.
The provider keys, their labels and the output files (``selection.json`` with
``metadata`` and ``rows`` of ``head_dim``/``length``/``timings_ms``/``errors``,
``selection.csv`` with a "<label> (ms)" column per provider) follow the
reference so its plotting reads them unchanged.  Providers:

* ``fused``: per-query routing with the leaf scored inline (``routing_schedule="fused"``);
* ``q1``/``q2``/``q4``: the grouped (block-major) leaf.  This library's tiles hold up to
  256 requests of one key block whatever ``leaf_tile`` is, so the three run one kernel
  sequence; each is timed for the table's sake;
* ``bsa``: flat BSA routing (``bsa_fn``).

Inputs: ``torch.randn`` from a CPU generator seeded 2024 (the reference seeds the
CUDA generator, whose stream this device does not reproduce).  A sample is one call
between two HIP events, preceded by a 512 MiB buffer write that evicts the L2 and the
Infinity Cache (the reference's ``do_bench`` flushes its L2); the mean is reported.
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import sys
from dataclasses import dataclass, field
from pathlib import Path

PROVIDERS = {
    "fused": "Direct-LSE fused",
    "q1": "Direct-LSE Q1",
    "q2": "Direct-LSE Q2",
    "q4": "Direct-LSE Q4",
    "bsa": "BSA Top-K",
}
LENGTHS = [4096, 8192, 16384, 32768, 65536, 131072, 262144]
SHAPE = dict(batch=1, query_heads=32, key_heads=2, block_size=64, topk=8, force_first=True,
             force_recent=2, seed=2024)

# The reference's routing_latency_scaling figure (assets/figures/), values read off
# the plot (about +-1 ms), on an unstated NVIDIA GPU; D = 64.
REFERENCE_FIGURE_MS = {
    "q4": {65536: 6.7, 131072: 14.4, 262144: 31.0},
    "fused": {65536: 8.6, 131072: 18.7, 262144: 41.0},
    "bsa": {65536: 19.0, 131072: 77.0, 262144: 313.0},
}


def selection_call(P, q, k, provider):
    """The operator call a provider key stands for (a closure over q and k)."""
    common = dict(block_size=SHAPE["block_size"], topk=SHAPE["topk"], backend="triton")
    if provider == "bsa":
        return lambda: P.bsa_fn(q, k, **common)
    grouped = provider != "fused"
    return lambda: P.select_blocks(q, k, method="pisa", force_first=SHAPE["force_first"],
                                   force_recent=SHAPE["force_recent"],
                                   routing_schedule="grouped" if grouped else "fused",
                                   leaf_tile=int(provider[1:]) if grouped else 4, **common)


class ColdTimer:
    """Mean HIP-event milliseconds of a call, every sample after a cache-evicting write."""

    def __init__(self, torch, warmup_ms, rep_ms, flush_bytes=512 << 20):
        self.torch = torch
        self.warmup_ms, self.rep_ms = warmup_ms, rep_ms
        self.flush = torch.empty(flush_bytes, dtype=torch.uint8, device="cuda")

    def _events(self, n):
        make = lambda: self.torch.cuda.Event(enable_timing=True)
        return [(make(), make()) for _ in range(n)]

    def _samples(self, run, n, cold=True):
        marks = self._events(n)
        for begin, end in marks:
            if cold:
                self.flush.zero_()
            begin.record()
            run()
            end.record()
        self.torch.cuda.synchronize()
        return [begin.elapsed_time(end) for begin, end in marks]

    def __call__(self, run):
        first = max(self._samples(run, 1)[0], 1e-3)          # sizes the warmup and the reps
        self._samples(run, max(1, int(self.warmup_ms / first)), cold=False)
        times = self._samples(run, max(3, int(self.rep_ms / first)))
        return sum(times) / len(times)


def length_label(length):
    return f"{length // 1024}K" if length % 1024 == 0 else str(length)


@dataclass
class Results:
    """Rows of the sweep and the two files they are written to after each length."""

    directory: Path
    metadata: dict
    providers: list
    rows: list = field(default_factory=list)

    def add(self, head_dim, length, timings, errors):
        self.rows.append({"head_dim": head_dim, "length": length, "timings_ms": timings,
                          "errors": errors})
        self.write()

    def write(self):
        self.directory.mkdir(parents=True, exist_ok=True)
        payload = {"metadata": self.metadata, "rows": self.rows}
        (self.directory / "selection.json").write_text(json.dumps(payload, indent=2) + "\n")
        columns = ["head_dim", "length"] + [f"{PROVIDERS[p]} (ms)" for p in self.providers]
        with (self.directory / "selection.csv").open("w", newline="") as handle:
            out = csv.writer(handle)
            out.writerow(columns)
            out.writerows([r["head_dim"], r["length"], *(r["timings_ms"][p] for p in self.providers)]
                          for r in self.rows)


def _arguments(argv):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--lengths", type=int, nargs="+", default=LENGTHS)
    ap.add_argument("--head-dims", type=int, nargs="+", choices=[64, 128], default=[64])
    ap.add_argument("--providers", nargs="+", choices=list(PROVIDERS), default=list(PROVIDERS))
    ap.add_argument("--warmup-ms", type=float, default=10)
    ap.add_argument("--rep-ms", type=float, default=30)
    ap.add_argument("--output-dir", type=Path, default=Path("stat/block-selection"))
    args = ap.parse_args(argv)
    problems = []
    if min(args.lengths) < 1:
        problems.append("every length must be at least 1")
    if not (math.isfinite(args.warmup_ms) and args.warmup_ms >= 0):
        problems.append("--warmup-ms must be a finite number >= 0")
    if not (math.isfinite(args.rep_ms) and args.rep_ms > 0):
        problems.append("--rep-ms must be a finite number > 0")
    if problems:
        ap.error("; ".join(problems))
    return ap, args


def _inputs(torch, length, dim):
    gen = torch.Generator().manual_seed(SHAPE["seed"])
    shape_q = (SHAPE["batch"], length, SHAPE["query_heads"], dim)
    shape_k = (SHAPE["batch"], length, SHAPE["key_heads"], dim)
    return tuple(torch.randn(s, generator=gen).to("cuda", torch.bfloat16) for s in (shape_q, shape_k))


def main(argv=None):
    ap, args = _arguments(argv)
    import torch
    import nlogn_pisa_amd as P

    if not torch.cuda.is_available():
        ap.error("a ROCm GPU is required")
    P._lib.library()
    metadata = {"gpu": torch.cuda.get_device_name(), "torch": torch.__version__,
                "hip": torch.version.hip, "batch_size": SHAPE["batch"],
                "query_heads": SHAPE["query_heads"], "key_heads": SHAPE["key_heads"],
                "dtype": "bfloat16", "block_size": SHAPE["block_size"], "topk": SHAPE["topk"],
                "seed": SHAPE["seed"], "force_first": SHAPE["force_first"],
                "force_recent": SHAPE["force_recent"], "lengths": args.lengths,
                "head_dims": args.head_dims, "providers": args.providers,
                "warmup_ms": args.warmup_ms, "rep_ms": args.rep_ms,
                "timer": "HIP events per call, mean, 512 MiB cache flush between samples",
                "scope": "fresh summaries and full-prefill selection; no attention or backward",
                "reference_figure_ms": REFERENCE_FIGURE_MS}
    results = Results(args.output_dir, metadata, list(args.providers))
    timer = ColdTimer(torch, args.warmup_ms, args.rep_ms)
    print(f"{metadata['gpu']}: bf16, B=1, Hq=32, Hkv=2, C=64, K=8, mean ms", flush=True)
    any_failed = False
    with torch.no_grad():
        for dim in args.head_dims:
            print(f"\nD = {dim}\n{'tokens':>10}" +
                  "".join(f"  {PROVIDERS[p]:>16}" for p in args.providers), flush=True)
            for length in args.lengths:
                q, k = _inputs(torch, length, dim)
                timings, errors = {}, {}
                for provider in args.providers:
                    print(f"  D={dim} N={length_label(length)} {PROVIDERS[provider]}",
                          file=sys.stderr, flush=True)
                    try:
                        run = selection_call(P, q, k, provider)
                        run()                                  # first call outside the timer
                        torch.cuda.synchronize()
                        timings[provider] = timer(run)
                    except Exception as error:                 # recorded per provider
                        any_failed = True
                        timings[provider], errors[provider] = "ERROR", str(error)
                        print(f"  {type(error).__name__}: {error}", file=sys.stderr, flush=True)
                shown = [f"{t:.4f}" if isinstance(t, float) else t for t in timings.values()]
                print(f"{length:10d}" + "".join(f"  {s:>16}" for s in shown), flush=True)
                results.add(dim, length, timings, errors)
                del q, k
                torch.cuda.empty_cache()
    print(f"\nResults: {args.output_dir.resolve()}", flush=True)
    return int(any_failed)


if __name__ == "__main__":
    sys.exit(main())
