"""Full-prefill block selection timings in milliseconds, per provider.

    python -m nlogn_pisa_amd.benchmark [--lengths 4096 ... 262144] [--head-dims 64 128]
                                       [--providers fused q4 bsa] [--output-dir DIR]

The reference's selection benchmark (``pisa/benchmarks/flash_sparse_attn/
top_k_pyramid/benchmark.py:13-150``) on this library: B=1, Hq=32, Hkv=2, bf16,
block 64, Top-K 8, method ``pisa`` (LSE), forced first + 2 recent blocks, fresh
summaries in every call (pooling included), no attention.  Providers:

* ``fused``: per-query routing with the leaf scored inline (``routing_schedule="fused"``);
* ``q1``/``q2``/``q4``: the grouped (block-major) leaf; this library's tiles hold up to
  256 requests of one key block whatever ``leaf_tile`` is, so the three are one kernel
  sequence and are timed once each for the table's sake;
* ``bsa``: flat BSA routing (``bsa_fn``).

Inputs are ``torch.randn`` from a CPU generator seeded 2024 (the reference seeds the
CUDA generator, whose stream this device cannot reproduce).  Each sample is one call
bracketed by HIP events after a 512 MiB buffer write that evicts the L2 and the
Infinity Cache, as ``triton.testing.do_bench`` flushes its L2; the mean over the
samples is reported.  Results go to ``selection.json`` / ``selection.csv``.
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import sys
from pathlib import Path

PROVIDERS = {
    "fused": "Direct-LSE fused",
    "q1": "Direct-LSE Q1",
    "q2": "Direct-LSE Q2",
    "q4": "Direct-LSE Q4",
    "bsa": "BSA Top-K",
}
LENGTHS = [4096, 8192, 16384, 32768, 65536, 131072, 262144]

# The reference's routing_latency_scaling figure (assets/figures/), values read off
# the plot (about +-1 ms), on an unstated NVIDIA GPU; D = 64.
REFERENCE_FIGURE_MS = {
    "q4": {65536: 6.7, 131072: 14.4, 262144: 31.0},
    "fused": {65536: 8.6, 131072: 18.7, 262144: 41.0},
    "bsa": {65536: 19.0, 131072: 77.0, 262144: 313.0},
}


def make_call(P, q, k, provider):
    if provider == "bsa":
        return lambda: P.bsa_fn(q, k, block_size=64, topk=8, backend="triton")
    schedule = "fused" if provider == "fused" else "grouped"
    tile = 4 if provider == "fused" else int(provider[1:])
    return lambda: P.select_blocks(q, k, method="pisa", block_size=64, topk=8, backend="triton",
                                   force_first=True, force_recent=2, routing_schedule=schedule,
                                   leaf_tile=tile)


def time_call(torch, run, warmup_ms, rep_ms, flush):
    """Mean milliseconds of ``run`` over samples that each start with cold caches."""
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    flush.zero_()
    start.record()
    run()
    stop.record()
    torch.cuda.synchronize()
    estimate = max(start.elapsed_time(stop), 1e-3)
    warm = max(1, int(warmup_ms / estimate))
    reps = max(3, int(rep_ms / estimate))
    for _ in range(warm):
        run()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(reps)]
    for a, b in pairs:
        flush.zero_()
        a.record()
        run()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in pairs) / reps


def length_label(length):
    return f"{length // 1024}K" if length % 1024 == 0 else str(length)


def save_results(directory, metadata, rows, providers):
    directory.mkdir(parents=True, exist_ok=True)
    (directory / "selection.json").write_text(
        json.dumps({"metadata": metadata, "rows": rows}, indent=2) + "\n")
    with (directory / "selection.csv").open("w", newline="") as stream:
        writer = csv.writer(stream)
        writer.writerow(["head_dim", "length"] + [PROVIDERS[p] + " (ms)" for p in providers])
        for row in rows:
            writer.writerow([row["head_dim"], row["length"]] +
                            [row["timings_ms"][p] for p in providers])


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--lengths", type=int, nargs="+", default=LENGTHS)
    parser.add_argument("--head-dims", type=int, nargs="+", choices=[64, 128], default=[64])
    parser.add_argument("--providers", nargs="+", choices=list(PROVIDERS), default=list(PROVIDERS))
    parser.add_argument("--warmup-ms", type=float, default=10)
    parser.add_argument("--rep-ms", type=float, default=30)
    parser.add_argument("--output-dir", type=Path, default=Path("stat/block-selection"))
    args = parser.parse_args(argv)
    if min(args.lengths) < 1 or not math.isfinite(args.warmup_ms) or args.warmup_ms < 0:
        parser.error("lengths must be positive and warmup-ms must be finite and nonnegative")
    if not math.isfinite(args.rep_ms) or args.rep_ms <= 0:
        parser.error("rep-ms must be finite and positive")

    import torch
    import nlogn_pisa_amd as P

    if not torch.cuda.is_available():
        parser.error("a ROCm GPU is required")
    P._lib.library()
    metadata = {
        "gpu": torch.cuda.get_device_name(), "torch": torch.__version__, "hip": torch.version.hip,
        "batch_size": 1, "query_heads": 32, "key_heads": 2, "dtype": "bfloat16",
        "block_size": 64, "topk": 8, "seed": 2024, "force_first": True, "force_recent": 2,
        "lengths": args.lengths, "head_dims": args.head_dims, "providers": args.providers,
        "warmup_ms": args.warmup_ms, "rep_ms": args.rep_ms,
        "timer": "HIP events per call, mean, 512 MiB cache flush between samples",
        "scope": "fresh summaries and full-prefill selection; no attention or backward",
        "reference_figure_ms": REFERENCE_FIGURE_MS,
    }
    print(f"GPU: {metadata['gpu']} | BF16 | B=1, Hq=32, Hkv=2, C=64, K=8", flush=True)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    rows, failed = [], False
    with torch.no_grad():
        for dimension in args.head_dims:
            print(f"\nblock-selection-d{dimension} (ms):", flush=True)
            print(f"{'n':>10}" + "".join(f"  {PROVIDERS[p]:>16}" for p in args.providers),
                  flush=True)
            for length in args.lengths:
                row = {"head_dim": dimension, "length": length, "timings_ms": {}, "errors": {}}
                gen = torch.Generator().manual_seed(2024)
                q = torch.randn(1, length, 32, dimension, generator=gen).to("cuda", torch.bfloat16)
                k = torch.randn(1, length, 2, dimension, generator=gen).to("cuda", torch.bfloat16)
                for provider in args.providers:
                    print(f"  D={dimension} N={length_label(length)} {PROVIDERS[provider]}",
                          file=sys.stderr, flush=True)
                    try:
                        run = make_call(P, q, k, provider)
                        run()
                        torch.cuda.synchronize()
                        row["timings_ms"][provider] = time_call(torch, run, args.warmup_ms,
                                                                args.rep_ms, flush)
                    except Exception as error:  # reported per provider, as the reference does
                        failed = True
                        row["timings_ms"][provider] = "ERROR"
                        row["errors"][provider] = str(error)
                        print(f"  {type(error).__name__}: {error}", file=sys.stderr, flush=True)
                cells = [f"{v:.4f}" if isinstance(v, float) else v
                         for v in row["timings_ms"].values()]
                print(f"{length:10d}" + "".join(f"  {v:>16}" for v in cells), flush=True)
                rows.append(row)
                save_results(args.output_dir, metadata, rows, args.providers)
                del q, k
                torch.cuda.empty_cache()
    print(f"\nResults: {args.output_dir.resolve()}", flush=True)
    return int(failed)


if __name__ == "__main__":
    sys.exit(main())
