#!/usr/bin/env python
"""PISA 64K prefill on one MI355X: block selection + sparse attention forward.

    python bench.py [--gpus 1] [--steps 5] [--warmup 2] [--config 2] [--no-cpu-baseline]

One step = the hot path over one batch of synthetic input already resident in
HBM: ``select_blocks`` (pyramid build, coarse LSE/second-order routing, grouped
leaf scoring, final top-K) followed by ``sparse_attention_with_lse`` (O and LSE).
Prints ONE JSON line.  ``value`` is the selection latency (ms, lower is better),
the first number of the metric; the sparse-attention TFLOP/s and the roofline
fractions sit beside it.  The ``roofline`` object describes the kernel with the
largest share of the step, timed by HIP events recorded on its own stream
(``nlogn_pisa_amd._lib.profile_begin/end``): the attention forward against the
bf16 MFMA peak (4 D G flops per visible (row, key) pair), the selection kernels
against HBM.  ``cpu_baseline`` times the NumPy oracle (the reference's Torch
equations restated) on a bounded sample of the same workload - the selection of
1024 query tokens and the attention of eight 32-token chunks - on this host's
cores, extrapolated to the full sequence.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12          # bytes/s, MI355X HBM3E
MFMA_PEAK = {"bf16": 2.5e15, "fp16": 2.5e15, "fp32": 157.3e12}
TILE = 256                 # requests per bucketed tile (csrc/pisa_capi.hip)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--tokens", type=int, default=None, help="config 4 length")
    ap.add_argument("--cpu-sample", type=int, default=1024,
                    help="query tokens of the oracle's selection timed on the CPU")
    ap.add_argument("--cpu-chunks", type=int, default=8,
                    help="32-token chunks of the oracle's attention timed on the CPU")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--backward", action="store_true",
                    help="also time sparse attention forward + backward (a training step's attention)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device copy (calibrates rocprofv3 FETCH/WRITE_SIZE)")
    return ap.parse_args()


def copy_probe():
    """A plain copy of exactly 1 GiB, three times, for counter calibration."""
    import torch
    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": src.numel() * 4, "launches": 3}), flush=True)
    return 0


def copy_rate():
    """Bytes per second (read + written) of a plain 1 GiB device copy: the
    practical ceiling of a kernel that reads and writes HBM in equal parts."""
    import torch
    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    rate = 5 * 2 * src.numel() * 4 / (e0.elapsed_time(e1) * 1e-3)
    del src, dst
    torch.cuda.empty_cache()
    return rate


# ---------------------------------------------------------------- work counts

def query_window(tokens, row_bytes):
    """Query tokens per bucketing window (mirrors query_window in csrc/pisa_capi.hip)."""
    w = 256
    while w * 2 * max(row_bytes, 1) <= (128 << 20):
        w *= 2
    return max(1, min(w, tokens))


def leaf_span(w, elem):
    """Sibling blocks per grouped leaf request (mirrors leaf_span in csrc/pisa_leaf.hip):
    head groups of up to 4 and blocks of up to 64 keys take the largest power of two
    <= min(branching, 4) whose blocks fit 256 LDS rows and 80 KB; 16-bit 128-key blocks
    (head dims 64 and 128, groups up to 8, from 16384 row items) go in pairs."""
    G = w.query_heads // w.key_heads
    D = w.head_dim
    if w.method == "pisa1" or D not in (16, 32, 64, 128):
        return 1
    if w.block_size > 64:   # 128-key blocks: pairs, two waves per block (16-bit, G <= 8)
        ok = (elem == 2 and w.block_size == 128 and w.branching >= 2 and D in (64, 128) and G <= 8
              and w.batch * w.tokens * w.key_heads >= 16384)
        return 2 if ok else 1
    if G > 4:
        return 1
    E = 1 if elem == 4 else (8 if (D // 4) % 8 == 0 else 4)
    kq = 32 if E == 8 else 16
    cq = -(-w.block_size // kq) * kq
    ldk = D + 16 // elem
    span = 1
    while (span * 2 <= min(w.branching, 4) and span * 2 * cq <= 256
           and span * 2 * cq * ldk * elem + TILE * 16 <= 80 << 10):
        span *= 2
    return span


def grouped_schedule(w):
    """Whether the automatic schedule routes grouped (top_k_pyramid.py:64-72): pisa
    or pisa2 with more than one query token; otherwise the fused route scores
    every level, the leaf included, by gathering."""
    return w.method != "pisa1" and w.tokens > 1


def dense_levels(w, top, first):
    """Routing levels scored densely, {level: nodes} (mirrors route_level_dense in
    csrc/pisa_route.hip: padded head groups of 4 or 8, branching <= 8, a level whose
    nodes are at most (16 / Gp) x its candidate width)."""
    gp = 1 << (w.query_heads // w.key_heads - 1).bit_length()
    if not 4 <= gp <= 8 or w.branching > 8 or not grouped_schedule(w):   # fused routes gather
        return {}
    out, nodes = {}, math.ceil(w.keys / w.block_size)
    sizes = [nodes]
    while len(sizes) <= top:
        sizes.append(math.ceil(sizes[-1] / w.branching))
    for level in range(1, top + 1):
        width = first if level == top else w.branching * w.topk
        if sizes[level] <= (16 // gp) * width:
            out[level] = sizes[level]
    return out


def tile_count(w, valid, ids, elem, blocks=None):
    """Tiles of <= TILE requests per (batch, kv head, block) group, bucketed per
    window of query tokens over the flattened (batch, token) axis."""
    import torch
    blocks = math.ceil(w.keys / w.block_size) if blocks is None else blocks
    window = query_window(w.batch * w.tokens, w.query_heads * w.head_dim * elem)
    windows = math.ceil(w.batch * w.tokens / window)
    dev = ids.device
    b = torch.arange(w.batch, device=dev)[:, None, None, None]
    t = torch.arange(w.tokens, device=dev)[None, :, None, None]
    h = torch.arange(w.key_heads, device=dev)[None, None, :, None]
    win = (b * w.tokens + t) // window
    group = ((win * w.batch * w.key_heads + b * w.key_heads + h) * blocks + ids)[valid]
    per = torch.bincount(group, minlength=windows * w.batch * w.key_heads * blocks)
    return int(((per + TILE - 1) // TILE).sum())

# kernel names of the bench's timing keys in the rocprofv3 summaries under profiles/
PROFILED = {"attn_fwd": ("attn_fwd_tile_kernel",),
            "leaf": ("leaf_split_kernel", "leaf_tile_kernel"),
            "route": ("route_grouped_kernel",),
            "route_dense": ("route_dense_lds_kernel", "route_dense_kernel"),
            "attn_combine": ("attn_combine2_kernel", "attn_combine_kernel"), "final": ("final_kernel",)}


def profiled_traffic(kernel, workload):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 PMC summary
    of ``workload`` (profiles/<workload>_kernels.md: FETCH_SIZE and WRITE_SIZE per
    dispatch, scaled by a plain copy), or None when no summary covers it."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"{workload}_kernels.md")
    names = PROFILED.get(kernel)
    if not names or not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
        if len(cells) >= 5 and any(cells[0].startswith(n + "<") for n in names):
            try:
                return int(float(cells[4]) * 1e9)   # total GB per dispatch
            except ValueError:
                return None
    return None


def selection_counts(P, w, q, k, positions):
    """Exact scoreable request counts per level (from the per-level selections)."""
    import torch
    ids, trace = P.selection.select_blocks_traced(
        q, k, w.method, w.block_size, w.topk, force_first=w.force_first,
        force_recent=w.force_recent, branching=w.branching)
    blocks = math.ceil(w.keys / w.block_size)
    top, first = P.routing_geometry(blocks, w.topk, w.branching)
    _, lengths = P.pooling.pyramid_layout(w.keys, w.block_size, w.branching, top)
    lengths = lengths + [lengths[-1]] * (top + 1 - len(lengths))
    pos = positions[..., None, None].expand(w.batch, w.tokens, w.key_heads, 1)
    leaf = pos // w.block_size
    counts, tiles = {}, 0
    b = w.branching
    for j, level in enumerate(range(top, -1, -1)):
        if level == top:
            cand = torch.arange(first, device=q.device).expand(w.batch, w.tokens, w.key_heads, first)
        else:
            sel = trace[..., j - 1, :].long()
            cand = (sel[..., None] * b + torch.arange(b, device=q.device)).flatten(-2)
            cand = torch.where(sel.repeat_interleave(b, -1) < 0, -1, cand)
        cand = torch.where(cand >= lengths[level], -1, cand)
        span = b ** level
        valid = (cand >= 0) & (cand * (w.block_size * span) <= pos)
        forced = valid & (cand == 0) if w.force_first else torch.zeros_like(valid)
        for r in range(w.force_recent):
            target = leaf - r
            forced |= valid & (target >= 0) & (cand == torch.div(target.clamp(min=0), span,
                                                                  rounding_mode="floor"))
        scoreable = valid & ~forced
        if w.method != "pisa1":
            scoreable &= (valid.sum(-1, keepdim=True) > w.topk)
        counts[level] = int(scoreable.sum())
        if level == 0 and w.method != "pisa1":
            # requests: spans of sibling slots with a scoreable block, grouped by block // span
            span = leaf_span(w, q.element_size())
            shape = scoreable.shape[:-1] + (scoreable.shape[-1] // span, span)
            sc, cd = scoreable.reshape(shape), cand.reshape(shape)
            first_blk = torch.where(sc, cd, torch.iinfo(cd.dtype).max).min(-1).values
            live = sc.any(-1)
            counts["leaf_requests"] = int(live.sum())
            counts["leaf_span"] = span
            tiles = tile_count(w, live, torch.where(live, first_blk // span, 0),
                               q.element_size(), blocks=-(-math.ceil(w.keys / w.block_size) // span))
    return ids, counts, tiles, top, first


def attention_counts(w, ids, positions, elem):
    """(requests, tiles, visible (row, key) pairs per KV head) of the attention step."""
    import torch
    blocks = math.ceil(w.keys / w.block_size)
    pos = positions[..., None, None]
    vis = (ids >= 0) & (ids < blocks) & (ids * w.block_size <= pos)
    start = ids * w.block_size
    keys = torch.minimum(torch.minimum(torch.full_like(ids, w.block_size), w.keys - start),
                         pos - start + 1).clamp(min=0)
    pairs = int(torch.where(vis, keys, 0).sum())
    return int(vis.sum()), tile_count(w, vis, ids, elem), pairs


# ---------------------------------------------------------------- CPU baseline

def cpu_model():
    """The host CPU's model name (``lscpu``'s "Model name", read from /proc/cpuinfo)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, q, k, v, sample, chunks):
    """Time the NumPy oracle (the reference's Torch equations restated) on a bounded
    sample of the workload and extrapolate to the whole step.

    Selection: the full pyramid, then ``sample`` evenly spaced query tokens
    (``pyramid_select``, ``top_k_pyramid_torch.py:137-177``).  Attention: ``chunks``
    evenly spaced 32-token chunks of the same rows over the oracle's selected ids
    (``sparse_attention``, ``sparse_attn_torch.py:6-35``, float32 as the reference's
    CPU path computes).  Both per-token costs are scaled to every token.
    """
    import numpy as np
    import torch
    import oracle as O
    dtype = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[w.dtype]
    qn, kn, vn = (x.float().cpu().numpy() for x in (q, k, v))
    positions = O.query_positions(w.batch, w.tokens, w.keys)
    tokens = np.unique(np.linspace(0, w.tokens - 1, sample).astype(np.int64))
    t0 = time.perf_counter()
    levels = O.build_pyramid(kn, w.block_size, w.branching, None, dtype)
    t1 = time.perf_counter()
    O.pyramid_select(qn, kn, w.method, w.block_size, w.topk, positions, w.force_first,
                     w.force_recent, levels, branching=w.branching, tokens=tokens)
    t2 = time.perf_counter()
    starts = np.unique(np.linspace(0, max(0, w.tokens - 32), chunks).astype(np.int64))
    rows = np.unique(np.concatenate([np.arange(s, min(s + 32, w.tokens)) for s in starts]))
    ids = O.pyramid_select(qn, kn, w.method, w.block_size, w.topk, positions, w.force_first,
                           w.force_recent, levels, branching=w.branching, tokens=rows)
    t3 = time.perf_counter()
    O.sparse_attention(qn[:, rows], kn, vn, ids, w.block_size, positions=positions[:, rows],
                       compute=np.float32)
    t4 = time.perf_counter()
    per_token = (t2 - t1) / len(tokens)
    attn_per_token = (t4 - t3) / len(rows)
    sel_ms = 1e3 * ((t1 - t0) + per_token * w.tokens)
    blas = None
    try:
        from threadpoolctl import threadpool_info
        blas = max(int(x.get("num_threads", 1)) for x in threadpool_info()) or None
    except Exception:
        pass
    return {"value": round(sel_ms, 1), "unit": "ms", "cores": int(blas or 1), "kind": "port",
            "sample": (f"oracle (NumPy restatement of the reference's Torch path): pyramid over all "
                       f"keys ({1e3 * (t1 - t0):.0f} ms) + selection of {len(tokens)} evenly spaced "
                       f"of {w.tokens} query tokens ({1e3 * per_token:.2f} ms/token), and attention "
                       f"forward of {len(starts)} evenly spaced 32-token chunks ({len(rows)} rows, "
                       f"{1e3 * attn_per_token:.2f} ms/token), each extrapolated to all tokens; "
                       f"matrix products on the BLAS pool, element-wise work on one thread"),
            "selection_ms": round(sel_ms, 1),
            "attention_fwd_ms": round(1e3 * attn_per_token * w.tokens * w.batch, 1),
            "step_ms": round(sel_ms + 1e3 * attn_per_token * w.tokens * w.batch, 1),
            "cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "blas_threads": blas, "cpu_model": cpu_model()}


# ---------------------------------------------------------------- main

def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe()
    import torch
    import nlogn_pisa_amd as P
    from nlogn_pisa_amd import _lib
    from nlogn_pisa_amd.inputs import config, make_inputs

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    _lib.library()
    w = config(args.config, args.tokens)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    print(f"[bench] generating {w.name}", file=sys.stderr, flush=True)
    q, k, v = make_inputs(w, dev)[:3]
    positions = P.query_positions(q, k)
    dname = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[w.dtype]

    # Decode keeps the key pyramid in a PyramidCache that each generated token
    # appends to; the step reads it (its append is timed on its own below).
    decode = w.tokens == 1
    cache = (P.PyramidCache.from_keys(k, w.block_size, w.branching) if decode else None)

    def select():
        return P.select_blocks(q, k, method=w.method, block_size=w.block_size, topk=w.topk,
                               force_first=w.force_first, force_recent=w.force_recent,
                               backend="auto", branching=w.branching, pyramid=cache)

    def attend(ids):
        return P.sparse_attention_with_lse(q, k, v, ids, block_size=w.block_size)

    with torch.no_grad():
        print("[bench] warmup", file=sys.stderr, flush=True)
        for _ in range(args.warmup):
            attend(select())
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
        print("[bench] timed steps", file=sys.stderr, flush=True)
        torch.cuda.synchronize()
        wall0 = time.perf_counter()
        for m in marks:
            m[0].record(stream)
            ids = select()
            m[1].record(stream)
            attend(ids)
            m[2].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        sel_ms = sum(m[0].elapsed_time(m[1]) for m in marks) / args.steps
        att_ms = sum(m[1].elapsed_time(m[2]) for m in marks) / args.steps
        step_ms = sel_ms + att_ms

        append_ms = None
        if decode:
            print("[bench] pyramid cache append", file=sys.stderr, flush=True)
            del cache
            start = w.keys - args.warmup - args.steps
            grow = P.PyramidCache.from_keys(k[:, :start], w.block_size, w.branching)
            for n in range(start, start + args.warmup):
                grow.append(k[:, n:n + 1])
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for n in range(start + args.warmup, w.keys):
                grow.append(k[:, n:n + 1])
            t1.record(stream)
            torch.cuda.synchronize()
            append_ms = t0.elapsed_time(t1) / args.steps
            cache = grow
            del grow

        train_ms, train_kernels = None, {}
        if args.backward:
            print("[bench] attention forward + backward", file=sys.stderr, flush=True)
            ids = select()
            gen = torch.Generator(device="cpu").manual_seed(7)
            dout = torch.randn(q.shape[:3] + (v.shape[-1],), generator=gen).to(dev, q.dtype)
            leaves = [x.detach().requires_grad_(True) for x in (q, k, v)]

            def train():
                with torch.enable_grad():
                    out = P.sparse_attention(*leaves, ids, block_size=w.block_size)
                    out.backward(dout)
                for x in leaves:
                    x.grad = None

            for _ in range(args.warmup):
                train()
            torch.cuda.synchronize()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for _ in range(args.steps):
                train()
            t1.record(stream)
            torch.cuda.synchronize()
            train_ms = t0.elapsed_time(t1) / args.steps
            _lib.profile_begin()
            train()
            train_kernels = {n: round(total, 4) for n, (cnt, total) in _lib.profile_end().items()}

        print("[bench] kernel timing", file=sys.stderr, flush=True)
        _lib.profile_begin()
        for _ in range(2):
            attend(select())
        kernels = _lib.profile_end()
        per_step = {name: total / 2 for name, (n, total) in kernels.items()}
        launches = {name: n / 2 for name, (n, total) in kernels.items()}

        print("[bench] work counts", file=sys.stderr, flush=True)
        ids, counts, leaf_tiles, top, first = selection_counts(P, w, q, k, positions)
        requests, attn_tiles, pairs = attention_counts(w, ids, positions, q.element_size())

    e = q.element_size()
    pe = 4 if e == 4 else 2    # partial rows: fp16 for 16-bit inputs, fp32 for fp32
    G = w.query_heads // w.key_heads
    D = w.head_dim
    items = w.batch * w.tokens * w.key_heads
    width = first if top == 0 else w.branching * w.topk
    r_leaf = counts.get(0, 0)
    dense = dense_levels(w, top, first)
    # internal requests gathered by the route kernel; dense levels' scores are read
    r_int = sum(v for lvl, v in counts.items() if isinstance(lvl, int) and lvl > 0
                and lvl not in dense)
    r_dense = sum(v for lvl, v in counts.items() if isinstance(lvl, int) and lvl in dense)
    # nodes of each dense level the items can see (the dense kernels stop after the
    # node visible to their latest query): the sum over items of min(nodes, pos // span + 1)
    visible = {lvl: int(torch.clamp(positions // (w.branching ** lvl * w.block_size) + 1,
                                    max=n).sum()) * w.key_heads for lvl, n in dense.items()}
    span = counts.get("leaf_span", 1)
    r_span = counts.get("leaf_requests", r_leaf)
    # algorithmic bytes / flops per launch of each hot kernel
    # the fused route (decode, pisa1) also scores the leaf: raw key rows of each
    # scored candidate (leaf means for pisa1)
    fused_leaf = 0 if grouped_schedule(w) else r_leaf * (D * e if w.method == "pisa1"
                                                          else w.block_size * D * e)
    algo = {
        "route": {"bound": "hbm",
                  "bytes": w.batch * w.tokens * w.query_heads * D * e + r_int * w.branching * D * e
                  + r_dense * 4 + items * width * 5 + fused_leaf},
        # per dense level: the query rows, each wave's pass over the visible support
        # rows (16 items per wave), the visible nodes' scores written
        "route_dense": {"bound": "mfma",
                        "bytes": sum(w.batch * w.tokens * w.query_heads * D * e
                                     + v / 16 * w.branching * D * e + v * 4
                                     for v in visible.values()),
                        "flops": sum(2 * G * v * w.branching * D for v in visible.values())},
        "leaf": {"bound": "hbm",   # key spans per tile, q rows once per span request, scores
                 "bytes": leaf_tiles * span * w.block_size * D * e + r_span * (G * D * e + 4)
                 + r_leaf * 4,
                 "flops": 2 * r_leaf * w.block_size * D * G},
        "final": {"bound": "hbm", "bytes": items * (width * 9 + w.topk * 8)},
        # MFMA-bound: 4 D G flops per visible (row, key) pair; "bytes" is the design's own
        # traffic (K/V per tile, q rows and the fp16 partial row of every request)
        "attn_fwd": {"bound": "mfma",
                     "bytes": attn_tiles * 2 * w.block_size * D * e
                     + requests * G * (D * e + D * pe + 4),
                     "flops": 4 * D * G * pairs},
        "attn_combine": {"bound": "hbm",
                         "bytes": requests * G * (D * pe + 4) + items * G * (D * e + 4)},
        "pool": {"bound": "hbm", "bytes": w.batch * w.keys * w.key_heads * D * e},
    }
    # compulsory HBM bytes of the attention step: q, K, V once, O and LSE once
    attn_compulsory = (w.batch * w.tokens * w.query_heads * D * e
                       + 2 * w.batch * w.keys * w.key_heads * D * e
                       + w.batch * w.tokens * w.query_heads * (D * e + 4))
    # the dominant kernel: its algorithmic work per launch over its average launch
    # (windowed kernels launch once per window of query tokens)
    dominant = max((n for n in per_step if n in algo), key=per_step.get)
    n_launch = max(launches[dominant], 1)
    dom_ms = per_step[dominant] / n_launch
    info = algo[dominant]
    traffic = profiled_traffic(dominant, w.name)
    if info["bound"] == "mfma":
        achieved = info["flops"] / n_launch / (dom_ms * 1e-3)
        peak = MFMA_PEAK[dname]
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(achieved / 1e12, 2),
                    "peak": peak / 1e12, "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                    "traffic": traffic, "avg_launch_ms": round(dom_ms, 4),
                    "launches_per_step": n_launch,
                    "algorithmic_flops_per_launch": int(info["flops"] / n_launch),
                    "design_bytes_per_launch": int(info["bytes"] / n_launch),
                    "design_bytes_frac_hbm": round(info["bytes"] / n_launch / (dom_ms * 1e-3)
                                                   / HBM_PEAK, 4)}
        if dominant == "attn_fwd":
            comp = attn_compulsory / n_launch
            roofline["compulsory_bytes_per_launch"] = int(comp)
            roofline["traffic_over_compulsory"] = round(traffic / comp, 2) if traffic else None
            # the kernel's counted HBM traffic per second beside a plain copy's rate
            # (it reads q rows and writes its partial rows in about equal parts)
            copy = copy_rate()
            roofline["copy_rate_gbps"] = round(copy / 1e9, 1)
            if traffic:
                roofline["traffic_rate_gbps"] = round(traffic / (dom_ms * 1e-3) / 1e9, 1)
                roofline["traffic_frac_copy_rate"] = round(traffic / (dom_ms * 1e-3) / copy, 3)
    else:
        achieved = info["bytes"] / n_launch / (dom_ms * 1e-3)
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved / 1e9, 1),
                    "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                    "traffic": traffic, "avg_launch_ms": round(dom_ms, 4),
                    "launches_per_step": n_launch,
                    "algorithmic_bytes_per_launch": int(info["bytes"] / n_launch)}
    # selection bytes of the reference's Q4 schedule (grouping_triton.py, leaf_triton.py:63-232):
    # q rows once, internal candidates' child rows, candidates, one key block per tile of
    # four leaf requests plus each request's q rows and bookkeeping, the final network's reads
    q4_bytes = (w.batch * w.tokens * w.query_heads * D * e + r_int * w.branching * D * e
                + items * width * 4
                + math.ceil(r_leaf / 4) * w.block_size * D * e + r_leaf * (G * D * e + 24)
                + items * (width * 8 + w.topk * 4))
    gather_bytes = items * 2 * w.topk * w.block_size * D * e

    attn_flops = 4 * D * G * pairs
    leaf_ms = per_step.get("leaf", 0)
    sel_bytes = sum(algo[n]["bytes"] for n in ("pool", "route", "route_dense", "leaf", "final"))
    result = {
        "metric": "selection ms + sparse-attn TFLOP/s at 64K prefill; % HBM / % MFMA peak",
        "value": round(sel_ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": "synthetic (seeded q,k,v; k with per-64-token offsets and 1% needle blocks)",
        "config": {"workload": w.name, "batch": w.batch, "tokens": w.tokens,
                   "query_heads": w.query_heads, "kv_heads": w.key_heads, "head_dim": D,
                   "block_size": w.block_size, "branching": w.branching, "topk": w.topk,
                   "method": w.method, "forced": f"first + {w.force_recent} recent",
                   "step": "select_blocks + sparse_attention forward (O, LSE)"
                           + (" over a PyramidCache" if decode else "")},
        "selection_ms": round(sel_ms, 3),
        "sparse_attn_ms": round(att_ms, 3),
        "sparse_attn_tflops": round(attn_flops / (att_ms * 1e-3) / 1e12, 2),
        "sparse_attn_mfma_frac": round(attn_flops / (att_ms * 1e-3) / MFMA_PEAK[dname], 4),
        "selection_hbm_frac": round(sel_bytes / (sel_ms * 1e-3) / HBM_PEAK, 4),
        "leaf_hbm_frac": round(algo["leaf"]["bytes"] / (leaf_ms * 1e-3) / HBM_PEAK, 4)
        if leaf_ms else None,
        "selection_q4_model_hbm_frac": round(q4_bytes / (sel_ms * 1e-3) / HBM_PEAK, 4),
        "sparse_attn_gather_tbps": round(gather_bytes / (att_ms * 1e-3) / 1e12, 2),
        "kernel_ms_per_step": {n: round(t, 4) for n, t in sorted(per_step.items(),
                                                                  key=lambda x: -x[1])},
        "work": {"route_requests": r_int, "dense_route_requests": r_dense,
                 "dense_levels": dense, "leaf_requests": r_leaf, "leaf_span": span,
                 "leaf_span_requests": r_span, "leaf_tiles": leaf_tiles,
                 "attn_requests": requests, "attn_tiles": attn_tiles, "attn_pairs": pairs,
                 "attn_flops": attn_flops, "top": top, "first_width": first},
        "roofline": roofline,
        "wall_s_timed": round(wall, 3),
    }
    if append_ms is not None:
        result["pyramid_append_ms"] = round(append_ms, 4)
    if train_ms is not None:
        # forward 4 D G P flops, backward 10 D G P (S recomputed)
        result["attn_fwd_bwd_ms"] = round(train_ms, 3)
        result["attn_fwd_bwd_tflops"] = round(14 * D * G * pairs / (train_ms * 1e-3) / 1e12, 2)
        result["attn_fwd_bwd_kernel_ms"] = dict(sorted(train_kernels.items(), key=lambda x: -x[1]))
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(w, q, k, v, args.cpu_sample, args.cpu_chunks)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
