"""Deterministic synthetic workloads of the benchmark configurations.

Each configuration is a selection + attention problem: shapes, selection
parameters and the input recipe (q, v ~ N(0,1); k = N(0,1) plus a per-64-token
offset ~ N(0, 0.5^2); optional 'needle' blocks whose offset is ~ N(0, 2^2)).
Inputs are drawn with a seeded CPU ``torch.Generator`` (seed 2024 + 1000*cfg;
per-sequence seeds for decode) so every box sees identical data.
"""

from __future__ import annotations

import concurrent.futures
import math
import os
from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    tokens: int            # query tokens per sequence
    keys: int              # key tokens per sequence
    query_heads: int
    key_heads: int
    head_dim: int
    block_size: int
    branching: int
    topk: int
    method: str
    force_first: bool
    force_recent: int
    dtype: torch.dtype
    needles: float = 0.0
    seed: int = 2024
    per_sequence_seed: bool = False
    grad: bool = False
    extra: dict = field(default_factory=dict)


def config(index: int, tokens: int | None = None) -> Workload:
    """The benchmark configuration ``index`` (0-4); ``tokens`` picks config 4's length."""
    if index == 0:
        return Workload("cfg0-T4096-fp32", 1, 4096, 4096, 4, 4, 64, 64, 4, 8, "pisa", True, 1,
                        torch.float32, seed=2024)
    if index == 1:
        return Workload("cfg1-B4-T16384-bf16", 4, 16384, 16384, 16, 4, 128, 64, 4, 16, "pisa", True,
                        1, torch.bfloat16, seed=3024, grad=True)
    if index == 2:
        return Workload("cfg2-T65536-bf16", 1, 65536, 65536, 32, 8, 128, 64, 4, 32, "pisa2", True, 2,
                        torch.bfloat16, needles=0.01, seed=4024)
    if index == 3:
        return Workload("cfg3-decode-B32-N131072-bf16", 32, 1, 131072, 32, 8, 128, 64, 4, 32, "pisa",
                        True, 1, torch.bfloat16, needles=0.01, seed=5024, per_sequence_seed=True)
    if index == 4:
        t = 65536 if tokens is None else tokens
        return Workload(f"cfg4-T{t}-bf16", 1, t, t, 16, 2, 128, 128, 8, 16, "pisa", True, 1,
                        torch.bfloat16, seed=6024)
    raise ValueError(f"unknown configuration {index}")


def _sequence(gen, w: Workload, batch: int, first_block_excluded: bool, last_excluded: bool,
              needles: list | None = None):
    q = torch.randn(batch, w.tokens, w.query_heads, w.head_dim, generator=gen)
    noise = torch.randn(batch, w.keys, w.key_heads, w.head_dim, generator=gen)
    blocks = math.ceil(w.keys / 64)
    off = 0.5 * torch.randn(batch, blocks, w.key_heads, w.head_dim, generator=gen)
    if w.needles:
        count = math.ceil(w.needles * blocks)
        low = 1 if first_block_excluded else 0
        high = blocks - (1 if last_excluded else 0)
        for b in range(batch):
            for h in range(w.key_heads):
                ids = torch.randperm(high - low, generator=gen)[:count] + low
                off[b, ids, h] = 2.0 * torch.randn(count, w.head_dim, generator=gen)
                if needles is not None:
                    needles.append((b, h, sorted(ids.tolist())))
    k = noise + off.repeat_interleave(64, 1)[:, :w.keys]
    v = torch.randn(batch, w.keys, w.key_heads, w.head_dim, generator=gen)
    return q, k, v


def make_inputs(w: Workload, device="cuda", needles: list | None = None):
    """(q, k, v[, dO]) of workload ``w`` in its dtype on ``device``.

    ``needles``, when a list, receives one ``(batch, kv_head, [block ids])``
    entry per sequence and kv head naming the planted needle blocks.
    """
    if w.per_sequence_seed:
        # every sequence has its own generator, so they are drawn concurrently
        def draw(b):
            gen = torch.Generator("cpu").manual_seed(w.seed + b)
            found = []
            q, k, v = _sequence(gen, w, 1, True, True, found)
            return [x.to(w.dtype) for x in (q, k, v)], [(b, h, ids) for _, h, ids in found]

        workers = max(1, min(16, os.cpu_count() or 1, w.batch))
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            drawn = list(pool.map(draw, range(w.batch)))
        if needles is not None:
            for _, found in drawn:
                needles.extend(found)
        return tuple(torch.cat([part[i].to(device) for part, _ in drawn], 0) for i in range(3))
    gen = torch.Generator("cpu").manual_seed(w.seed)
    q, k, v = _sequence(gen, w, w.batch, True, False, needles)
    out = [q, k, v]
    if w.grad:
        out.append(torch.randn(w.batch, w.tokens, w.query_heads, w.head_dim, generator=gen))
    return tuple(x.to(w.dtype).to(device) for x in out)
