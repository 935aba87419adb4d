"""Write golden vectors from the reference's Torch selection path.

Run ONCE, in the build container only, with the reference checkout on disk:

    PYTHONPATH=/root/reference/pisa python tests/golden/make_golden.py

It imports ``pisa`` (Aphelios-Tang/NlogN_PISA, ``pisa/pisa``) and records, as
plain arrays in ``tests/golden/*.npz``:

* ``network_topk.npz``: inputs/outputs of ``network_topk``
  (``top_k_pyramid_torch.py:84-110``) on score vectors full of exact ties
  (the sentinels 1e9 / 0 / -1e9 and repeated values) - the tie order of the
  comparison network is fixed by nothing but the reference itself;
* ``select_b2.npz``: end-to-end ids of ``select_blocks(..., backend="torch")``
  (``top_k_pyramid.py:11-121`` -> ``pyramid_select``, ``top_k_pyramid_torch.py:137-177``)
  at branching 2 and depth >= 2, including slot order, for pisa/pisa1/pisa2,
  fp32 and bf16 inputs, tails, decode offsets and force policies, plus the
  per-level selected ids for a few tokens recorded by replaying the loop with
  the reference's own helpers (``routing_masks``, ``block_scores``,
  ``network_topk``).

Nothing else runs the reference: pooling and attention are pinned by closed
forms in ``tests/test_oracle.py``.  The fixtures are data only; the GPU box
never reads ``/root/reference``.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def structured_inputs(gen, batch, length, qh, kh, dim, dtype, block=16):
    q = torch.randn(batch, length, qh, dim, generator=gen)
    noise = torch.randn(batch, length, kh, dim, generator=gen)
    off = 0.5 * torch.randn(batch, (length + block - 1) // block, kh, dim, generator=gen)
    k = noise + off.repeat_interleave(block, 1)[:, :length]
    return q.to(dtype), k.to(dtype)


def network_cases(network_topk):
    gen = torch.Generator().manual_seed(7)
    cases = []
    for width, topk in [(8, 4), (16, 8), (24, 8), (32, 8), (32, 16), (64, 16), (64, 32),
                        (128, 32), (128, 64), (256, 64), (100, 16)]:
        rows = 64
        palette = torch.tensor([1e9, 0.0, -1e9, 0.5, -0.25, 3.0], dtype=torch.float32)
        choice = torch.randint(0, palette.numel(), (rows, width), generator=gen)
        scores = palette[choice]
        # half the rows also carry distinct random scores in some lanes
        noise = torch.randn(rows, width, generator=gen)
        use = torch.rand(rows, width, generator=gen) < 0.3
        use[: rows // 2] = False
        scores = torch.where(use, noise, scores)
        ids = torch.arange(width).expand(rows, width).clone()
        ids = torch.where(torch.rand(rows, width, generator=gen) < 0.1, torch.full_like(ids, -1), ids)
        out = network_topk(scores, ids, topk)
        cases.append((width, topk, scores.numpy(), ids.numpy(), out.numpy()))
    return cases


def traced_select(q, k, method, block_size, topk, positions, force_first, force_recent, levels,
                  tokens, helpers):
    """Replay ``pyramid_select`` for ``tokens`` with the reference's helpers,
    recording the selected ids of every level."""
    routing_masks, block_scores, network_topk, routing_geometry = helpers
    heads = k.shape[2]
    batch = q.shape[0]
    top, first_width = routing_geometry(levels[0].shape[1], topk)
    levels = list(levels) + [levels[-1]] * max(0, top + 1 - len(levels))
    per_token = []
    for token in tokens:
        position = positions[:, token, None].expand(batch, heads)
        ids = torch.arange(first_width).expand(batch, heads, -1)
        record = []
        for level in range(top, -1, -1):
            total = levels[level].shape[1]
            ids = ids.masked_fill(ids >= total, -1)
            valid, forced, scoreable = routing_masks(ids, position, block_size, topk,
                                                     force_first, force_recent, level)
            if method == "pisa1":
                scoreable = valid & ~forced
                source, support, scale = levels[level], 1, 1.0
            else:
                source, support = (k, block_size) if level == 0 else (levels[level - 1], 2)
                scale = k.shape[-1] ** -0.5
            scores = torch.zeros_like(ids, dtype=torch.float32)
            if bool(scoreable.any()):
                scores = block_scores(q[:, token], source, ids.masked_fill(~scoreable, -1),
                                      support, method, scale)
            scores = scores.masked_fill(~scoreable, 0).masked_fill(~valid, -1e9).masked_fill(forced, 1e9)
            ids = network_topk(scores, ids, topk)
            record.append(ids.clone())
            if level:
                children = ids[..., None] * 2 + torch.arange(2)
                ids = children.masked_fill(ids[..., None] < 0, -1).flatten(-2)
        final = ids.masked_fill((ids < 0) | (ids * block_size > position[..., None]), -1)
        per_token.append((torch.stack(record, 2), final))
    return per_token


def main():
    from pisa.ops.flash_sparse_attn.top_k_pyramid import select_blocks
    from pisa.ops.flash_sparse_attn.top_k_pyramid.top_k_pyramid_torch import (
        block_scores, network_topk, routing_geometry, routing_masks)
    from pisa.utils.validation import query_positions

    helpers = (routing_masks, block_scores, network_topk, routing_geometry)
    arrays = {}
    for index, (width, topk, scores, ids, out) in enumerate(network_cases(network_topk)):
        arrays[f"c{index}_scores"] = scores
        arrays[f"c{index}_ids"] = ids.astype(np.int32)
        arrays[f"c{index}_topk"] = np.array(topk)
        arrays[f"c{index}_out"] = out.astype(np.int32)
    arrays["count"] = np.array(index + 1)
    np.savez_compressed(os.path.join(HERE, "network_topk.npz"), **arrays)

    shapes = [
        # name, batch, Tq, N, Hq, Hkv, D, C, offset
        ("prefill256", 1, 256, 256, 4, 2, 32, 16, None),
        ("tail1000", 2, 1000, 1000, 4, 1, 16, 16, None),
        ("gqa16", 1, 512, 512, 16, 1, 32, 16, None),
        ("decode", 2, 1, 1000, 4, 2, 32, 16, None),
        ("suffix", 1, 64, 777, 4, 2, 32, 16, 600),
    ]
    select = {}
    case = 0
    for s_index, (name, batch, tq, n, qh, kh, dim, block, offset) in enumerate(shapes):
        for dtype_name, dtype in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
            gen = torch.Generator().manual_seed(1000 + 10 * s_index + (dtype_name == "bf16"))
            qf, kf = structured_inputs(gen, batch, n, qh, kh, dim, dtype, block)
            q = qf[:, n - tq:] if offset is None else qf[:, offset:offset + tq]
            k = kf
            select[f"in{s_index}{dtype_name}_q"] = q.float().numpy()
            select[f"in{s_index}{dtype_name}_k"] = k.float().numpy()
            for method in ("pisa", "pisa1", "pisa2"):
                for topk in (4, 8):
                    for force_first, force_recent in ((True, 1), (True, 2), (False, 1)):
                        out = select_blocks(q, k, method=method, block_size=block, topk=topk,
                                            query_offset=offset, force_first=force_first,
                                            force_recent=force_recent, backend="torch")
                        key = f"s{case}"
                        select[key + "_meta"] = np.array(
                            [s_index, dtype_name == "bf16", ("pisa", "pisa1", "pisa2").index(method),
                             topk, force_first, force_recent, block, -1 if offset is None else offset],
                            dtype=np.int64)
                        select[key + "_out"] = out.numpy().astype(np.int16)
                        if topk == 4 and force_recent == 2:
                            from pisa.ops.compress.mean_pooling import build_pyramid
                            levels = build_pyramid(k, block, backend="torch")
                            positions = query_positions(q, k, offset)
                            tokens = list(range(0, tq, max(1, tq // 8)))[:8]
                            traced = traced_select(q, k, method, block, topk, positions,
                                                   force_first, force_recent, levels, tokens, helpers)
                            for (record, final), token in zip(traced, tokens):
                                assert torch.equal(final, out[:, token]), "replay differs"
                            select[key + "_trace_tokens"] = np.array(tokens)
                            select[key + "_trace"] = torch.stack(
                                [r for r, _ in traced], 1).numpy().astype(np.int16)
                        case += 1
    select["count"] = np.array(case)
    np.savez_compressed(os.path.join(HERE, "select_b2.npz"), **select)
    print("network cases", arrays["count"], "select cases", case)


if __name__ == "__main__":
    sys.exit(main())
