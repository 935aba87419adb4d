"""Parity helpers for the GPU tests: input generators and tie adjudication.

A selected-id mismatch between the HIP path and the CPU oracle is exempt only
if, at the first level where the two networks kept different ids, every pair of
ids swapped between them has oracle scores closer than ``tol`` times the largest
real (non-sentinel) score magnitude of that row and level.  Every other
mismatch counts as a failure.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle as O

TORCH_DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def structured_qkv(seed, batch, length, qh, kh, dim, dtype="fp32", offset_block=64, needles=0.0,
                   value=True, tq=None):
    """q, k (, v) as float32 numpy arrays exactly representable in ``dtype``.

    q ~ N(0,1); k = N(0,1) + a per-``offset_block`` offset ~ N(0, 0.5^2); a
    fraction ``needles`` of the blocks (never block 0) gets an N(0, 2^2) offset.
    """
    rng = np.random.default_rng(seed)
    tq = length if tq is None else tq
    q = rng.standard_normal((batch, tq, qh, dim)).astype(np.float32)
    noise = rng.standard_normal((batch, length, kh, dim)).astype(np.float32)
    blocks = -(-length // offset_block)
    off = 0.5 * rng.standard_normal((batch, blocks, kh, dim)).astype(np.float32)
    if needles:
        count = max(1, int(np.ceil(needles * blocks)))
        for b in range(batch):
            for h in range(kh):
                ids = rng.permutation(np.arange(1, blocks))[:count]
                off[b, ids, h] = 2.0 * rng.standard_normal((count, dim))
    k = noise + np.repeat(off, offset_block, 1)[:, :length]
    arrays = [q, k]
    if value:
        arrays.append(rng.standard_normal((batch, length, kh, dim)).astype(np.float32))
    return [O.round_storage(x, dtype) for x in arrays]


def to_gpu(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x)).to(TORCH_DTYPES[dtype]).cuda()


def half_ulp(ref, dtype):
    """Half a unit in the last place of ``ref`` in the output dtype (0 for fp32).

    A 16-bit output cannot be closer to a float64 reference than its own final
    rounding; the attention bar is applied to the difference beyond it.
    """
    if dtype == "fp32":
        return np.zeros_like(ref)
    mant = {"bf16": 7, "fp16": 10}[dtype]
    mag = np.maximum(np.abs(ref), 2.0 ** -14)
    return np.exp2(np.floor(np.log2(mag)) - mant) / 2


def excess_error(mine, ref, dtype):
    """max(|mine - ref| - half_ulp(ref)) over all elements."""
    return float((np.abs(mine - ref) - half_ulp(ref, dtype)).max())


def adjudicate(gpu_ids, gpu_trace, oracle_ids, oracle_trace, tol=1e-4):
    """Return (rows, mismatched, exempt, failures) for [R, H, K] ids.

    ``gpu_trace`` is [R, H, L, K] (levels top..0); ``oracle_trace`` the list of
    per-level dicts of ``oracle.pyramid_select(..., trace=True)``.
    """
    rows = gpu_ids.shape[0] * gpu_ids.shape[1]
    bad = np.argwhere((gpu_ids != oracle_ids).any(-1))
    exempt, failures = 0, []
    for r, h in bad:
        verdict = None
        for j, entry in enumerate(oracle_trace):
            o_sel = entry["selected"][r, h]
            g_sel = gpu_trace[r, h, j]
            if np.array_equal(o_sel, g_sel):
                continue
            ids, scores = entry["ids"][r, h], entry["scores"][r, h]
            lookup = {}
            for i, s in zip(ids.tolist(), scores.tolist()):
                lookup.setdefault(i, s)
            real = np.abs(scores[(np.abs(scores) < 1e8) & (scores != 0)])
            scale = float(real.max()) if real.size else 0.0
            ok = scale > 0
            for a, b in zip(g_sel.tolist(), o_sel.tolist()):
                if a == b:
                    continue
                if a not in lookup or b not in lookup or \
                        abs(lookup[a] - lookup[b]) >= tol * scale:
                    ok = False
            verdict = ("exempt" if ok else "fail", j)
            break
        if verdict is None:
            verdict = ("fail", -1)       # final differs although every level agreed
        if verdict[0] == "exempt":
            exempt += 1
        else:
            failures.append((int(r), int(h), verdict[1]))
    return rows, len(bad), exempt, failures


def adjudicate_flat(got, want, scores, ids, tol=1e-4):
    """Flat (BSA) selections: (rows that differ, exempt rows, failing rows).

    ``scores``/``ids`` are the oracle's per-block scores and ids [..., M] of each
    row (``oracle.bsa_scores``).  A differing row is exempt when, slot by slot,
    the oracle scores of the two ids (0 for the -1 padding, as the network pads)
    are closer than ``tol`` times the row's largest score: the two selections
    then differ only by near-tied blocks trading places.
    """
    got = np.asarray(got).reshape(-1, got.shape[-1])
    want = np.asarray(want).reshape(-1, want.shape[-1])
    scores = np.asarray(scores).reshape(-1, scores.shape[-1])
    ids = np.asarray(ids).reshape(-1, ids.shape[-1])
    bad = np.flatnonzero((got != want).any(-1))
    exempt, failures = 0, []
    for r in bad:
        lookup = {-1: 0.0}
        for i, s in zip(ids[r].tolist(), scores[r].tolist()):
            if i >= 0:
                lookup[i] = s
        scale = float(np.abs(scores[r]).max())
        ok = scale > 0 and all(
            a in lookup and b in lookup and abs(lookup[a] - lookup[b]) < tol * scale
            for a, b in zip(got[r].tolist(), want[r].tolist()))
        if ok:
            exempt += 1
        else:
            failures.append(int(r))
    return len(bad), exempt, failures
