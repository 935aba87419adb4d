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


def midpoint_blocks(heads=1, starts=(0.1345, 0.3, 0.7, 1.5, 3.1, 0.07, 12.0, 0.02)):
    """fp16 keys [1, 128, heads, len(starts)] whose 128-row mean (per column) is an
    fp16 midpoint plus 2^-30: 126 rows of h (even last mantissa bit), one of
    2h + 64 ulp(h), one of 2^-23.  Rounded to float32 the mean is the midpoint,
    which rounds (half to even) to h; rounded straight to fp16 it is h + ulp(h).
    Returns (keys, h per column)."""
    cols, hs = [], []
    for x in starts:
        h = np.float16(x)
        if int(h.view(np.uint16)) & 1:
            h = np.nextafter(h, np.float16(np.inf))
        ulp = 2.0 ** (np.floor(np.log2(float(h))) - 10)
        cols.append([float(h)] * 126 + [2 * float(h) + 64 * ulp, 2.0 ** -23])
        hs.append(float(h))
    col = np.asarray(cols, dtype=np.float16).T.astype(np.float32)  # [128, columns]
    keys = np.broadcast_to(col[None, :, None, :], (1, 128, heads, len(starts))).copy()
    return keys, np.asarray(hs, dtype=np.float32)


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


def stratified_tokens(length, count, seed=0, low=0):
    """About ``count`` sorted query indices in [low, length): one uniform draw per
    equal stratum, plus the first and last index (identity region and the end)."""
    rng = np.random.default_rng(seed)
    edges = np.linspace(low, length, count + 1)
    picks = [int(rng.integers(int(a), max(int(a) + 1, int(b)))) for a, b in zip(edges[:-1], edges[1:])]
    return np.unique(np.clip(np.array(picks + [low, length - 1], dtype=np.int64), low, length - 1))


def selection_parity(qn, kn, ids, trace, tokens, method, block, topk, force_first, force_recent,
                     branching, levels, positions, geometry=None):
    """Compare GPU ids [B, Tq, H, K] (numpy, all tokens) on ``tokens`` with the oracle.

    ``trace`` is the GPU's per-level ids [B, Tq, H, L, K].  Returns a dict with
    the rows compared, mismatched rows, tie-exempt rows and the failing rows
    (batch-major row index, kv head, diverging level).
    """
    expected, otrace = O.pyramid_select(qn, kn, method, block, topk, positions, force_first,
                                        force_recent, levels, branching=branching, tokens=tokens,
                                        trace=True, geometry=geometry)
    got = ids[:, tokens]
    heads = got.shape[2]
    rows = got.shape[0] * got.shape[1] * heads
    if np.array_equal(got, expected):
        return {"rows": rows, "mismatched": 0, "exempt": 0, "failures": [], "expected": expected}
    gtrace = trace[:, tokens]
    _, mism, exempt, failures = adjudicate(
        got.reshape(-1, heads, got.shape[-1]), gtrace.reshape(-1, heads, *gtrace.shape[-2:]),
        expected.reshape(-1, heads, got.shape[-1]), otrace)
    return {"rows": rows, "mismatched": mism, "exempt": exempt, "failures": failures,
            "expected": expected}


def needle_recall(qn, kn, selected, tokens, needles, block, topk, force_first, force_recent,
                  positions):
    """Needle blocks ranked inside the top ``topk - |forced|`` of the exhaustive leaf
    log-sum-exp (summed over the query heads, forced blocks excluded) that the
    selection ``selected`` [B, len(tokens), Hkv, K] contains: (hits, total)."""
    batch, _, query_heads, dim = qn.shape
    heads = kn.shape[2]
    groups = query_heads // heads
    scale = dim ** -0.5
    hits = total = 0
    for b, h, ids in needles:
        planted = set(int(x) for x in ids)
        query = qn[b, tokens, h * groups:(h + 1) * groups].reshape(-1, dim).astype(np.float64)
        keys = kn[b, :, h].astype(np.float64)
        n = keys.shape[0]
        blocks = -(-n // block)
        logits = np.full((len(tokens) * groups, blocks * block), -np.inf)
        logits[:, :n] = query @ keys.T * scale
        logits = logits.reshape(len(tokens), groups, blocks, block)
        peak = logits.max(-1, keepdims=True)
        lse = (peak[..., 0] + np.log(np.exp(logits - peak).sum(-1))).sum(1)   # [tokens, blocks]
        for i, t in enumerate(tokens):
            pos = int(positions[b, t])
            current = pos // block
            excluded = set(range(max(0, current - force_recent + 1), current + 1))
            if force_first:
                excluded.add(0)
            cand = np.array([j for j in range(current + 1) if j not in excluded])
            if cand.size == 0:
                continue
            best = cand[np.argsort(-lse[i, cand], kind="stable")[:topk - len(excluded)]]
            must = planted.intersection(best.tolist())
            chosen = set(selected[b, i, h].tolist())
            hits += len(must & chosen)
            total += len(must)
    return hits, total


def torch_sparse_attention(q, k, v, indices, block, positions, dout=None, scale=None, chunk=256):
    """Float32 restatement of ``sparse_attn_torch.py:6-35`` on the tensors' device.

    Returns (O, LSE) and, when ``dout`` is given, (dQ, dK, dV) from the closed-form
    gradients (dV = P^T dO, dS = P (dO V^T - rowsum(dO O)), dQ = s dS K,
    dK = s dS^T Q), scattered back through the gathers.  Chunks of ``chunk`` query
    tokens bound the gathered keys.
    """
    batch, length, query_heads, dim = q.shape
    n, heads = k.shape[1], k.shape[2]
    groups = query_heads // heads
    scale = dim ** -0.5 if scale is None else scale
    dev = q.device
    k32, v32 = k.float(), v.float()
    out = torch.zeros(batch, length, query_heads, v.shape[-1], device=dev)
    lse = torch.full((batch, length, query_heads), -float("inf"), device=dev)
    grads = None
    if dout is not None:
        grads = (torch.zeros(batch, length, query_heads, dim, device=dev),
                 torch.zeros(batch, n, heads, dim, device=dev),
                 torch.zeros(batch, n, heads, v.shape[-1], device=dev))
    offs = torch.arange(block, device=dev)
    b_ids = torch.arange(batch, device=dev)[:, None, None, None]
    h_ids = torch.arange(heads, device=dev)[None, None, :, None]
    for s in range(0, length, chunk):
        e = min(length, s + chunk)
        ids = indices[:, s:e].long()
        tok = (ids[..., None] * block + offs).flatten(-2)                     # [B,t,H,S]
        valid = (ids[..., None] >= 0).expand(*ids.shape, block).flatten(-2)
        valid &= (tok >= 0) & (tok < n) & (tok <= positions[:, s:e, None, None])
        tok = tok.clamp(0, n - 1)
        bb = b_ids.expand_as(tok)
        hh = h_ids.expand_as(tok)
        keys = k32[bb, tok, hh]                                                # [B,t,H,S,D]
        vals = v32[bb, tok, hh]
        query = q[:, s:e].float().reshape(batch, e - s, heads, groups, dim)
        logits = torch.matmul(query, keys.transpose(-1, -2).contiguous()) * scale
        mask = valid[:, :, :, None, :]
        logits = logits.masked_fill(~mask, -float("inf"))
        peak = logits.amax(-1, keepdim=True)
        safe = torch.where(torch.isfinite(peak), peak, torch.zeros_like(peak))
        w = torch.exp(logits - safe).masked_fill(~mask, 0.0)
        den = w.sum(-1, keepdim=True)
        prob = w / torch.where(den > 0, den, torch.ones_like(den))
        o = torch.matmul(prob, vals)                                           # [B,t,H,G,Dv]
        out[:, s:e] = o.reshape(batch, e - s, query_heads, -1)
        row_lse = torch.where(den[..., 0] > 0, safe[..., 0] + torch.log(den[..., 0]),
                              torch.full_like(den[..., 0], -float("inf")))
        lse[:, s:e] = row_lse.reshape(batch, e - s, query_heads)
        if dout is None:
            continue
        do = dout[:, s:e].float().reshape(batch, e - s, heads, groups, -1)
        dprob = torch.matmul(do, vals.transpose(-1, -2).contiguous())
        delta = (do * o).sum(-1, keepdim=True)
        dlog = prob * (dprob - delta)
        grads[0][:, s:e] = (torch.matmul(dlog, keys) * scale).reshape(batch, e - s, query_heads, dim)
        dkeys = torch.matmul(dlog.transpose(-1, -2).contiguous(), query) * scale   # [B,t,H,S,D]
        dvals = torch.matmul(prob.transpose(-1, -2).contiguous(), do)
        sel = valid
        grads[1].index_put_((bb[sel], tok[sel], hh[sel]), dkeys[sel], accumulate=True)
        grads[2].index_put_((bb[sel], tok[sel], hh[sel]), dvals[sel], accumulate=True)
    return (out, lse) if dout is None else (out, lse, *grads)
