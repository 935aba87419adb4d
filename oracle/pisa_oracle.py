"""NumPy restatement of the reference's PISA selection and sparse attention.

TEST INFRASTRUCTURE ONLY: this module is the checker for the HIP library.  It
is imported by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` and by nothing in the product package.

Every function cites the reference file:line it restates (paths relative to
``pisa/pisa/`` of Aphelios-Tang/NlogN_PISA).  Two deliberate generalisations:

* ``branching`` (b) replaces the reference's hard-coded 2 at
  ``mean_pooling.py:51`` and ``top_k_pyramid_torch.py:128,162,174``; b=2 is the
  reference exactly.  ``force_mask`` shifts by ``level`` there, i.e. divides by
  2**level; the generalisation divides by b**level.
* pooled sums are exact (float64) before the single rounding to float32 and to
  the storage dtype; the reference sums in float32 (``mean_pooling_torch.py:10-13``)
  whose order-dependent last bits the GPU cannot reproduce.  The two agree up
  to one storage ulp on rare elements; on the reference's golden selections
  (``tests/golden/select_b2.npz``, ``tests/test_oracle.py``) the ids are equal.

Parity status of each function (what pins it) is listed in the module
docstring of ``tests/test_oracle.py``; none is "parity unpinned".
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "round_storage", "mean_pool", "build_pyramid", "routing_geometry", "force_mask",
    "routing_masks", "block_scores", "network_topk", "pyramid_select", "query_positions",
    "sparse_attention", "sparse_attention_dense", "sparse_attention_backward",
    "leaf_scores", "flops_visible", "rotary", "rotary_frequency", "bitonic_merge",
    "streaming_topk", "bsa_tile_width", "bsa_scores", "bsa_select", "SENTINEL_FORCED",
    "SENTINEL_INVALID",
]

SENTINEL_FORCED = np.float32(1.0e9)
SENTINEL_INVALID = np.float32(-1.0e9)


# --------------------------------------------------------------------------- dtypes

def round_storage(x, dtype):
    """Round float values to a storage dtype and return them as float32 (or float64).

    ``dtype`` is one of ``"fp32"``, ``"bf16"``, ``"fp16"``, ``"fp64"``.  bf16 uses
    round-to-nearest-even on the float32 bit pattern, as torch's ``.to(bfloat16)``.
    """
    if dtype == "fp64":
        return np.asarray(x, dtype=np.float64)
    x32 = np.asarray(x, dtype=np.float32)
    if dtype == "fp32":
        return x32.copy()
    if dtype == "fp16":
        return x32.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        bits = x32.view(np.uint32).astype(np.uint64)
        nan = np.isnan(x32)
        rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        out = rounded.view(np.float32).copy()
        out[nan] = np.float32("nan")
        return out
    raise ValueError(f"unknown storage dtype {dtype}")


# --------------------------------------------------------------------------- pyramid

def mean_pool(keys, size, dtype="fp32"):
    """Mean of each run of ``size`` rows over its valid count.

    Follows ``compress/mean_pooling/mean_pooling_torch.py:7-14``: blocks of
    ``size`` along axis 1, the tail block divides by ``N - j*size``, the result is
    cast to the storage dtype.  Sums are exact (float64).
    """
    keys = np.asarray(keys)
    batch, length, heads, dim = keys.shape
    blocks = (length + size - 1) // size
    padded = np.zeros((batch, blocks * size, heads, dim), dtype=np.float64)
    padded[:, :length] = keys
    sums = padded.reshape(batch, blocks, size, heads, dim).sum(2)
    counts = np.clip(length - np.arange(blocks) * size, 1, size).astype(np.float64)
    means = (sums / counts[None, :, None, None]).astype(np.float32)
    return round_storage(means, dtype)


def build_pyramid(keys, block_size, branching=2, max_level=None, dtype="fp32"):
    """Leaf means first, then means of ``branching`` children up to the root.

    Follows ``compress/mean_pooling/mean_pooling.py:45-52`` (b=2 there).
    """
    if max_level is not None and (not isinstance(max_level, int) or max_level < 0):
        raise ValueError("max_level must be a nonnegative integer or None")
    levels = [mean_pool(keys, block_size, dtype)]
    while levels[-1].shape[1] > 1 and (max_level is None or len(levels) <= max_level):
        levels.append(mean_pool(levels[-1], branching, dtype))
    return levels


def routing_geometry(blocks, topk, branching=2):
    """(top level, first network width); ``top_k_pyramid_torch.py:124-133``."""
    top = 0
    while blocks > topk:
        parent = (blocks + branching - 1) // branching
        if parent < topk or parent == blocks:
            break
        blocks = parent
        top += 1
    return top, max(16, 1 << (max(blocks, topk) - 1).bit_length())


# --------------------------------------------------------------------------- masks

def force_mask(ids, positions, block_size, force_first=True, force_recent=2, level=0, branching=2):
    """Required ids at ``level``; ``top_k_pyramid_torch.py:6-14``."""
    ids = np.asarray(ids)
    leaf = np.asarray(positions) // block_size
    result = np.zeros(ids.shape, dtype=bool)
    if force_first:
        result |= ids == 0
    span = branching ** level
    for recent in range(force_recent):
        target = leaf - recent
        result |= (target[..., None] >= 0) & (ids == (np.maximum(target, 0) // span)[..., None])
    return result & (ids >= 0)


def routing_masks(ids, positions, block_size, topk, force_first, force_recent, level=0,
                  branching=2):
    """valid / forced / scoreable; ``top_k_pyramid_torch.py:114-120``."""
    span = block_size * branching ** level
    valid = (ids >= 0) & (ids.astype(np.int64) * span <= positions[..., None])
    forced = force_mask(ids, positions, block_size, force_first, force_recent, level,
                        branching) & valid
    if bool((forced.sum(-1) > topk).any()):
        raise ValueError("topk is smaller than the number of required distinct blocks")
    identity = valid.sum(-1) <= topk
    return valid, forced, valid & ~forced & ~identity[..., None]


# --------------------------------------------------------------------------- scores

def _support_scores(products, mask, method, support, scale):
    """Per-head score of one candidate from its support products.

    ``products`` [..., S] are unscaled q.x products; restates the method branches
    of ``top_k_pyramid_torch.py:62-79``.
    """
    f32 = products.dtype
    scale_c = products.dtype.type(scale)
    if method == "pisa":
        z = np.where(mask, products * scale_c, -np.inf)
        peak = z.max(-1)
        safe = np.where(np.isfinite(peak), peak, 0).astype(f32)
        with np.errstate(divide="ignore"):
            total = np.where(mask, np.exp(z - safe[..., None]), 0).sum(-1)
            return (safe + np.log(total)).astype(f32)
    count = np.maximum(mask.sum(-1), 1).astype(f32)
    mean = np.where(mask, products, 0).sum(-1) / count
    score = scale_c * mean
    if method == "pisa2":
        if support == 2:
            z = np.where(mask, products * scale_c, 0)
            total = z.sum(-1)
            difference = z[..., 0] - z[..., 1]
            score = np.where(count == 2, f32.type(0.5) * total
                             + f32.type(0.125) * difference * difference, total)
        else:
            second = np.where(mask, products * products, 0).sum(-1) / count
            variance = np.maximum(second - mean * mean, 0)
            score = scale_c * mean + f32.type(0.5 * scale * scale) * variance
    return score.astype(f32)


def block_scores(query, source, ids, support, method, scale, compute=np.float32):
    """Scores of one query token per batch row; ``top_k_pyramid_torch.py:48-80``.

    ``query`` [B, Hq, D], ``source`` [B, M, H, D], ``ids`` [B, H, W] (-1 = skip).
    Returns float32 [B, H, W], summed over the query heads of each KV head.
    Entries whose support is empty are not meaningful (the caller overwrites
    them with sentinels, ``top_k_pyramid_torch.py:169-171``).
    """
    query = np.asarray(query)
    batch, query_heads, dim = query.shape
    heads, width = ids.shape[1], ids.shape[2]
    groups = query_heads // heads
    b, h, w = np.meshgrid(np.arange(batch), np.arange(heads), np.arange(width), indexing="ij")
    b, h, w = b.ravel(), h.ravel(), w.ravel()
    flat_ids = np.asarray(ids)[b, h, w]
    rows = query.reshape(batch, heads, groups, dim)[b, h]
    scores = _scores_for(rows, np.asarray(source), b, h, flat_ids, support, method, scale, compute)
    return scores.reshape(batch, heads, width)


def _scores_for(query, source, batch_ids, head_ids, ids, support, method, scale, compute):
    """Compacted ``block_scores``: one score per (row, head, candidate) triple.

    query [n, G, D]; source [B, M, H, D]; batch_ids, head_ids, ids [n].
    The support of candidate ``i`` is rows ``i*support + [0, support)`` of
    ``source`` (``top_k_pyramid_torch.py:52-56``), masked to ``< M``.
    """
    n = ids.shape[0]
    if n == 0:
        return np.zeros(0, dtype=np.float32)
    samples = ids[:, None].astype(np.int64) * support + np.arange(support)
    mask = (samples >= 0) & (samples < source.shape[1])
    values = source[batch_ids[:, None], np.clip(samples, 0, source.shape[1] - 1),
                    head_ids[:, None]].astype(compute)                    # [n, S, D]
    products = np.matmul(query.astype(compute), np.swapaxes(values, 1, 2))  # [n, G, S]
    per_head = _support_scores(products, np.broadcast_to(mask[:, None, :], products.shape),
                               method, support, scale)
    return per_head.sum(1).astype(np.float32)


# --------------------------------------------------------------------------- network

def network_topk(scores, ids, topk):
    """Descending bitonic network with its compare/exchange tie order.

    Restates ``top_k_pyramid_torch.py:84-110``: pad to a power of two with
    (-1e9, -1); for each stage ``group = 2**e`` (all-descending when it spans the
    whole width) and each distance from group/2 down to 1, lanes exchange iff
    ``(left > right) != descending``.  Returns ids of lanes [0, topk).
    """
    scores = np.asarray(scores)
    ids = np.asarray(ids)
    n = scores.shape[-1]
    width = 1 << (n - 1).bit_length()
    if width != n:
        pad = [(0, 0)] * (scores.ndim - 1) + [(0, width - n)]
        scores = np.pad(scores, pad, constant_values=SENTINEL_INVALID)
        ids = np.pad(ids, pad, constant_values=-1)
    lane = np.arange(width)
    for exponent in range(1, width.bit_length()):
        group = 1 << exponent
        descending = np.ones(width, bool) if group == width else (lane & group) != 0
        for shift in range(exponent - 1, -1, -1):
            distance = 1 << shift
            partner = lane ^ distance
            peer_score, peer_id = scores[..., partner], ids[..., partner]
            left = (lane & distance) == 0
            left_score = np.where(left, scores, peer_score)
            right_score = np.where(left, peer_score, scores)
            exchange = (left_score > right_score) != descending
            scores = np.where(exchange, peer_score, scores)
            ids = np.where(exchange, peer_id, ids)
    return ids[..., :topk]


# --------------------------------------------------------------------------- selection

def query_positions(batch, tq, n, query_offset=None):
    """Absolute query positions [B, Tq]; ``utils/validation.py:38-56``."""
    if query_offset is None or isinstance(query_offset, (int, np.integer)):
        offset = n - tq if query_offset is None else int(query_offset)
        if offset < 0 or offset + tq > n:
            raise ValueError("queries must refer to positions within their key sequence")
        return np.broadcast_to(np.arange(offset, offset + tq, dtype=np.int64), (batch, tq)).copy()
    offset = np.asarray(query_offset, dtype=np.int64).reshape(-1, 1)
    positions = np.broadcast_to(offset + np.arange(tq), (batch, tq)).copy()
    if (positions < 0).any() or (positions >= n).any():
        raise ValueError("queries must refer to positions within their key sequence")
    return positions


def pyramid_select(q, k, method, block_size, topk, positions, force_first, force_recent, levels,
                   branching=2, geometry=None, tokens=None, trace=False, compute=np.float32,
                   chunk_rows=None):
    """Coarse-to-fine selection; ``top_k_pyramid_torch.py:137-177``.

    Vectorised over (batch, token) rows instead of the reference's per-token
    loop; each row is independent so the result is the same.  ``tokens``
    restricts the work to a subset of query indices (sampled parity checks).
    Returns int64 ids [B, len(tokens), Hkv, topk] and, with ``trace=True``, a
    list of per-level dicts ``{"level", "ids", "scores", "selected"}`` whose
    arrays have leading shape [B*len(tokens), Hkv] (batch-major).
    """
    q = np.asarray(q)
    k = np.asarray(k)
    batch, length, query_heads, dim = q.shape
    heads = k.shape[2]
    groups = query_heads // heads
    if hasattr(levels, "levels"):
        levels = levels.levels
    top, first_width = geometry or routing_geometry(levels[0].shape[1], topk, branching)
    levels = list(levels) + [levels[-1]] * max(0, top + 1 - len(levels))
    tokens = np.arange(length) if tokens is None else np.asarray(tokens, dtype=np.int64)
    rows_b = np.repeat(np.arange(batch), len(tokens))
    rows_t = np.tile(tokens, batch)
    total_rows = rows_b.shape[0]
    positions = np.asarray(positions, dtype=np.int64)
    if chunk_rows is None:
        # bound the gathered support (rows x heads x W x C x D floats) to ~256 MB
        width = max(first_width, branching * topk)
        per_row = heads * width * max(block_size, branching) * dim * 4
        chunk_rows = max(1, int(256e6 // max(per_row, 1)))
    result = np.empty((total_rows, heads, topk), dtype=np.int64)
    traces = []
    for start in range(0, total_rows, chunk_rows):
        stop = min(total_rows, start + chunk_rows)
        bidx, tidx = rows_b[start:stop], rows_t[start:stop]
        n = stop - start
        position = np.broadcast_to(positions[bidx, tidx][:, None], (n, heads))
        query = q[bidx, tidx].reshape(n, heads, groups, dim)
        ids = np.broadcast_to(np.arange(first_width, dtype=np.int64), (n, heads, first_width)).copy()
        chunk_trace = []
        for level in range(top, -1, -1):
            total = levels[level].shape[1]
            ids = np.where(ids >= total, -1, ids)
            valid, forced, scoreable = routing_masks(ids, position, block_size, topk, force_first,
                                                     force_recent, level, branching)
            if method == "pisa1":
                scoreable = valid & ~forced
                source, support, scale = levels[level], 1, 1.0
            else:
                source, support = (k, block_size) if level == 0 else (levels[level - 1], branching)
                scale = dim ** -0.5
            scores = np.zeros(ids.shape, dtype=np.float32)
            if scoreable.any():
                r, h, w = np.nonzero(scoreable)
                scores[r, h, w] = _scores_for(query[r, h], source, bidx[r], h, ids[r, h, w],
                                              support, method, scale, compute)
            scores = np.where(scoreable, scores, np.float32(0))
            scores = np.where(valid, scores, SENTINEL_INVALID)
            scores = np.where(forced, SENTINEL_FORCED, scores).astype(np.float32)
            selected = network_topk(scores, ids, topk)
            if trace:
                chunk_trace.append({"level": level, "ids": ids.copy(), "scores": scores.copy(),
                                    "selected": selected.copy()})
            if level:
                children = selected[..., None] * branching + np.arange(branching)
                children = np.where(selected[..., None] < 0, -1, children)
                ids = children.reshape(n, heads, topk * branching)
            else:
                ids = selected
        final = np.where((ids < 0) | (ids * block_size > position[..., None]), -1, ids)
        result[start:stop] = final
        if trace:
            traces.append(chunk_trace)
    out = result.reshape(batch, len(tokens), heads, topk)
    if not trace:
        return out
    merged = []
    for index in range(len(traces[0]) if traces else 0):
        merged.append({key: (traces[0][index][key] if key == "level" else
                             np.concatenate([t[index][key] for t in traces], 0))
                       for key in ("level", "ids", "scores", "selected")})
    return out, merged


def leaf_scores(q, k, candidates, block_size, method, positions, topk, force_first, force_recent,
                leaf_means=None, compute=np.float32):
    """Leaf scores with the shape of ``candidates`` [B,Tq,Hkv,W]; -inf where not scored.

    Restates the scoring half of ``leaf_triton.py:144-232`` with the Torch
    equations (``top_k_pyramid_torch.py:48-80``): scoreable slots follow
    ``leaf_triton.py:23-60`` (identity rule off for pisa1).
    """
    q, k, candidates = np.asarray(q), np.asarray(k), np.asarray(candidates, dtype=np.int64)
    batch, tokens, heads, width = candidates.shape
    dim = q.shape[-1]
    groups = q.shape[2] // heads
    blocks = (k.shape[1] + block_size - 1) // block_size
    ids = np.where((candidates >= blocks), -1, candidates)
    pos = np.broadcast_to(np.asarray(positions)[:, :, None], (batch, tokens, heads))
    valid = (ids >= 0) & (ids * block_size <= pos[..., None])
    forced = force_mask(ids, pos, block_size, force_first, force_recent, 0) & valid
    scoreable = valid & ~forced
    if method != "pisa1":
        scoreable &= (valid.sum(-1) > topk)[..., None]
    out = np.full(candidates.shape, -np.inf, dtype=np.float32)
    b, t, h, w = np.nonzero(scoreable)
    query = q[b, t].reshape(-1, heads, groups, dim)[np.arange(b.shape[0]), h]
    if method == "pisa1":
        source = leaf_means if leaf_means is not None else mean_pool(k, block_size)
        vals = _scores_for(query, source, b, h, ids[b, t, h, w], 1, method, 1.0, compute)
    else:
        vals = _scores_for(query, k, b, h, ids[b, t, h, w], block_size, method, dim ** -0.5,
                           compute)
    out[b, t, h, w] = vals
    return out


# --------------------------------------------------------------------------- attention

def _gather_tokens(indices, block_size, n, positions, causal):
    tokens = (np.asarray(indices, dtype=np.int64)[..., None] * block_size
              + np.arange(block_size)).reshape(*indices.shape[:-1], -1)
    valid = (tokens >= 0) & (tokens < n)
    if causal:
        valid &= tokens <= np.asarray(positions)[:, :, None, None]
    return np.clip(tokens, 0, n - 1), valid


def sparse_attention(q, k, v, indices, block_size, scale=None, positions=None, causal=True,
                     compute=np.float64, chunk=32):
    """Attention over the keys of the selected blocks; returns (O, LSE).

    Restates ``sparse_attn/sparse_attn_torch.py:6-35`` (32-token chunks, gathered
    keys, masked softmax, rows without a valid key give 0) and adds the natural
    log-sum-exp of the masked logits, -inf for empty rows.  O is returned in the
    compute dtype (callers round it to the storage dtype).
    """
    q, k, v = (np.asarray(x, dtype=compute) for x in (q, k, v))
    batch, length, query_heads, dim = q.shape
    heads, n = k.shape[2], k.shape[1]
    groups = query_heads // heads
    scale = dim ** -0.5 if scale is None else scale
    if positions is None:
        positions = query_positions(batch, length, n)
    out = np.zeros((batch, length, query_heads, v.shape[-1]), dtype=compute)
    lse = np.full((batch, length, query_heads), -np.inf, dtype=compute)
    b_ids = np.arange(batch)[:, None, None, None]
    h_ids = np.arange(heads)[None, None, :, None]
    for start in range(0, length, chunk):
        ids = np.asarray(indices)[:, start:start + chunk]
        tokens, valid = _gather_tokens(ids, block_size, n, positions[:, start:start + chunk],
                                       causal)
        keys = k[b_ids, tokens, h_ids]                                     # [B,t,H,S,D]
        values = v[b_ids, tokens, h_ids]
        query = q[:, start:start + chunk].reshape(batch, -1, heads, groups, dim)
        logits = np.einsum("bthgd,bthsd->bthgs", query, keys) * scale
        masked = np.where(valid[..., None, :], logits, -np.inf)
        peak = masked.max(-1, keepdims=True)
        safe = np.where(np.isfinite(peak), peak, 0)
        weights = np.where(valid[..., None, :], np.exp(masked - safe), 0)
        denom = weights.sum(-1, keepdims=True)
        prob = weights / np.where(denom > 0, denom, 1)
        result = np.einsum("bthgs,bthsv->bthgv", prob, values)
        out[:, start:start + chunk] = result.reshape(batch, -1, query_heads, v.shape[-1])
        with np.errstate(divide="ignore"):
            row_lse = np.where(denom[..., 0] > 0, safe[..., 0] + np.log(denom[..., 0]), -np.inf)
        lse[:, start:start + chunk] = row_lse.reshape(batch, -1, query_heads)
    return out, lse


def sparse_attention_dense(q, k, v, indices, block_size, scale=None, positions=None, causal=True):
    """Textbook dense attention under the union-of-selected-blocks mask (float64).

    Independent of the gather formulation: mask[t, n] = key n lies in one of
    row t's selected blocks (and n <= pos when causal).  Equal to
    ``sparse_attention`` whenever a row's ids are distinct.
    """
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    batch, length, query_heads, dim = q.shape
    heads, n = k.shape[2], k.shape[1]
    groups = query_heads // heads
    scale = dim ** -0.5 if scale is None else scale
    if positions is None:
        positions = query_positions(batch, length, n)
    tokens, valid = _gather_tokens(np.asarray(indices), block_size, n, positions, causal)
    out = np.zeros((batch, length, query_heads, v.shape[-1]))
    lse = np.full((batch, length, query_heads), -np.inf)
    for b in range(batch):
        for h in range(heads):
            mask = np.zeros((length, n), dtype=bool)
            t_ids = np.broadcast_to(np.arange(length)[:, None], tokens[b, :, h].shape)
            mask[t_ids[valid[b, :, h]], tokens[b, :, h][valid[b, :, h]]] = True
            for g in range(groups):
                hq = h * groups + g
                logits = q[b, :, hq] @ k[b, :, h].T * scale
                logits = np.where(mask, logits, -np.inf)
                peak = logits.max(-1, keepdims=True)
                safe = np.where(np.isfinite(peak), peak, 0)
                w = np.where(mask, np.exp(logits - safe), 0)
                denom = w.sum(-1, keepdims=True)
                out[b, :, hq] = (w / np.where(denom > 0, denom, 1)) @ v[b, :, h]
                with np.errstate(divide="ignore"):
                    lse[b, :, hq] = np.where(denom[:, 0] > 0, safe[:, 0] + np.log(denom[:, 0]),
                                             -np.inf)
    return out, lse


def sparse_attention_backward(q, k, v, indices, grad_out, block_size, scale=None, positions=None,
                              causal=True, chunk=32):
    """Closed-form gradients (float64) of ``sparse_attention`` w.r.t. q, k, v.

    With P the masked softmax and dO the upstream gradient:
    dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dO * O)), dQ = s dS K, dK = s dS^T Q,
    scattered back through the gathers of ``sparse_attn_torch.py:19-24``.
    """
    q, k, v, grad_out = (np.asarray(x, dtype=np.float64) for x in (q, k, v, grad_out))
    batch, length, query_heads, dim = q.shape
    heads, n = k.shape[2], k.shape[1]
    groups = query_heads // heads
    scale = dim ** -0.5 if scale is None else scale
    if positions is None:
        positions = query_positions(batch, length, n)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    b_ids = np.arange(batch)[:, None, None, None]
    h_ids = np.arange(heads)[None, None, :, None]
    for start in range(0, length, chunk):
        ids = np.asarray(indices)[:, start:start + chunk]
        tokens, valid = _gather_tokens(ids, block_size, n, positions[:, start:start + chunk],
                                       causal)
        keys = k[b_ids, tokens, h_ids]
        values = v[b_ids, tokens, h_ids]
        query = q[:, start:start + chunk].reshape(batch, -1, heads, groups, dim)
        dout = grad_out[:, start:start + chunk].reshape(batch, -1, heads, groups, v.shape[-1])
        logits = np.einsum("bthgd,bthsd->bthgs", query, keys) * scale
        masked = np.where(valid[..., None, :], logits, -np.inf)
        peak = masked.max(-1, keepdims=True)
        safe = np.where(np.isfinite(peak), peak, 0)
        weights = np.where(valid[..., None, :], np.exp(masked - safe), 0)
        denom = weights.sum(-1, keepdims=True)
        prob = weights / np.where(denom > 0, denom, 1)
        out = np.einsum("bthgs,bthsv->bthgv", prob, values)
        dvals = np.einsum("bthgs,bthgv->bthsv", prob, dout)
        dprob = np.einsum("bthgv,bthsv->bthgs", dout, values)
        delta = (dout * out).sum(-1, keepdims=True)
        dlogits = prob * (dprob - delta)
        dquery = np.einsum("bthgs,bthsd->bthgd", dlogits, keys) * scale
        dkeys = np.einsum("bthgs,bthgd->bthsd", dlogits, query) * scale
        dq[:, start:start + chunk] = dquery.reshape(batch, -1, query_heads, dim)
        bb = np.broadcast_to(b_ids, tokens.shape)
        hh = np.broadcast_to(h_ids, tokens.shape)
        sel = valid
        np.add.at(dk, (bb[sel], tokens[sel], hh[sel]), dkeys[sel])
        np.add.at(dv, (bb[sel], tokens[sel], hh[sel]), dvals[sel])
    return dq, dk, dv


def flops_visible(indices, block_size, n, positions, causal=True):
    """Number of (row, key) pairs attended per KV head row: sum of visible keys."""
    _, valid = _gather_tokens(np.asarray(indices), block_size, n, positions, causal)
    return int(valid.sum())


# --------------------------------------------------------------------------- rotary encoding


def rotary_frequency(head_dim, base, fraction):
    """Frequencies of ``xmixers/xmixers/modules/pes/lrpe.py:20-28`` (type 3): the float32
    values base^(-2 i / head_dim) for i < head_dim // 2 * fraction, zero after."""
    exponent = np.float32(-2.0 / head_dim) * np.arange(head_dim // 2, dtype=np.float32)
    theta = np.power(np.float32(base), exponent, dtype=np.float32)
    theta[int(head_dim // 2 * fraction):] = 0
    return theta


def rotary(x, frequency, positions):
    """Split-half rotary encoding (``pisa/pisa/ops/lrpe/rotary_torch.py:5-10``).

    The angle is the reference's float32 product position x frequency; the turn
    itself is evaluated in float64 (callers round to the storage dtype).
    ``positions`` is ``[B or 1, T]``.
    """
    x = np.asarray(x, dtype=np.float64)
    angles = (np.asarray(positions, dtype=np.float32)[..., None, None]
              * np.asarray(frequency, dtype=np.float32).reshape(-1)).astype(np.float64)
    first, second = np.split(x, 2, axis=-1)
    cos, sin = np.cos(angles), np.sin(angles)
    return np.concatenate((first * cos - second * sin, first * sin + second * cos), -1)



# --------------------------------------------------------------------------- flat BSA routing


def bitonic_merge(scores, ids, stage, descending):
    """One merge of the streaming network (``ops/flash_sparse_attn/bsa/bsa_torch.py:8-25``).

    Lanes pair at distances 2**(stage-1) .. 1; a pair exchanges iff
    ``(lower > upper) != descending`` where ``descending`` is the lane's bit
    ``stage`` (``None``, alternating runs) or the given constant.  ids ride along.
    """
    width = scores.shape[-1]
    lanes = np.arange(width)
    direction = ((lanes & (1 << stage)) != 0) if descending is None else np.full(width, descending)
    for exponent in range(stage - 1, -1, -1):
        distance = 1 << exponent
        partner = lanes ^ distance
        lower = lanes & ~distance
        upper = lower | distance
        exchange = (scores[..., lower] > scores[..., upper]) != direction
        scores = np.where(exchange, scores[..., partner], scores)
        ids = np.where(exchange, ids[..., partner], ids)
    return scores, ids


def streaming_topk(scores, ids, topk, tile_size):
    """Top-``topk`` ids in network rank order over tiles of ``tile_size`` lanes
    (``bsa_torch.py:28-58``): each tile is sorted into alternating runs, its best half
    merged with the retained best half of the tiles before; tiles holding no id >= 0
    are skipped; the tail tile pads with score 0 and id -1."""
    if topk < 1 or tile_size < 2 * topk or tile_size & (tile_size - 1):
        raise ValueError("tile_size must be a power of two and at least 2 * topk")
    scores = np.asarray(scores)
    ids = np.asarray(ids)
    if scores.shape != ids.shape or scores.shape[-1] < 1:
        raise ValueError("scores and ids must have the same nonempty shape")
    stages = tile_size.bit_length() - 1
    lead = scores.shape[:-1]
    retained_scores = np.full(lead + (tile_size,), -1, dtype=scores.dtype)
    retained_ids = np.zeros(lead + (tile_size,), dtype=ids.dtype)
    half = tile_size // 2
    for start in range(0, scores.shape[-1], tile_size):
        values = scores[..., start:start + tile_size]
        indices = ids[..., start:start + tile_size]
        active = (indices >= 0).any(-1, keepdims=True)
        padding = tile_size - values.shape[-1]
        pad = [(0, 0)] * len(lead) + [(0, padding)]
        values = np.pad(values, pad, constant_values=0)
        indices = np.pad(indices, pad, constant_values=-1)
        for stage in range(1, stages):
            values, indices = bitonic_merge(values, indices, stage, None)
        if start:
            values, indices = bitonic_merge(values, indices, stages, False)
            values = np.concatenate((retained_scores[..., :half], values[..., half:]), -1)
            indices = np.concatenate((retained_ids[..., :half], indices[..., half:]), -1)
        values, indices = bitonic_merge(values, indices, stages, True)
        retained_scores = np.where(active, values, retained_scores)
        retained_ids = np.where(active, indices, retained_ids)
    return retained_ids[..., :topk]


def bsa_tile_width(block_size, topk):
    """Comparison tile of flat routing: the power of two >= max(block_size, 2 topk)
    (``bsa_torch.py:74``)."""
    return 1 << (max(block_size, 2 * topk) - 1).bit_length()


def bsa_scores(q, k, block_size, positions, force_first, force_recent, dtype="fp32"):
    """Per-block routing scores [B, Tq, Hkv, M] and ids (-1 beyond the current block).

    Restates ``bsa_torch.py:61-103``: summaries are the block means of k
    (``mean_pool``), queries are scaled by D^-1/2 in float32 and rounded to the
    storage dtype, each head's logits are normalised by the log-sum-exp over the
    complete blocks (0 when none is complete), a block's score is the sum over the
    group's heads of exp(logit - normaliser) for blocks before the current one, the
    number of heads for forced blocks (block 0 with ``force_first``, the current
    block and the ``force_recent - 1`` before it), and 0 otherwise.  Raises the
    reference's ValueError when a token has more distinct forced blocks than
    ``topk`` would hold (checked by the caller, ``bsa_select``).
    """
    compute = np.float64 if dtype == "fp64" else np.float32
    q = np.asarray(q)
    batch, length, heads_q, dim = q.shape
    heads = k.shape[2]
    groups = heads_q // heads
    summaries = mean_pool(k, block_size, dtype).astype(compute)
    blocks = np.arange(summaries.shape[1])
    scale = compute(dim ** -0.5)
    query = round_storage(np.asarray(q, dtype=compute) * scale, dtype).astype(compute)
    query = query.reshape(batch, length, heads, groups, dim)
    logits = np.einsum("bthgd,bmhd->bthgm", query, summaries).astype(compute)
    position = np.asarray(positions, dtype=np.int64)
    position = np.broadcast_to(position, (batch, length))[:, :, None, None]
    current = position // block_size
    complete = (position + 1) // block_size
    visible = blocks < complete[..., None]
    masked = np.where(visible, logits, -np.inf)
    peak = masked.max(-1, keepdims=True)
    safe = np.where(np.isfinite(peak), peak, 0)
    with np.errstate(divide="ignore"):
        normalizer = np.log(np.exp(masked - safe).sum(-1, keepdims=True)) + safe
    normalizer = np.where(complete[..., None] > 0, normalizer, 0).astype(compute)
    forced = np.zeros(current.shape[:2] + (1, blocks.size), dtype=bool)
    if force_first:
        forced |= blocks == 0
    for recent in range(force_recent):
        forced |= (current >= recent) & (blocks == current - recent)
    valid = blocks <= current
    candidate = np.where((blocks < current)[..., None, :], logits, -np.inf)
    probabilities = np.exp(candidate - normalizer).astype(compute)
    probabilities = np.where(forced[..., None, :], compute(1), probabilities)
    scores = probabilities.sum(-2, dtype=compute)
    ids = np.where(valid, blocks, -1)
    ids = np.broadcast_to(ids, scores.shape).astype(np.int64)
    required = (forced & valid).sum(-1)
    return scores, ids, required


def bsa_select(q, k, block_size, topk, positions, force_first, force_recent, dtype="fp32"):
    """Flat BSA block selection (``bsa_torch.py:61-106``): ids [B, Tq, Hkv, topk] in
    network rank order, -1 padded."""
    scores, ids, required = bsa_scores(q, k, block_size, positions, force_first,
                                       force_recent, dtype)
    if (required > topk).any():
        raise ValueError("topk is smaller than the number of required distinct blocks")
    return streaming_topk(scores, ids, topk, bsa_tile_width(block_size, topk))
