"""Shape, position and packing contracts of the public operators.

Same behaviour and messages as the reference's ``pisa/utils/validation.py``
(cited per function) so callers see identical ``ValueError``s.
"""

from __future__ import annotations

import torch


def sequence_slices(cu_seqlens, length):
    """Document boundaries as (start, end) pairs; ``validation.py:8-18``."""
    if cu_seqlens is None:
        return [(0, length)]
    if cu_seqlens.ndim != 1 or cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise ValueError("cu_seqlens must be a one-dimensional integer tensor")
    bounds = [int(x) for x in cu_seqlens.detach().cpu().tolist()]
    if len(bounds) < 2 or bounds[0] != 0 or bounds[-1] != length:
        raise ValueError("cu_seqlens must start at zero and end at the key length")
    pairs = list(zip(bounds[:-1], bounds[1:]))
    if any(start >= end for start, end in pairs):
        raise ValueError("packed sequences must be nonempty and strictly ordered")
    return pairs


def validate_qkv(q, k, v=None):
    """``validation.py:21-35``."""
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("q and k must have shape [batch, tokens, heads, head_dim]")
    if q.shape[0] != k.shape[0] or q.shape[-1] != k.shape[-1]:
        raise ValueError("q and k must share batch size and head dimension")
    if min(*q.shape, *k.shape) <= 0 or q.shape[2] % k.shape[2]:
        raise ValueError(
            "nonempty tensors and a whole number of query heads per KV head are required")
    if q.device != k.device or q.dtype != k.dtype or not q.is_floating_point():
        raise ValueError("q and k must share a floating dtype and device")
    if v is not None and (v.ndim != 4 or v.shape[:3] != k.shape[:3] or v.device != k.device
                          or v.dtype != k.dtype):
        raise ValueError("v must share k's batch, length, heads, dtype and device")


def query_positions(q, k, query_offset=None):
    """Absolute positions int64 [B, Tq] on q's device; ``validation.py:38-56``.

    Integer offsets are checked on the host (no device read); tensor offsets
    (one per batch row) are checked with a device reduction, as the reference.
    """
    batch, tokens, keys = q.shape[0], q.shape[1], k.shape[1]
    if query_offset is None or isinstance(query_offset, int):
        offset = keys - tokens if query_offset is None else int(query_offset)
        if offset < 0 or offset + tokens > keys:
            raise ValueError("queries must refer to positions within their key sequence")
        return torch.arange(offset, offset + tokens, device=q.device,
                            dtype=torch.long)[None].expand(batch, -1)
    offset = torch.as_tensor(query_offset, device=q.device, dtype=torch.long)
    if offset.ndim > 1 or offset.numel() not in (1, batch):
        raise ValueError("query_offset must be a scalar or one offset per batch element")
    positions = (offset.reshape(-1, 1) + torch.arange(tokens, device=q.device)).expand(batch, -1)
    if bool((positions < 0).any()) or bool((positions >= keys).any()):
        raise ValueError("queries must refer to positions within their key sequence")
    return positions


def packed_queries(q, k, cu_seqlens, query_offset=None):
    """Per-document (q_start, q_end, k_start, k_end, local_offset); ``validation.py:59-81``."""
    if q.shape[0] != 1:
        raise ValueError("packed inputs require batch size one")
    segments = sequence_slices(cu_seqlens, k.shape[1])
    if q.shape[1] == k.shape[1]:
        if query_offset is not None and bool(torch.as_tensor(query_offset).ne(0).any()):
            raise ValueError("packed prefill has local query_offset zero")
        return [(start, end, start, end, 0) for start, end in segments]
    if q.shape[1] == len(segments):
        offsets = None if query_offset is None else torch.as_tensor(query_offset).reshape(-1)
        if offsets is not None and offsets.numel() not in (1, len(segments)):
            raise ValueError("packed decode needs a scalar or one offset per document")
        out = []
        for index, (start, end) in enumerate(segments):
            local = end - start - 1 if offsets is None else int(offsets[min(index, offsets.numel() - 1)])
            out.append((index, index + 1, start, end, local))
        return out
    raise ValueError("packed inputs support full prefill or one decode query per document")
