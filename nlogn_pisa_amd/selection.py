"""PISA block selection on the GPU: ``select_blocks`` / ``top_k_pyramid_fn``.

Same signature, defaults, validation messages and return convention as the
reference's ``pisa/ops/flash_sparse_attn/top_k_pyramid/top_k_pyramid.py:11-121``
(ids int64 [B, Tq, Hkv, K], -1 padded, slot order of the comparison network),
plus one keyword, ``branching`` (the reference hard-codes 2).  Every backend
name runs the HIP library on ROCm tensors; CPU tensors are rejected.
"""

from __future__ import annotations

import ctypes
import math
import types

import torch

from . import _lib
from ._common import (dtype_code, kernel_layout, positions_layout, ptr, require_gpu, stream_of,
                      workspace)
from .pooling import build_pyramid_storage
from .validation import packed_queries, query_positions, validate_qkv

BACKENDS = ("torch", "triton", "auto", "hip")
MAX_BLOCK = 1 << 16  # largest key block of the GPU selection (kMaxSelectBlock)


def routing_geometry(blocks, topk, branching=2):
    """(top level, first network width); ``top_k_pyramid_torch.py:124-133`` with b in place of 2."""
    top = 0
    while blocks > topk:
        parent = (blocks + branching - 1) // branching
        if parent < topk or parent == blocks:
            break
        blocks = parent
        top += 1
    return top, max(16, 1 << (max(blocks, topk) - 1).bit_length())


@torch.no_grad()
def select_blocks(q, k, method="pisa", block_size=64, topk=8, cu_seqlens=None, query_offset=None,
                  force_first=True, force_recent=2, backend="torch", pyramid=None, leaf_tile=4,
                  routing_schedule="auto", branching=2):
    """Return block ids [B, Tq, Hkv, K] (int64), padded by -1.

    Queries/keys must already carry any positional encoding.  Packed ids are
    local to each document.  Slot order follows the comparison network; the
    required blocks (first, and the ``force_recent`` most recent) count toward
    the K slots.  ``routing_schedule="auto"`` uses the grouped (block-major)
    leaf for pisa/pisa2 prefill and multi-query suffixes and the fused leaf for
    single-query decode and pisa1 (``top_k_pyramid.py:64-72``).  ``leaf_tile``
    is accepted for compatibility; grouped tiles here hold up to 256 requests.
    """
    validate_qkv(q, k)
    if method not in ("bsa", "pisa1", "pisa2", "pisa"):
        raise ValueError("method must be bsa, pisa1, pisa2 or pisa")
    if backend not in BACKENDS:
        raise ValueError("backend must be torch, triton or auto")
    if leaf_tile not in (1, 2, 4):
        raise ValueError("leaf_tile must be 1, 2 or 4")
    if routing_schedule not in ("auto", "grouped", "fused"):
        raise ValueError("routing_schedule must be auto, grouped or fused")
    if block_size < 1 or topk < 1 or force_recent < 0:
        raise ValueError("positive block_size/topk and nonnegative force_recent required")
    if method != "bsa" and force_recent == 0:
        raise ValueError("causal pyramid routing requires force_recent >= 1")
    if method == "bsa":
        from .bsa import bsa_fn
        return bsa_fn(q, k, block_size, topk, cu_seqlens=cu_seqlens, query_offset=query_offset,
                      force_first=force_first, force_recent=force_recent, backend=backend)
    if branching < 2 or branching & (branching - 1):
        raise ValueError("branching must be a power of two >= 2")
    if routing_schedule == "auto":
        grouped = method != "pisa1" and (
            q.shape[1] == k.shape[1] or (cu_seqlens is None and q.shape[1] > 1))
        routing_schedule = "grouped" if grouped else "fused"
    if cu_seqlens is not None:
        return _select_packed(q, k, method, block_size, topk, cu_seqlens, query_offset,
                              force_first, force_recent, routing_schedule, branching)
    return _select_unpacked(q, k, method, block_size, topk, query_offset, force_first,
                            force_recent, pyramid, routing_schedule, None, branching)


def _select_packed(q, k, method, block_size, topk, cu_seqlens, query_offset, force_first,
                   force_recent, routing_schedule, branching):
    """Packed documents (``top_k_pyramid.py:73-86``): document-local ids, each document
    routed with its own depth (grouped) or the longest document's (fused).

    Documents run as the rows of zero-padded batches, one launch series per batch:
    a document's ids do not depend on keys past its end, because a scored block or
    node lies wholly before the query's current block (later ones fail the position
    test, the current block's ancestors are forced), so padding and a document's
    partial last block are never scored.  A batch holds the documents of one routing
    geometry and one power-of-two length class, which bounds the padding to 2x.
    """
    segments = packed_queries(q, k, cu_seqlens, query_offset)
    nblocks = [(ke - ks + block_size - 1) // block_size for _, _, ks, ke, _ in segments]
    shared = (routing_geometry(max(nblocks), topk, branching) if routing_schedule == "fused"
              else None)
    classes = {}
    for index, ((qs, qe, ks, ke, _), nb) in enumerate(zip(segments, nblocks)):
        geometry = shared or routing_geometry(nb, topk, branching)
        size = 1 << max(0, ke - ks - 1).bit_length()
        classes.setdefault((geometry, size), []).append(index)
    out = torch.empty((1, q.shape[1], k.shape[2], topk), device=q.device, dtype=torch.long)
    dev = q.device
    for (geometry, _), members in classes.items():
        qs, qe, ks, ke, offsets = (torch.tensor(col, device=dev, dtype=torch.long)
                                   for col in zip(*(segments[i] for i in members)))
        # rows of the padded batch (padding repeats the document's first row)
        kj = torch.arange(int((ke - ks).max()), device=dev)[None]
        qj = torch.arange(int((qe - qs).max()), device=dev)[None]
        key_rows = ks[:, None] + torch.where(kj < (ke - ks)[:, None], kj, 0)
        live = qj < (qe - qs)[:, None]
        query_rows = qs[:, None] + torch.where(live, qj, 0)
        ids = _select_unpacked(q[0][query_rows], k[0][key_rows], method, block_size, topk,
                               offsets, force_first, force_recent, None, routing_schedule,
                               geometry, branching)
        out[0, query_rows[live]] = ids[live]
    return out


def _pad_dim(x, width):
    return torch.nn.functional.pad(x, (0, width - x.shape[-1])).contiguous()


def _padded_pyramid(pyramid, width):
    """A caller's pyramid (cache or levels) with rows zero-padded to ``width``."""
    if pyramid is None:
        return None
    if hasattr(pyramid, "storage"):
        starts = getattr(pyramid, "starts", None)
        return types.SimpleNamespace(
            storage=_pad_dim(pyramid.storage, width), level_sizes=list(pyramid.level_sizes),
            starts=list(starts if starts is not None else pyramid.offsets.tolist()))
    levels = list(pyramid.levels if hasattr(pyramid, "levels") else pyramid)
    return [_pad_dim(x, width) for x in levels]


def _pyramid_desc(q, k, block_size, branching, top, pyramid):
    """Packed level storage and its descriptor (levels padded to top + 1)."""
    if pyramid is None:
        storage, offsets, lengths = build_pyramid_storage(k, block_size, branching, max_level=top)
    elif hasattr(pyramid, "storage"):
        storage = pyramid.storage
        lengths = [int(x) for x in pyramid.level_sizes]
        starts = getattr(pyramid, "starts", None)
        offsets = [int(x) for x in (starts if starts is not None else pyramid.offsets.tolist())]
        offsets = offsets[:len(lengths)]
    else:
        levels = list(pyramid.levels if hasattr(pyramid, "levels") else pyramid)
        lengths = [int(x.shape[1]) for x in levels]
        offsets = [sum(lengths[:i]) for i in range(len(lengths))]
        storage = torch.cat([x.to(k.dtype) for x in levels], dim=1).contiguous()
    if storage.device != q.device or storage.dtype != q.dtype:
        raise ValueError("the pyramid must share q's dtype and device")
    if storage.stride(-1) != 1 or storage.stride(-2) != storage.shape[-1] or \
            storage.stride(1) != storage.shape[-1] * storage.shape[-2]:
        raise ValueError("pyramid storage rows must be contiguous [Hkv, D]")
    while len(lengths) < top + 1:
        offsets.append(offsets[-1])
        lengths.append(lengths[-1])
    desc = _lib.PyramidDesc()
    desc.storage = storage.data_ptr()
    desc.stride_batch = storage.stride(0)
    desc.levels = len(lengths)
    for i, (o, n) in enumerate(zip(offsets, lengths)):
        desc.offsets[i] = o
        desc.lengths[i] = n
    return storage, desc


def _qk_desc(q, k):
    d = _lib.QkDesc()
    d.batch, d.query_tokens, d.query_heads, d.head_dim = q.shape
    d.key_tokens, d.key_heads = k.shape[1], k.shape[2]
    d.q_stride_batch, d.q_stride_token = q.stride(0), q.stride(1)
    d.k_stride_batch, d.k_stride_token = k.stride(0), k.stride(1)
    d.dtype = dtype_code(q, "GPU routing supports FP16, BF16 and FP32")
    return d


def _select_params(method, block_size, branching, topk, force_first, force_recent, top,
                   first_width, schedule, scale=0.0):
    p = _lib.SelectParams()
    p.scale = scale
    p.method = _lib.METHODS[method]
    p.block_size, p.branching, p.topk = block_size, branching, topk
    p.force_first, p.force_recent = int(bool(force_first)), force_recent
    p.top, p.first_width = top, first_width
    p.schedule = _lib.SCHEDULES[schedule]
    return p


def _check_gpu_shape(q, k, block_size, topk, branching, force_first, force_recent):
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("GPU routing supports FP16, BF16 and FP32")
    if block_size & (block_size - 1) or not 16 <= block_size <= MAX_BLOCK or not 1 <= topk <= 64:
        raise ValueError(f"GPU routing requires power-of-two block_size >= 16 (up to {MAX_BLOCK}) and "
                         "topk in [1, 64]")
    if branching * topk > 512:
        raise ValueError("branching * topk must not exceed 512")
    blocks = (k.shape[1] + block_size - 1) // block_size
    if topk < min(blocks, force_recent + int(force_first)):
        raise ValueError("topk cannot hold all required blocks")
    return blocks


def _select_unpacked(q, k, method, block_size, topk, query_offset, force_first, force_recent,
                     pyramid, routing_schedule, geometry, branching, trace=False):
    positions = positions_layout(query_positions(q, k, query_offset))
    require_gpu(q, "select_blocks")
    blocks = _check_gpu_shape(q, k, block_size, topk, branching, force_first, force_recent)
    top, first_width = geometry or routing_geometry(blocks, topk, branching)
    q = q.contiguous()
    k = kernel_layout(k)
    scale = 0.0
    if q.shape[-1] % 16:
        # the kernels take head dims on the 16 grid: zero dimensions change no product
        # or block mean, and the leaf keeps the scale of the true head dim
        scale = 1.0 / math.sqrt(q.shape[-1])
        width = -(-q.shape[-1] // 16) * 16
        q, k = _pad_dim(q, width), _pad_dim(k, width)
        pyramid = _padded_pyramid(pyramid, width)
    storage, pdesc = _pyramid_desc(q, k, block_size, branching, top, pyramid)
    qk = _qk_desc(q, k)
    params = _select_params(method, block_size, branching, topk, force_first, force_recent, top,
                            first_width, routing_schedule, scale)
    lib = _lib.library()
    batch, tokens, heads = q.shape[0], q.shape[1], k.shape[2]
    out = torch.empty((batch, tokens, heads, topk), device=q.device, dtype=torch.long)
    levels = torch.empty((batch, tokens, heads, top + 1, topk), device=q.device,
                         dtype=torch.int32) if trace else None
    with torch.cuda.device(q.device):
        nbytes = lib.pisa_select_workspace_size(ctypes.byref(qk), ctypes.byref(params))
        ws = workspace(nbytes, q.device)
        _lib.check(lib.pisa_select(ctypes.byref(qk), ctypes.byref(params), ptr(q), ptr(k),
                                   ctypes.byref(pdesc), ptr(positions), positions.stride(0),
                                   ptr(out), ptr(levels), ptr(ws), ws.numel(), stream_of(q)))
    del storage
    return (out, levels) if trace else out


@torch.no_grad()
def select_blocks_traced(q, k, method="pisa", block_size=64, topk=8, query_offset=None,
                         force_first=True, force_recent=2, routing_schedule="auto", branching=2,
                         pyramid=None, geometry=None):
    """``select_blocks`` plus int32 [B, Tq, Hkv, top + 1, K]: the ids each level kept.

    ``geometry`` (top, first width) overrides the keys' own routing geometry, as a
    packed fused selection shares the longest document's.  For tie adjudication
    against a CPU restatement; not a reference API.
    """
    validate_qkv(q, k)
    if routing_schedule == "auto":
        grouped = method != "pisa1" and q.shape[1] > 1
        routing_schedule = "grouped" if grouped else "fused"
    return _select_unpacked(q, k, method, block_size, topk, query_offset, force_first,
                            force_recent, pyramid, routing_schedule, geometry, branching,
                            trace=True)


@torch.no_grad()
def leaf_scores(q, k, candidates, block_size, method, positions, topk, force_first=True,
                force_recent=2, leaf_means=None):
    """Float32 scores shaped like ``candidates`` [B,Tq,Hkv,W]; -inf where not scoreable.

    Mirrors ``grouped_leaf_scores`` (``leaf_triton.py:144-232``) with the
    scoreable mask of ``leaf_triton.py:44-60`` always applied.
    """
    validate_qkv(q, k)
    require_gpu(q, "leaf scoring")
    if method not in ("pisa1", "pisa2", "pisa"):
        raise ValueError("expected method pisa1/pisa2/pisa and tile_size 1/2/4")
    if candidates.ndim != 4 or tuple(candidates.shape[:3]) != (*q.shape[:2], k.shape[2]):
        raise ValueError("candidates must have shape [B,Tq,Hkv,W]")
    if candidates.dtype not in (torch.int32, torch.int64) or candidates.device != q.device:
        raise ValueError("candidates must use an integer dtype on the query device")
    q = q.contiguous()
    k = kernel_layout(k)
    cand = candidates.to(torch.int32).contiguous()
    positions = positions_layout(torch.broadcast_to(positions, q.shape[:2]).to(q.device))
    if method == "pisa1" and leaf_means is None:
        from .pooling import mean_pool
        leaf_means = mean_pool(k, block_size)
    if leaf_means is not None:
        leaf_means = leaf_means.contiguous()
    qk = _qk_desc(q, k)
    params = _select_params(method, block_size, 2, topk, force_first, force_recent, 0, 16,
                            "grouped")
    out = torch.empty(cand.shape, device=q.device, dtype=torch.float32)
    width = cand.shape[-1]
    lib = _lib.library()
    ws = workspace(lib.pisa_leaf_workspace_size(ctypes.byref(qk), block_size, width), q.device)
    with torch.cuda.device(q.device):
        _lib.check(lib.pisa_leaf_scores(
            ctypes.byref(qk), ctypes.byref(params), ptr(q), ptr(k), ptr(leaf_means),
            leaf_means.stride(0) if leaf_means is not None else 0, ptr(cand), width,
            ptr(positions), positions.stride(0), ptr(out), ptr(ws), ws.numel(), stream_of(q)))
    return out


top_k_pyramid_fn = select_blocks
