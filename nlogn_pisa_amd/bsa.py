"""Flat BSA block selection on the GPU: ``bsa_fn`` (the reference's benchmark baseline).

Same signature, defaults and validation messages as the reference's
``pisa/ops/flash_sparse_attn/bsa/bsa.py:9-52``; the selection is
``bsa_select`` (``bsa_torch.py:61-106``: probabilities of the block means,
normalised per head over the complete blocks, summed over the head group,
forced blocks, streaming comparison-network top-K) computed by the HIP kernel
``pisa_bsa_select``.  Ids are int64 [B, Tq, Hkv, topk] in network rank order,
-1 padded; packed documents (``cu_seqlens``) get document-local ids.  Every
backend name runs the HIP library on ROCm tensors; CPU tensors are rejected.

The reference's GPU path also hands one shape family (bf16, 16 query heads per
kv head, C = 64, topk 8 or 32, first + two recent blocks, full prefill) to FLA's
``parallel_nsa_topk`` (``bsa_fla.py:6-41``), whose tie order is FLA's; this
module keeps the streaming network's order for every shape.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._common import kernel_layout, positions_layout, ptr, require_gpu, stream_of, workspace
from .selection import _qk_desc
from .validation import packed_queries, query_positions, validate_qkv

BACKENDS = ("torch", "triton", "auto", "hip")


@torch.no_grad()
def bsa_fn(q, k, block_size=64, topk=8, *, cu_seqlens=None, query_offset=None,
           force_first=True, force_recent=2, backend="auto"):
    """Return block ids [B, Tq, Hkv, topk] (int64), padded by -1 (``bsa.py:9-25``)."""
    validate_qkv(q, k)
    if backend not in BACKENDS:
        raise ValueError("backend must be torch, triton or auto")
    if block_size < 1 or topk < 1 or force_recent < 0:
        raise ValueError("positive block_size/topk and nonnegative force_recent required")
    if cu_seqlens is not None:
        segments = list(packed_queries(q, k, cu_seqlens, query_offset))
        return torch.cat([
            _bsa_unpacked(q[:, qs:qe], k[:, ks:ke], block_size, topk, offset, force_first,
                          force_recent)
            for qs, qe, ks, ke, offset in segments
        ], dim=1)
    return _bsa_unpacked(q, k, block_size, topk, query_offset, force_first, force_recent)


def _bsa_unpacked(q, k, block_size, topk, query_offset, force_first, force_recent):
    """``select_unpacked`` (``bsa.py:28-52``) on the HIP kernel."""
    positions = positions_layout(query_positions(q, k, query_offset))
    require_gpu(q, "bsa_fn")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("Triton routing supports FP16, BF16 and FP32")
    if block_size > 128 or topk > 64:
        raise ValueError("GPU BSA routing requires block_size <= 128 and topk <= 64")
    blocks = (k.shape[1] + block_size - 1) // block_size
    if topk < min(blocks, force_recent + int(force_first)):
        raise ValueError("topk cannot hold all required blocks")
    q = q.contiguous()
    k = kernel_layout(k)
    qk = _qk_desc(q, k)
    lib = _lib.library()
    out = torch.empty((q.shape[0], q.shape[1], k.shape[2], topk), device=q.device,
                      dtype=torch.long)
    with torch.cuda.device(q.device):
        nbytes = lib.pisa_bsa_workspace_size(ctypes.byref(qk), block_size)
        ws = workspace(nbytes, q.device)
        _lib.check(lib.pisa_bsa_select(ctypes.byref(qk), block_size, topk, int(bool(force_first)),
                                       force_recent, ptr(q), ptr(k), ptr(positions),
                                       positions.stride(0), ptr(out), ptr(ws), ws.numel(),
                                       stream_of(q)))
    return out
