"""Sparse attention over selected blocks on the GPU: ``sparse_attention`` / ``sparse_attn_fn``.

Same signature, validation and semantics as the reference's
``pisa/ops/flash_sparse_attn/sparse_attn/sparse_attn.py:10-61`` (equations
``sparse_attn_torch.py:6-35``): each query row attends the keys of its selected
blocks, causally masked to its position; a row with no visible key outputs 0.
The forward and backward run in libpisa_hip.so; ``sparse_attention_with_lse``
also returns the natural-log LSE of every row (-inf for empty rows).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._common import (dtype_code, kernel_layout, positions_layout, ptr, require_gpu, stream_of,
                      workspace)
from .validation import packed_queries, query_positions, validate_qkv


class PackedKeys:
    """Packed documents laid out on whole key blocks, for one launch over all of them.

    Document d (keys [ks, ke), ``nb = ceil((ke - ks) / C)`` blocks) takes blocks
    ``base_d .. base_d + nb - 1`` of the launch; block ``base_d + j`` holds its keys
    ``ks + j C .. min(ke, ks + (j + 1) C) - 1``.  A query of the document at local
    position p sits at ``base_d C + p`` and its local id j becomes ``base_d + j``
    (ids outside ``[0, nb)`` select nothing, as for a document alone), so the
    kernels see one sequence of whole blocks and no row reaches another document.
    """

    def __init__(self, segments, tokens, block_size, device):
        seg = np.asarray(segments, dtype=np.int64).reshape(-1, 5)
        qs, qe, ks, ke, offset = seg.T
        nb = (ke - ks + block_size - 1) // block_size
        base = np.concatenate([[0], np.cumsum(nb)[:-1]])
        owner = np.repeat(np.arange(len(seg)), qe - qs)           # document of each query
        if owner.shape[0] != tokens:
            raise ValueError("packed segments must cover every query token")
        local = offset[owner] + np.arange(tokens) - qs[owner]
        doc_of_block = np.repeat(np.arange(len(seg)), nb)
        j = np.arange(doc_of_block.shape[0]) - base[doc_of_block]
        start = ks[doc_of_block] + j * block_size
        rows = np.minimum(block_size, ke[doc_of_block] - start)
        self.blocks = int(doc_of_block.shape[0])
        self.key_start = torch.from_numpy(start).to(device)
        self.key_rows = torch.from_numpy(rows.astype(np.int32)).to(device)
        self.positions = torch.from_numpy(base[owner] * block_size + local)[None].to(device)
        self._base = torch.from_numpy(base[owner]).to(device)[None, :, None, None]
        self._count = torch.from_numpy(nb[owner]).to(device)[None, :, None, None]

    def block_ids(self, indices):
        """Document-local ids [1, Tq, Hkv, K] -> ids of the launch's blocks (-1: none)."""
        ids = indices.long()
        return torch.where((ids >= 0) & (ids < self._count), ids + self._base,
                           torch.full_like(ids, -1))


def _attn_desc(q, k, v, indices, block_size, scale, causal, packed=None):
    d = _lib.AttnDesc()
    d.batch, d.query_tokens, d.query_heads, d.head_dim = q.shape
    d.key_tokens, d.key_heads = k.shape[1], k.shape[2]
    d.value_dim = v.shape[-1]
    d.q_stride_batch, d.q_stride_token = q.stride(0), q.stride(1)
    d.k_stride_batch, d.k_stride_token = k.stride(0), k.stride(1)
    d.v_stride_batch, d.v_stride_token = v.stride(0), v.stride(1)
    d.dtype = dtype_code(q, "CUDA attention supports FP16, BF16 and FP32")
    d.topk = indices.shape[-1]
    d.index_bits = 64 if indices.dtype == torch.int64 else 32
    d.block_size = block_size
    d.causal = int(bool(causal))
    d.scale = float(scale)
    if packed is not None:
        d.block_key_start = packed.key_start.data_ptr()
        d.block_key_rows = packed.key_rows.data_ptr()
        d.blocks = packed.blocks
    return d


def _forward(q, k, v, indices, positions, block_size, scale, causal, keep_f32=False,
             packed=None):
    d, dv_ = q.shape[-1], v.shape[-1]
    if d % 16 or dv_ % 16:
        # the kernels take head dims on the 16 grid: zero dimensions change no logit
        # (the scale stays the caller's) and add value columns that are dropped
        out, lse, out32 = _forward(_pad_dim(q, -(-d // 16) * 16).contiguous(),
                                   _pad_dim(k, -(-d // 16) * 16).contiguous(),
                                   _pad_dim(v, -(-dv_ // 16) * 16).contiguous(), indices,
                                   positions, block_size, scale, causal, keep_f32, packed)
        return (out[..., :dv_].contiguous(), lse,
                None if out32 is None else out32[..., :dv_].contiguous())
    desc = _attn_desc(q, k, v, indices, block_size, scale, causal, packed)
    lib = _lib.library()
    out = torch.empty((*q.shape[:3], v.shape[-1]), device=q.device, dtype=q.dtype)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    out32 = (torch.empty(out.shape, device=q.device, dtype=torch.float32)
             if keep_f32 and q.dtype != torch.float32 else None)
    with torch.cuda.device(q.device):
        ws = workspace(lib.pisa_attention_workspace_size(ctypes.byref(desc), 0), q.device)
        _lib.check(lib.pisa_sparse_attention_fwd(
            ctypes.byref(desc), ptr(q), ptr(k), ptr(v), ptr(indices), ptr(positions),
            positions.stride(0), ptr(out), ptr(lse), ptr(out32), ptr(ws), ws.numel(),
            stream_of(q)))
    return out, lse, out32


BACKWARD_DIMS = (16, 32, 64, 128)


def _pad_dim(x, dim):
    return x if x is None or x.shape[-1] == dim else torch.nn.functional.pad(x, (0, dim - x.shape[-1]))


def _backward(q, k, v, indices, positions, out, out32, lse, grad_out, block_size, scale,
              causal, packed=None):
    d, dv_ = q.shape[-1], v.shape[-1]
    if (d, dv_) != (d, d) or d not in BACKWARD_DIMS:
        # zero dimensions up to the next kernel head dim change no logit, probability or
        # rowsum(dO O); their gradient columns are dropped
        width = next((w for w in BACKWARD_DIMS if w >= max(d, dv_)), None)
        if width is None:
            raise ValueError("attention backward supports head dims up to 128")
        padded = [_pad_dim(x, width).contiguous() if x is not None else None
                  for x in (q, k, v, out, out32, grad_out)]
        dq, dk, dv = _backward(padded[0], padded[1], padded[2], indices, positions, padded[3],
                               padded[4], lse, padded[5], block_size, scale, causal, packed)
        return dq[..., :d], dk[..., :d], dv[..., :dv_]
    desc = _attn_desc(q, k, v, indices, block_size, scale, causal, packed)
    lib = _lib.library()
    grad_out = grad_out.contiguous()
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty(k.shape, device=k.device, dtype=k.dtype)
    dv = torch.empty(v.shape, device=v.device, dtype=v.dtype)
    with torch.cuda.device(q.device):
        ws = workspace(lib.pisa_attention_workspace_size(ctypes.byref(desc), 1), q.device)
        _lib.check(lib.pisa_sparse_attention_bwd(
            ctypes.byref(desc), ptr(q), ptr(k), ptr(v), ptr(indices), ptr(positions),
            positions.stride(0), ptr(out), ptr(out32), ptr(lse), ptr(grad_out), ptr(dq),
            ptr(dk), ptr(dv),
            ptr(ws), ws.numel(), stream_of(q)))
    return dq, dk, dv


class _SparseAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, indices, positions, block_size, scale, causal, packed):
        keep = any(ctx.needs_input_grad[:3])
        out, lse, out32 = _forward(q, k, v, indices, positions, block_size, scale, causal, keep,
                                   packed)
        ctx.save_for_backward(q, k, v, indices, positions, out, out32, lse)
        ctx.config = (block_size, scale, causal, packed)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        q, k, v, indices, positions, out, out32, lse = ctx.saved_tensors
        block_size, scale, causal, packed = ctx.config
        dq, dk, dv = _backward(q, k, v, indices, positions, out, out32, lse, grad_out,
                               block_size, scale, causal, packed)
        return dq, dk, dv, None, None, None, None, None, None


def _check(q, k, v, indices, block_size, backend):
    validate_qkv(q, k, v)
    if indices.ndim != 4 or tuple(indices.shape[:3]) != (*q.shape[:2], k.shape[2]):
        raise ValueError("indices must have shape [B,Tq,Hkv,K]")
    if indices.dtype not in (torch.int32, torch.int64) or indices.device != q.device:
        raise ValueError("indices must be integers on the query device")
    if block_size < 1 or backend not in ("torch", "auto", "triton", "fla", "hip"):
        raise ValueError("invalid block_size or attention backend")


# Largest key block the attention kernels stage (keys of a block in LDS); wide
# fp32 rows take less (kernel_block).
MAX_KERNEL_BLOCK = 128


def kernel_block(q, v, backward):
    """The largest key block the kernels take for q's dtype and the head dims on
    q's device (``pisa_attention_block_limit``: its tiles must fit the LDS), the
    backward's too when gradients will be asked for."""
    lib = _lib.library()
    code = dtype_code(q, "CUDA attention supports FP16, BF16 and FP32")
    with torch.cuda.device(q.device):
        limit = lib.pisa_attention_block_limit(code, q.shape[-1], v.shape[-1], int(backward))
    if limit <= 0:
        raise ValueError("attention head dims too wide for the GPU's LDS")
    return limit


def split_blocks(indices, block_size, limit=MAX_KERNEL_BLOCK):
    """Ids of blocks over `limit` keys as ids of their sub-blocks.

    A block of C keys is f consecutive sub-blocks of C / f keys (the largest divisor
    of C that is at most `limit`); block j becomes sub-blocks j f .. j f + f - 1
    and -1 stays -1.  The keys a row attends are the same set, so O, LSE and the
    gradients are those of the original blocks.  Returns (ids, sub-block size).
    """
    if block_size <= limit:
        return indices, block_size
    sub = max(d for d in range(1, limit + 1) if block_size % d == 0)
    f = block_size // sub
    ids = indices.long()
    parts = ids[..., None] * f + torch.arange(f, device=ids.device)
    return torch.where(ids[..., None] >= 0, parts, torch.full_like(parts, -1)).flatten(-2), sub


def _launch(q, k, v, indices, positions, block_size, scale, causal, packed=None):
    require_gpu(q, "sparse_attention")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("CUDA attention supports FP16, BF16 and FP32")
    scale = k.shape[-1] ** -0.5 if scale is None else scale
    q = q.contiguous()
    k = kernel_layout(k)
    v = kernel_layout(v)
    indices = indices.contiguous()
    return _SparseAttention.apply(q, k, v, indices, positions_layout(positions), block_size,
                                  scale, causal, packed)


def _needs_grad(q, k, v):
    return torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)


def _unpacked(q, k, v, indices, block_size, scale, query_offset, causal):
    require_gpu(q, "sparse_attention")
    indices, block_size = split_blocks(indices, block_size,
                                       kernel_block(q, v, _needs_grad(q, k, v)))
    return _launch(q, k, v, indices, query_positions(q, k, query_offset), block_size, scale,
                   causal)


def _packed(q, k, v, indices, block_size, scale, cu_seqlens, query_offset, causal):
    """Every document of a packed batch in one launch sequence (``sparse_attn.py:29-54``
    semantics: document-local ids and positions, keys of the row's own document)."""
    require_gpu(q, "sparse_attention")
    indices, block_size = split_blocks(indices, block_size,
                                       kernel_block(q, v, _needs_grad(q, k, v)))
    layout = PackedKeys(packed_queries(q, k, cu_seqlens, query_offset), q.shape[1], block_size,
                        q.device)
    return _launch(q, k, v, layout.block_ids(indices), layout.positions, block_size, scale,
                   causal, layout)


def sparse_attention_with_lse(q, k, v, indices, block_size=64, scale=None, cu_seqlens=None,
                              query_offset=None, backend="torch", causal=True):
    """(O [B,Tq,Hq,Dv], LSE float32 [B,Tq,Hq]); O is differentiable w.r.t. q, k, v."""
    _check(q, k, v, indices, block_size, backend)
    if cu_seqlens is not None:
        return _packed(q, k, v, indices, block_size, scale, cu_seqlens, query_offset, causal)
    return _unpacked(q, k, v, indices, block_size, scale, query_offset, causal)


def sparse_attention(q, k, v, indices, block_size=64, scale=None, cu_seqlens=None,
                     query_offset=None, backend="torch", causal=True):
    """Attention over the selected original K/V blocks -> [B, Tq, Hq, Dv] in q.dtype."""
    return sparse_attention_with_lse(q, k, v, indices, block_size, scale, cu_seqlens,
                                     query_offset, backend, causal)[0]


sparse_attn_fn = sparse_attention
