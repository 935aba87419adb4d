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

import torch

from . import _lib
from ._common import (dtype_code, kernel_layout, positions_layout, ptr, require_gpu, stream_of,
                      workspace)
from .validation import packed_queries, query_positions, validate_qkv


def _attn_desc(q, k, v, indices, block_size, scale, causal):
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
    return d


def _forward(q, k, v, indices, positions, block_size, scale, causal, keep_f32=False):
    desc = _attn_desc(q, k, v, indices, block_size, scale, causal)
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


def _backward(q, k, v, indices, positions, out, out32, lse, grad_out, block_size, scale,
              causal):
    desc = _attn_desc(q, k, v, indices, block_size, scale, causal)
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
    def forward(ctx, q, k, v, indices, positions, block_size, scale, causal):
        keep = any(ctx.needs_input_grad[:3])
        out, lse, out32 = _forward(q, k, v, indices, positions, block_size, scale, causal, keep)
        ctx.save_for_backward(q, k, v, indices, positions, out, out32, lse)
        ctx.config = (block_size, scale, causal)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        q, k, v, indices, positions, out, out32, lse = ctx.saved_tensors
        block_size, scale, causal = ctx.config
        dq, dk, dv = _backward(q, k, v, indices, positions, out, out32, lse, grad_out,
                               block_size, scale, causal)
        return dq, dk, dv, None, None, None, None, None


def _check(q, k, v, indices, block_size, backend):
    validate_qkv(q, k, v)
    if indices.ndim != 4 or tuple(indices.shape[:3]) != (*q.shape[:2], k.shape[2]):
        raise ValueError("indices must have shape [B,Tq,Hkv,K]")
    if indices.dtype not in (torch.int32, torch.int64) or indices.device != q.device:
        raise ValueError("indices must be integers on the query device")
    if block_size < 1 or backend not in ("torch", "auto", "triton", "fla", "hip"):
        raise ValueError("invalid block_size or attention backend")


def _unpacked(q, k, v, indices, block_size, scale, query_offset, causal):
    positions = positions_layout(query_positions(q, k, query_offset))
    require_gpu(q, "sparse_attention")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("CUDA attention supports FP16, BF16 and FP32")
    scale = k.shape[-1] ** -0.5 if scale is None else scale
    q = q.contiguous()
    k = kernel_layout(k)
    v = kernel_layout(v)
    indices = indices.contiguous()
    return _SparseAttention.apply(q, k, v, indices, positions, block_size, scale, causal)


def sparse_attention_with_lse(q, k, v, indices, block_size=64, scale=None, cu_seqlens=None,
                              query_offset=None, backend="torch", causal=True):
    """(O [B,Tq,Hq,Dv], LSE float32 [B,Tq,Hq]); O is differentiable w.r.t. q, k, v."""
    _check(q, k, v, indices, block_size, backend)
    if cu_seqlens is not None:
        outs, lses = [], []
        for qs, qe, ks, ke, offset in packed_queries(q, k, cu_seqlens, query_offset):
            o, l = _unpacked(q[:, qs:qe], k[:, ks:ke], v[:, ks:ke], indices[:, qs:qe],
                             block_size, scale, offset, causal)
            outs.append(o)
            lses.append(l)
        return torch.cat(outs, 1), torch.cat(lses, 1)
    return _unpacked(q, k, v, indices, block_size, scale, query_offset, causal)


def sparse_attention(q, k, v, indices, block_size=64, scale=None, cu_seqlens=None,
                     query_offset=None, backend="torch", causal=True):
    """Attention over the selected original K/V blocks -> [B, Tq, Hq, Dv] in q.dtype."""
    return sparse_attention_with_lse(q, k, v, indices, block_size, scale, cu_seqlens,
                                     query_offset, backend, causal)[0]


sparse_attn_fn = sparse_attention
