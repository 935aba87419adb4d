"""Tensor plumbing shared by the operators: dtype codes, streams, layouts."""

from __future__ import annotations

import ctypes

import torch

from . import _lib

DTYPES = {torch.float32: _lib.PISA_F32, torch.float16: _lib.PISA_F16,
          torch.bfloat16: _lib.PISA_BF16}


def require_gpu(tensor, what="this operator"):
    """The product runs on ROCm devices only; there is no CPU implementation."""
    if not tensor.is_cuda:
        raise ValueError(f"{what} runs on a ROCm GPU (HIP); got a tensor on {tensor.device}")


def dtype_code(tensor, message):
    code = DTYPES.get(tensor.dtype)
    if code is None:
        raise ValueError(message)
    return code


def stream_of(tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)


def kernel_layout(x):
    """Return ``x`` with head/dim contiguous and 16-byte aligned batch/token strides.

    Mirrors the reference's copy rule (copy only if stride(-1) != 1 or
    stride(-2) != D, top_k_pyramid_triton.py:345-347) plus the alignment the
    vectorised kernels need.
    """
    vec = 16 // x.element_size()
    ok = (x.stride(-1) == 1 and x.stride(-2) == x.shape[-1] and x.stride(0) % vec == 0
          and x.stride(1) % vec == 0 and x.data_ptr() % 16 == 0)
    return x if ok else x.contiguous()


def positions_layout(positions):
    if positions.dtype != torch.long:
        positions = positions.long()
    if positions.stride(-1) != 1:
        positions = positions.contiguous()
    return positions


def ptr(tensor):
    return ctypes.c_void_p(tensor.data_ptr()) if tensor is not None else None


def workspace(nbytes, device):
    """A byte buffer from torch's caching allocator (no device sync)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
