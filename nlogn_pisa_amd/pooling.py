"""Mean-pooled key pyramid on the GPU.

Mirrors ``pisa/ops/compress/mean_pooling/mean_pooling.py`` (``mean_pool``
:8-41, ``build_pyramid`` :45-52) with the HIP kernel of ``csrc/pisa_pool.hip``
in place of the Triton ``pool_kernel``.  Sums are always exact before one
rounding to the key dtype, so ``fp32_accumulation`` is accepted and has no
further effect.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._common import dtype_code, kernel_layout, ptr, require_gpu, stream_of


def _check_pool_input(keys, backend):
    if backend not in ("auto", "torch", "triton", "hip"):
        raise ValueError("pooling backend must be auto, torch, or triton")
    require_gpu(keys, "mean pooling")
    dtype_code(keys, "HIP pooling requires float16, bfloat16, or float32 dtype")
    if torch.is_grad_enabled() and keys.requires_grad:
        raise ValueError("HIP pooling does not support gradients")
    if keys.ndim != 4 or keys.numel() == 0:
        raise ValueError("pooling requires a nonempty [B,N,H,D] input")


def mean_pool(keys, size, *, backend="auto", fp32_accumulation=False):
    """Mean of each run of ``size`` tokens over its valid count -> [B, ceil(N/size), H, D]."""
    if size < 1:
        raise ValueError("pool size must be positive")
    _check_pool_input(keys, backend)
    keys = kernel_layout(keys)
    batch, length, heads, dim = keys.shape
    blocks = (length + size - 1) // size
    out = torch.empty((batch, blocks, heads, dim), device=keys.device, dtype=keys.dtype)
    with torch.cuda.device(keys.device):
        _lib.check(_lib.library().pisa_mean_pool(
            ptr(keys), keys.stride(0), keys.stride(1), batch, length, heads, dim, size,
            ptr(out), out.stride(0), out.stride(1), dtype_code(keys, ""), stream_of(keys)))
    return out


def pyramid_layout(keys, block_size, branching=2, max_level=None):
    """(offsets, lengths) of levels 0..max_level (None: up to the root)."""
    levels = ctypes.c_int32()
    offsets = (ctypes.c_int32 * _lib.MAX_LEVELS)()
    lengths = (ctypes.c_int32 * _lib.MAX_LEVELS)()
    _lib.check(_lib.library().pisa_pyramid_layout(
        keys, block_size, branching, -1 if max_level is None else max_level,
        ctypes.byref(levels), offsets, lengths))
    return list(offsets[:levels.value]), list(lengths[:levels.value])


def build_pyramid_storage(keys, block_size, branching=2, max_level=None):
    """Packed storage [B, sum(M_l), Hkv, D] plus host offsets/lengths."""
    keys = kernel_layout(keys)
    batch, length, heads, dim = keys.shape
    offsets, lengths = pyramid_layout(length, block_size, branching, max_level)
    storage = torch.empty((batch, offsets[-1] + lengths[-1], heads, dim), device=keys.device,
                          dtype=keys.dtype)
    with torch.cuda.device(keys.device):
        _lib.check(_lib.library().pisa_build_pyramid(
            ptr(keys), keys.stride(0), keys.stride(1), batch, length, heads, dim, block_size,
            branching, -1 if max_level is None else max_level, ptr(storage), storage.stride(0),
            dtype_code(keys, ""), stream_of(keys)))
    return storage, offsets, lengths


def build_pyramid(keys, block_size, *, backend="auto", max_level=None, branching=2):
    """Leaf means first, then means of ``branching`` children, up to the root or ``max_level``.

    Returns views into one packed allocation.
    """
    if max_level is not None and (type(max_level) is not int or max_level < 0):
        raise ValueError("max_level must be a nonnegative integer or None")
    if block_size < 1:
        raise ValueError("pool size must be positive")
    if branching < 2:
        raise ValueError("branching must be at least 2")
    _check_pool_input(keys, backend)
    storage, offsets, lengths = build_pyramid_storage(keys, block_size, branching, max_level)
    return [storage[:, o:o + n] for o, n in zip(offsets, lengths)]


mean_pooling_fn = mean_pool
