"""Decode-time token and key-pyramid caches: ``TensorCache`` and ``PyramidCache``.

Mirrors ``xmixers/xmixers/utils/attention_cache.py:8-140``.  ``TensorCache``
keeps appended [B, T, H, D] tokens in a buffer whose capacity grows to the next
power of two.  ``PyramidCache`` keeps every level of the key pyramid in one
allocation -- level capacities are the next power of two of the leaf count, then
``ceil(c / branching)`` down to 1, so level offsets change only when the leaf
capacity grows -- and ``append`` recomputes only the changed leaf and its
ancestors on the GPU (``pisa_pyramid_append``), with the numerics of
``build_pyramid``.  The cache plugs into ``select_blocks(pyramid=...)``: it
exposes ``storage``, ``starts``/``offsets``, ``lengths`` and ``level_sizes``, and
its views have a batch stride larger than their length.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import dtype_code, ptr, require_gpu, stream_of


class TensorCache:
    """Append-only, detached [B, T, H, D] storage for inference."""

    def __init__(self):
        self.buffer = None
        self.length = 0

    @classmethod
    def from_tensor(cls, tensor):
        return cls().append(tensor)

    @property
    def tensor(self):
        if self.buffer is None:
            raise ValueError("the token cache is empty")
        return self.buffer[:, : self.length]

    @torch.no_grad()
    def append(self, tensor):
        if tensor.ndim != 4 or tensor.shape[1] == 0 or not tensor.is_floating_point():
            raise ValueError("new tokens must be a nonempty [B,T,H,D] floating tensor")
        if self.buffer is not None:
            held = (self.buffer.shape[0], *self.buffer.shape[2:], self.buffer.dtype,
                    self.buffer.device)
            if held != (tensor.shape[0], *tensor.shape[2:], tensor.dtype, tensor.device):
                raise ValueError("cache batch, heads, dimension, dtype and device cannot change")
        end = self.length + tensor.shape[1]
        if self.buffer is None or end > self.buffer.shape[1]:
            capacity = 1 << (end - 1).bit_length()
            grown = tensor.new_empty(tensor.shape[0], capacity, *tensor.shape[2:])
            if self.buffer is not None:
                grown[:, : self.length].copy_(self.tensor)
            self.buffer = grown
        self.buffer[:, self.length : end].copy_(tensor)
        self.length = end
        return self


class PyramidCache:
    """Key means of every pyramid level in one allocation, updated incrementally.

    ``branching`` generalises the reference's binary pyramid (2, the default).
    """

    def __init__(self, block_size=64, branching=2):
        if block_size < 1:
            raise ValueError("block_size must be positive")
        if branching < 2:
            raise ValueError("branching must be at least 2")
        self.block_size = block_size
        self.branching = branching
        self.tokens = TensorCache()
        self.storage = None
        self.capacities = ()
        self.starts = ()
        self.sizes = []
        self.offsets = None
        self.lengths = None

    @classmethod
    def from_keys(cls, keys, block_size=64, branching=2):
        return cls(block_size, branching).append(keys)

    @property
    def length(self):
        return self.tokens.length

    @property
    def key_buffer(self):
        return self.tokens.buffer

    @property
    def keys(self):
        return self.tokens.tensor

    @property
    def level_sizes(self):
        return tuple(self.sizes)

    @property
    def buffers(self):
        if self.storage is None:
            return []
        return [self.storage[:, start:start + capacity]
                for start, capacity in zip(self.starts, self.capacities)]

    @property
    def levels(self):
        return [buffer[:, :size] for buffer, size in zip(self.buffers, self.sizes)]

    def reserve(self, reference, leaves):
        """Room for ``leaves`` leaf means; grows (and re-lays out) to a power of two."""
        if self.capacities and leaves <= self.capacities[0]:
            return
        capacity = 1 << (leaves - 1).bit_length()
        capacities, starts, total = [], [], 0
        while True:
            capacities.append(capacity)
            starts.append(total)
            total += capacity
            if capacity == 1:
                break
            capacity = -(-capacity // self.branching)
        storage = reference.new_empty(reference.shape[0], total, *reference.shape[2:])
        for start, previous in zip(starts, self.levels):
            storage[:, start:start + previous.shape[1]].copy_(previous)
        self.storage = storage
        self.capacities, self.starts = tuple(capacities), tuple(starts)
        self.offsets = torch.tensor(starts, device=reference.device, dtype=torch.int32)
        self.lengths = torch.zeros(len(starts), device=reference.device, dtype=torch.int32)

    @torch.no_grad()
    def append(self, keys):
        """Append [B, T, Hkv, D] keys; recompute the changed leaves and their ancestors."""
        require_gpu(keys, "the pyramid cache")
        code = dtype_code(keys, "HIP pooling requires float16, bfloat16, or float32 dtype")
        previous = self.length
        self.tokens.append(keys)
        length = self.length
        leaves = -(-length // self.block_size)
        self.reserve(keys, leaves)
        source = self.tokens.buffer
        batch, _, heads, dim = source.shape
        levels = len(self.starts)
        starts = (_lib.ctypes.c_int32 * levels)(*self.starts)
        with torch.cuda.device(keys.device):
            _lib.check(_lib.library().pisa_pyramid_append(
                ptr(source), source.stride(0), source.stride(1), batch, previous, length, heads,
                dim, self.block_size, self.branching, levels, starts, ptr(self.storage),
                self.storage.stride(0), code, stream_of(keys)))
        sizes, count = [], leaves
        for _ in range(levels):
            sizes.append(count)
            count = -(-count // self.branching)
        self.sizes = sizes
        self.lengths.copy_(torch.tensor(sizes, dtype=torch.int32))
        return self
