"""Decode-time caches: appended key/value tokens and the key pyramid over them.

Format and attributes of ``xmixers/xmixers/utils/attention_cache.py:8-140``
(``TensorCache``, ``PyramidCache``), which ``select_blocks(pyramid=...)`` and the
layer's decode path consume: one ``storage`` allocation ``[B, sum(capacity_l),
Hkv, D]`` holding every level, host ``starts``/``capacities``/``level_sizes``,
device ``offsets``/``lengths`` (int32), views whose batch stride exceeds their
length.

Design here: level capacities and live sizes both come from the library's
``pisa_pyramid_layout`` (capacities are the layout of a power-of-two leaf
count, so they halve - or divide by ``branching`` - down to one); the means are
written by the HIP ``pisa_pyramid_append`` kernel, which recomputes only the
changed leaves and their ancestors.  When the leaf capacity grows, the new
storage is rebuilt from all held keys by the same kernel (a pass over the keys
per doubling) instead of copying the old levels.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import dtype_code, ptr, require_gpu, stream_of
from .pooling import pyramid_layout


def _pow2_at_least(n):
    return 1 << max(0, int(n) - 1).bit_length()


class TensorCache:
    """Append-only, detached [B, T, H, D] token storage for inference.

    ``buffer`` holds a power-of-two number of token slots; ``tensor`` is the
    filled prefix of ``length`` tokens.
    """

    def __init__(self):
        self.buffer = None
        self.length = 0

    @classmethod
    def from_tensor(cls, tensor):
        cache = cls()
        cache.append(tensor)
        return cache

    @property
    def tensor(self):
        if self.buffer is None:
            raise ValueError("the token cache is empty")
        return self.buffer.narrow(1, 0, self.length)

    @staticmethod
    def _signature(t):
        return t.shape[0], tuple(t.shape[2:]), t.dtype, t.device

    def _admit(self, tensor):
        if tensor.ndim != 4 or tensor.shape[1] == 0 or not tensor.is_floating_point():
            raise ValueError("new tokens must be a nonempty [B,T,H,D] floating tensor")
        if self.buffer is not None and self._signature(self.buffer) != self._signature(tensor):
            raise ValueError("cache batch, heads, dimension, dtype and device cannot change")

    def _room_for(self, tokens, like):
        held = 0 if self.buffer is None else self.buffer.shape[1]
        if tokens <= held:
            return
        slots = like.new_empty((like.shape[0], _pow2_at_least(tokens), *like.shape[2:]))
        if self.length:
            slots.narrow(1, 0, self.length).copy_(self.tensor)
        self.buffer = slots

    @torch.no_grad()
    def append(self, tensor):
        self._admit(tensor)
        count = tensor.shape[1]
        self._room_for(self.length + count, tensor)
        self.buffer.narrow(1, self.length, count).copy_(tensor)
        self.length += count
        return self


class PyramidCache:
    """Key means of every pyramid level in one allocation, updated incrementally on the GPU.

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
        cache = cls(block_size, branching)
        cache.append(keys)
        return cache

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
        return [self.storage.narrow(1, s, c) for s, c in zip(self.starts, self.capacities)]

    @property
    def levels(self):
        return [self.storage.narrow(1, s, n) for s, n in zip(self.starts, self.sizes)]

    def _live_sizes(self):
        """Nodes per level for the held tokens: the pyramid layout of ``length``
        keys, continued at one node up to the capacity's level count."""
        if not self.length:
            return [0] * len(self.starts)
        _, live = pyramid_layout(self.length, self.block_size, self.branching)
        return (live + [1] * len(self.starts))[:len(self.starts)]

    def _recompute(self, previous):
        """Means of the leaves from ``previous // block_size`` on and their
        ancestors, from the held keys (``previous = 0``: every node)."""
        source = self.tokens.buffer
        batch, _, heads, dim = source.shape
        starts = (_lib.ctypes.c_int32 * len(self.starts))(*self.starts)
        code = dtype_code(source, "HIP pooling requires float16, bfloat16, or float32 dtype")
        with torch.cuda.device(source.device):
            _lib.check(_lib.library().pisa_pyramid_append(
                ptr(source), source.stride(0), source.stride(1), batch, previous, self.length,
                heads, dim, self.block_size, self.branching, len(self.starts), starts,
                ptr(self.storage), self.storage.stride(0), code, stream_of(source)))
        self.sizes = self._live_sizes()
        self.lengths = torch.tensor(self.sizes, dtype=torch.int32).to(source.device,
                                                                      non_blocking=True)

    def reserve(self, reference, leaves):
        """Room for ``leaves`` leaf means (a power-of-two capacity).  Growing re-lays
        out the levels and rebuilds them from the held keys; returns whether it grew."""
        if self.capacities and leaves <= self.capacities[0]:
            return False
        cap = _pow2_at_least(leaves)
        starts, capacities = pyramid_layout(cap * self.block_size, self.block_size,
                                            self.branching)
        total = starts[-1] + capacities[-1]
        self.storage = reference.new_empty((reference.shape[0], total, *reference.shape[2:]))
        self.starts, self.capacities = tuple(starts), tuple(capacities)
        self.offsets = torch.tensor(starts, dtype=torch.int32).to(reference.device)
        if self.length:
            self._recompute(0)
        else:
            self.sizes = [0] * len(starts)
            self.lengths = torch.zeros(len(starts), dtype=torch.int32, device=reference.device)
        return True

    @torch.no_grad()
    def append(self, keys):
        """Append [B, T, Hkv, D] keys; recompute the changed leaves and their ancestors."""
        require_gpu(keys, "the pyramid cache")
        dtype_code(keys, "HIP pooling requires float16, bfloat16, or float32 dtype")
        previous = self.length
        self.tokens.append(keys)
        leaves = -(-self.length // self.block_size)
        if not self.reserve(keys, leaves):       # a grown storage is rebuilt already
            self._recompute(previous)
        return self
