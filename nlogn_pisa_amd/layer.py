"""The PISA attention layer on the HIP operators: ``PyramidSparseAttention``.

Mirrors ``xmixers/xmixers/modules/token_mixers/vanilla_attention/pyramid_sparse_attention.py``
(``token_positions`` :6-11, ``full_attention`` :13-69, the layer :71-222) and
the split-half rotary encoding of ``xmixers/xmixers/modules/pes/lrpe.py`` /
``pisa/pisa/ops/lrpe/rotary_torch.py``: q/k/v projections, rotary encoding at
sequence or document positions, a ``PyramidCache`` / ``TensorCache`` for decode,
``select_blocks`` + ``sparse_attention`` (``attention_method`` pisa, pisa1,
pisa2) or dense causal attention ("full"), and the output projection.  The
projections are library GEMMs (torch ``nn.Linear``); rotary encoding, pooling,
routing and attention are the HIP kernels of ``libpisa_hip.so``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from ._common import dtype_code, positions_layout, ptr, require_gpu, stream_of
from .attention import sparse_attention
from .cache import PyramidCache, TensorCache
from .selection import select_blocks
from .validation import sequence_slices, validate_qkv


@dataclass
class PisaLayerConfig:
    """The fields of ``xmixers/xmixers/pisa_config.py:8-42`` the attention layer reads."""

    hidden_size: int = 1024
    num_attention_heads: int = 32
    num_key_value_heads: int = 2
    head_dim: int = 64
    attention_method: str = "pisa"
    block_size: int = 64
    topk: int = 8
    prefill_routing: str | None = None
    leaf_tile: int = 4
    force_first: bool = True
    force_recent: int = 2
    rope_theta: float = 10000.0
    rope_fraction: float = 0.5
    rope_position_mode: str = "document"
    bias: bool = False
    backend: str = "auto"
    branching: int = 2

    def __post_init__(self):
        dims = (self.hidden_size, self.num_attention_heads, self.num_key_value_heads,
                self.head_dim, self.block_size, self.topk)
        if any(value <= 0 for value in dims):
            raise ValueError("Model dimensions and block budgets must be positive")
        if self.rope_position_mode not in {"document", "sequence"}:
            raise ValueError("rope_position_mode must be document or sequence")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("Query heads must be divisible by KV heads")
        if self.head_dim % 2 or not 0 <= self.rope_fraction <= 1:
            raise ValueError("head_dim must be even and rope_fraction in [0, 1]")
        if self.attention_method not in {"pisa", "pisa1", "pisa2", "full"}:
            raise ValueError("attention_method must be pisa, pisa1, pisa2 or full")
        if self.prefill_routing not in {None, "auto", "grouped", "fused"}:
            raise ValueError("prefill_routing must be auto, grouped, fused or None")


class _Rotary(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, frequency, positions):
        ctx.save_for_backward(frequency, positions)
        return _rotate(x, frequency, positions, inverse=False)

    @staticmethod
    def backward(ctx, grad):
        frequency, positions = ctx.saved_tensors
        return _rotate(grad, frequency, positions, inverse=True), None, None


def _rotate(x, frequency, positions, inverse):
    require_gpu(x, "rotary encoding")
    code = dtype_code(x, "rotary encoding supports FP16, BF16 and FP32")
    if x.ndim != 4 or x.stride(-1) != 1 or x.stride(-2) != x.shape[-1]:
        x = x.contiguous()
    batch, tokens, heads, dim = x.shape
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    frequency = frequency.to(device=x.device, dtype=torch.float32).contiguous()
    positions = positions_layout(positions.to(x.device)).expand(batch, tokens)
    with torch.cuda.device(x.device):
        _lib.check(_lib.library().pisa_rotary(
            ptr(x), x.stride(0), x.stride(1), ptr(out), out.stride(0), out.stride(1), batch, tokens,
            heads, dim, ptr(frequency), ptr(positions), positions.stride(0), int(inverse), code,
            stream_of(x)))
    return out


def rotary(x, frequency, positions):
    """Split-half rotary encoding of ``x [B,T,H,D]`` at ``positions [B or 1, T]``
    (``rotary_torch.py:5-10``): pairs (f, f + D/2) turn by positions x frequency[f]."""
    return _Rotary.apply(x, frequency.flatten(), positions)


class RotaryEmbedding(nn.Module):
    """``RotaryEmbedding`` of ``xmixers/xmixers/modules/pes/lrpe.py:37-39`` (type 3: the
    first ``head_dim // 2 * fraction`` frequencies turn, the rest stay zero)."""

    def __init__(self, head_dim, base, fraction):
        super().__init__()
        # the reference's table: float32 powers formed on the CPU (lrpe.py:20-28)
        theta = base ** (-2 / head_dim * torch.arange(head_dim // 2, dtype=torch.int64,
                                                      device="cpu")).float()
        count = int(head_dim // 2 * fraction)
        theta[count:] = 0
        self.register_buffer("theta", theta.reshape(1, -1), persistent=False)

    def forward(self, x, positions):
        return rotary(x, self.theta, positions)


def token_positions(length, device, cu_seqlens=None, offset=0):
    """Rotary positions ``[1, length]`` (``pyramid_sparse_attention.py:6-11``): offset + t,
    restarted at each document of a packed sequence."""
    positions = torch.arange(length, device=device)[None] + offset
    if cu_seqlens is not None:
        for begin, end in sequence_slices(cu_seqlens, length):
            positions[:, begin:end] -= begin
    return positions


def full_attention(q, k, v, cu_seqlens=None, query_offset=0):
    """Dense causal GQA attention (``pyramid_sparse_attention.py:13-69``) by SDPA."""
    validate_qkv(q, k, v)
    if cu_seqlens is not None:
        if q.shape[0] != 1 or q.shape[1] != k.shape[1] or query_offset != 0:
            raise ValueError("Packed full attention requires a complete prefill")
        return torch.cat([full_attention(q[:, a:b], k[:, a:b], v[:, a:b])
                          for a, b in sequence_slices(cu_seqlens, k.shape[1])], dim=1)
    queries, keys, values = (x.transpose(1, 2) for x in (q, k, v))
    gqa = q.shape[2] != k.shape[2]
    if query_offset == 0 and q.shape[1] == k.shape[1]:
        result = F.scaled_dot_product_attention(queries, keys, values, is_causal=True,
                                                enable_gqa=gqa)
    else:
        qpos = torch.arange(q.shape[1], device=q.device) + query_offset
        kpos = torch.arange(k.shape[1], device=q.device)
        result = F.scaled_dot_product_attention(queries, keys, values,
                                                attn_mask=kpos[None] <= qpos[:, None],
                                                enable_gqa=gqa)
    return result.transpose(1, 2)


class PyramidSparseAttention(nn.Module):
    """The PISA attention layer (``pyramid_sparse_attention.py:71-222``).

    ``forward(x, cu_seqlens=None, cache=None, use_cache=False, backend=None,
    attention_mask=None, past_key_values=None)`` returns ``(output, next_cache)``;
    with ``use_cache`` the keys live in a ``PyramidCache`` (pisa methods) that
    ``select_blocks`` reads directly, appended on the GPU each step.
    """

    def __init__(self, config, layer_idx=0):
        super().__init__()
        if config.attention_method == "nsa":
            raise ValueError("attention_method 'nsa' is not provided by nlogn_pisa_amd")
        self.config = config
        self.layer_idx = layer_idx
        q_width = config.num_attention_heads * config.head_dim
        kv_width = config.num_key_value_heads * config.head_dim
        self.q_proj = nn.Linear(config.hidden_size, q_width, bias=config.bias)
        self.k_proj = nn.Linear(config.hidden_size, kv_width, bias=config.bias)
        self.v_proj = nn.Linear(config.hidden_size, kv_width, bias=config.bias)
        self.o_proj = nn.Linear(q_width, config.hidden_size, bias=config.bias)
        self.rope = RotaryEmbedding(config.head_dim, config.rope_theta, config.rope_fraction)

    def forward(self, x, cu_seqlens=None, cache=None, use_cache=False, backend=None,
                attention_mask=None, past_key_values=None, **kwargs):
        if attention_mask is not None and not bool(attention_mask.all()):
            raise ValueError("Remove evaluation padding before native attention")
        if past_key_values is not None:
            cache = past_key_values[self.layer_idx] if len(past_key_values) > self.layer_idx else None
        config = self.config
        batch, length, _ = x.shape
        q = self.q_proj(x).view(batch, length, config.num_attention_heads, config.head_dim)
        raw_k = self.k_proj(x).view(batch, length, config.num_key_value_heads, config.head_dim)
        v = self.v_proj(x).view(batch, length, config.num_key_value_heads, config.head_dim)
        offset = 0 if cache is None else cache["k"].shape[1]
        boundaries = cu_seqlens if config.rope_position_mode == "document" else None
        positions = token_positions(length, x.device, boundaries, offset)
        q = self.rope(q, positions)
        new_k = self.rope(raw_k, positions)
        pyramid = None
        next_cache = None
        if use_cache:
            next_cache = {} if cache is None else cache
            if config.attention_method != "full":
                pyramid = (PyramidCache.from_keys(new_k, block_size=config.block_size,
                                                  branching=config.branching)
                           if cache is None else cache["pyramid"].append(new_k))
                next_cache["pyramid"] = pyramid
                k = pyramid.keys
            else:
                keys = (TensorCache.from_tensor(new_k) if cache is None
                        else cache["key_storage"].append(new_k))
                next_cache["key_storage"] = keys
                k = keys.tensor
            values = (TensorCache.from_tensor(v) if cache is None
                      else cache["value_storage"].append(v))
            next_cache.update(k=k, v=values.tensor, value_storage=values)
            v = values.tensor
        else:
            k = new_k if cache is None else torch.cat((cache["k"], new_k), dim=1)
            if cache is not None:
                v = torch.cat((cache["v"], v), dim=1)
        backend = backend or config.backend
        if config.attention_method == "full":
            output = full_attention(q, k, v, cu_seqlens, offset)
        else:
            schedule = ("fused" if cache is not None and length == 1
                        else (config.prefill_routing or "auto"))
            indices = select_blocks(q, k, method=config.attention_method,
                                    block_size=config.block_size, topk=config.topk,
                                    cu_seqlens=cu_seqlens, query_offset=offset,
                                    force_first=config.force_first,
                                    force_recent=config.force_recent, backend=backend,
                                    pyramid=pyramid, leaf_tile=config.leaf_tile,
                                    routing_schedule=schedule, branching=config.branching)
            output = sparse_attention(q, k, v, indices, block_size=config.block_size,
                                      cu_seqlens=cu_seqlens, query_offset=offset,
                                      backend=backend)
        if past_key_values is not None and use_cache:
            while len(past_key_values) <= self.layer_idx:
                past_key_values.append(None)
            past_key_values[self.layer_idx] = next_cache
            next_cache = past_key_values
        return self.o_proj(output.reshape(batch, length, -1)), next_cache
