"""The PISA attention layer on the HIP operators: ``PyramidSparseAttention``.

Interface of ``xmixers/xmixers/modules/token_mixers/vanilla_attention/pyramid_sparse_attention.py``
(the layer :71-222, ``token_positions`` :6-11, ``full_attention`` :13-69): the
constructor takes the config fields of ``xmixers/xmixers/pisa_config.py:8-79``,
the parameters are ``q_proj``/``k_proj``/``v_proj``/``o_proj`` and the rotary
table ``rope.theta`` (``xmixers/xmixers/modules/pes/lrpe.py:18-39``, type 3),
``forward(x, cu_seqlens, cache, use_cache, backend, attention_mask,
past_key_values)`` returns ``(output, next_cache)`` and the decode cache is a
dict with the keys ``k``, ``v``, ``value_storage`` and ``pyramid`` (pisa
methods) or ``key_storage`` (bsa, full).

Work per call: projections (torch GEMMs), the split-half rotary encoding
(``pisa_rotary``), then ``select_blocks`` + ``sparse_attention`` for
``attention_method`` pisa/pisa1/pisa2/bsa or dense causal attention for
"full".  Decode keeps keys in a ``PyramidCache`` whose levels ``select_blocks``
reads directly and which the HIP append kernel updates in place.
"""

from __future__ import annotations

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

PYRAMID_METHODS = ("pisa1", "pisa2", "pisa")
METHODS = ("full", "bsa") + PYRAMID_METHODS


@dataclass
class PisaLayerConfig:
    """The fields of ``xmixers/xmixers/pisa_config.py:8-42`` the attention layer reads
    (plus ``branching``, the pyramid's fan-out; 2 is the reference's)."""

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
        sizes = [self.hidden_size, self.num_attention_heads, self.num_key_value_heads,
                 self.head_dim, self.block_size, self.topk]
        if min(sizes) <= 0:
            raise ValueError("Model dimensions and block budgets must be positive")
        if self.rope_position_mode not in ("document", "sequence"):
            raise ValueError("rope_position_mode must be document or sequence")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("Query heads must be divisible by KV heads")
        if self.head_dim % 2 or not 0 <= self.rope_fraction <= 1:
            raise ValueError("RoPE needs an even head dimension and a fraction in [0, 1]")
        if self.attention_method not in METHODS + ("nsa",):
            raise ValueError(f"Unknown attention method: {self.attention_method}")
        # pisa_config.py:72-75: pisa1 routes fused, the others grouped, unless told
        if self.prefill_routing is None:
            self.prefill_routing = "fused" if self.attention_method == "pisa1" else "grouped"
        if self.prefill_routing not in ("grouped", "fused", "auto"):
            raise ValueError("prefill_routing must be grouped or fused")
        if type(self.leaf_tile) is not int or self.leaf_tile not in (1, 2, 4):
            raise ValueError("leaf_tile must be 1, 2 or 4")
        if self.rope_theta <= 0:
            raise ValueError("RoPE base and normalization epsilon must be positive")


# ---------------------------------------------------------------- rotary encoding

def _turn(x, frequency, positions, inverse):
    """pisa_rotary over ``x [B,T,H,D]``: a new tensor turned by +-positions x frequency."""
    require_gpu(x, "rotary encoding")
    code = dtype_code(x, "rotary encoding supports FP16, BF16 and FP32")
    if x.ndim != 4:
        raise ValueError("rotary encoding expects [B,T,H,D] input")
    src = x if (x.stride(-1) == 1 and x.stride(-2) == x.shape[-1]) else x.contiguous()
    batch, tokens, heads, dim = src.shape
    dst = torch.empty(src.shape, device=src.device, dtype=src.dtype)
    table = frequency.to(device=src.device, dtype=torch.float32).reshape(-1).contiguous()
    where = positions_layout(positions.to(src.device)).expand(batch, tokens)
    with torch.cuda.device(src.device):
        _lib.check(_lib.library().pisa_rotary(
            ptr(src), src.stride(0), src.stride(1), ptr(dst), dst.stride(0), dst.stride(1),
            batch, tokens, heads, dim, ptr(table), ptr(where), where.stride(0), int(inverse),
            code, stream_of(src)))
    return dst


class _RotaryFn(torch.autograd.Function):
    """A rotation's gradient is the opposite rotation of the upstream gradient."""

    @staticmethod
    def forward(ctx, x, frequency, positions):
        ctx.save_for_backward(frequency, positions)
        return _turn(x, frequency, positions, inverse=False)

    @staticmethod
    def backward(ctx, grad):
        frequency, positions = ctx.saved_tensors
        return _turn(grad, frequency, positions, inverse=True), None, None


def rotary(x, frequency, positions):
    """Split-half rotary encoding of ``x [B,T,H,D]`` at ``positions [B or 1, T]``
    (``rotary_torch.py:5-10``): pairs (f, f + D/2) turn by positions x frequency[f]."""
    return _RotaryFn.apply(x, frequency.reshape(-1), positions)


def rotary_fn(x, frequency, positions, *, use_triton=True):
    """``rotary_fn`` (``pisa/pisa/ops/lrpe/rotary.py:9-15``): the HIP rotary for either
    ``use_triton`` choice (the reference's eager and Triton paths compute the same
    float32 rotation); a CPU tensor raises."""
    return rotary(x, frequency.flatten().to(device=x.device, dtype=torch.float32), positions)


def rotary_frequency(head_dim, base, fraction):
    """Float32 frequencies base^(-2 i / head_dim) for i < head_dim // 2 * fraction,
    zero after (``lrpe.py:20-28``, type 3).  Both the exponent and the power are
    evaluated in float32 on the CPU, so every device gets the same table."""
    half = head_dim // 2
    exponent = torch.arange(half, dtype=torch.int64) * (-2 / head_dim)
    table = torch.pow(base, exponent).float()
    table[int(half * fraction):] = 0
    return table


class RotaryEmbedding(nn.Module):
    """``RotaryEmbedding`` of ``lrpe.py:37-39``: a fixed [1, head_dim // 2] table ``theta``."""

    def __init__(self, head_dim, base, fraction):
        super().__init__()
        self.register_buffer("theta", rotary_frequency(head_dim, base, fraction)[None],
                             persistent=False)

    def forward(self, x, positions):
        return rotary(x, self.theta, positions)


# ---------------------------------------------------------------- positions and dense attention

def token_positions(length, device, cu_seqlens=None, offset=0):
    """Rotary positions ``[1, length]``: ``offset + t``, counted from each document's
    first token when ``cu_seqlens`` packs several (``pyramid_sparse_attention.py:6-11``)."""
    steps = torch.arange(length, device=device)
    if cu_seqlens is None:
        return (steps + offset)[None]
    starts = cu_seqlens[:-1].to(device=device, dtype=torch.long)
    # the document of token t is the last one starting at or before t
    owner = (torch.searchsorted(starts, steps, right=True) - 1).clamp(min=0)
    return (steps - starts[owner] + offset)[None]


def _sdpa(q, k, v, query_offset):
    """Causal GQA attention of one sequence; query t sits at key position t + offset."""
    queries, keys, values = (t.transpose(1, 2) for t in (q, k, v))
    gqa = q.shape[2] != k.shape[2]
    if query_offset == 0 and q.shape[1] == k.shape[1]:
        mixed = F.scaled_dot_product_attention(queries, keys, values, is_causal=True,
                                               enable_gqa=gqa)
    else:
        seen = (torch.arange(k.shape[1], device=q.device)[None]
                <= torch.arange(q.shape[1], device=q.device)[:, None] + query_offset)
        mixed = F.scaled_dot_product_attention(queries, keys, values, attn_mask=seen,
                                               enable_gqa=gqa)
    return mixed.transpose(1, 2)


def full_attention(q, k, v, cu_seqlens=None, query_offset=0):
    """Dense causal GQA attention (``pyramid_sparse_attention.py:13-69``) by torch SDPA;
    packed documents attend only within themselves."""
    validate_qkv(q, k, v)
    if cu_seqlens is None:
        return _sdpa(q, k, v, query_offset)
    if q.shape[0] != 1 or q.shape[1] != k.shape[1] or query_offset != 0:
        raise ValueError("Packed full attention requires a complete prefill")
    docs = sequence_slices(cu_seqlens, k.shape[1])
    return torch.cat([_sdpa(q[:, a:b], k[:, a:b], v[:, a:b], 0) for a, b in docs], dim=1)


# ---------------------------------------------------------------- the layer

def _grow(storage, tensor, make):
    """Append ``tensor`` to a cache entry, creating it with ``make`` when absent."""
    return make(tensor) if storage is None else storage.append(tensor)


class PyramidSparseAttention(nn.Module):
    """The PISA attention layer (``pyramid_sparse_attention.py:71-222``) on HIP kernels.

    ``attention_method`` "nsa" (the NSA baseline of the reference) is not provided.
    """

    def __init__(self, config, layer_idx=0):
        super().__init__()
        if config.attention_method == "nsa":
            raise ValueError("attention_method 'nsa' is not provided by nlogn_pisa_amd")
        self.config = config
        self.layer_idx = layer_idx
        heads_q = config.num_attention_heads * config.head_dim
        heads_kv = config.num_key_value_heads * config.head_dim
        linear = lambda n_in, n_out: nn.Linear(n_in, n_out, bias=config.bias)
        self.q_proj = linear(config.hidden_size, heads_q)
        self.k_proj = linear(config.hidden_size, heads_kv)
        self.v_proj = linear(config.hidden_size, heads_kv)
        self.o_proj = linear(heads_q, config.hidden_size)
        self.rope = RotaryEmbedding(config.head_dim, config.rope_theta, config.rope_fraction)

    def _split_heads(self, x):
        c = self.config
        b, t, _ = x.shape
        return (self.q_proj(x).view(b, t, c.num_attention_heads, c.head_dim),
                self.k_proj(x).view(b, t, c.num_key_value_heads, c.head_dim),
                self.v_proj(x).view(b, t, c.num_key_value_heads, c.head_dim))

    def _keep(self, cache, k_new, v_new):
        """Extend (or open) the decode cache; returns (k, v, pyramid, cache dict)."""
        c = self.config
        state = {} if cache is None else cache
        pyramid = None
        if c.attention_method in PYRAMID_METHODS:
            pyramid = _grow(None if cache is None else cache["pyramid"], k_new,
                            lambda t: PyramidCache.from_keys(t, c.block_size, c.branching))
            state["pyramid"] = pyramid
            keys = pyramid.keys
        else:
            stored = _grow(None if cache is None else cache["key_storage"], k_new,
                           TensorCache.from_tensor)
            state["key_storage"] = stored
            keys = stored.tensor
        values = _grow(None if cache is None else cache["value_storage"], v_new,
                       TensorCache.from_tensor)
        state["k"], state["v"], state["value_storage"] = keys, values.tensor, values
        return keys, values.tensor, pyramid, state

    def _mix(self, q, k, v, pyramid, cu_seqlens, offset, decoding, backend):
        """Dense, or selected-block attention over the keys ``k`` -> [B, Tq, Hq, D]."""
        c = self.config
        if c.attention_method == "full":
            return full_attention(q, k, v, cu_seqlens, offset)
        routing = {}
        if c.attention_method in PYRAMID_METHODS:
            routing = dict(routing_schedule="fused" if decoding else c.prefill_routing,
                           leaf_tile=c.leaf_tile, branching=c.branching)
        ids = select_blocks(q, k, method=c.attention_method, block_size=c.block_size,
                            topk=c.topk, cu_seqlens=cu_seqlens, query_offset=offset,
                            force_first=c.force_first, force_recent=c.force_recent,
                            backend=backend, pyramid=pyramid, **routing)
        return sparse_attention(q, k, v, ids, block_size=c.block_size, cu_seqlens=cu_seqlens,
                                query_offset=offset, backend=backend)

    def forward(self, x, cu_seqlens=None, cache=None, use_cache=False, backend=None,
                attention_mask=None, past_key_values=None, **kwargs):
        if attention_mask is not None and not bool(attention_mask.all()):
            raise ValueError("Remove evaluation padding before native attention")
        c = self.config
        if past_key_values is not None:
            cache = (past_key_values[self.layer_idx] if self.layer_idx < len(past_key_values)
                     else None)
        q, k_new, v_new = self._split_heads(x)
        offset = cache["k"].shape[1] if cache is not None else 0
        docs = cu_seqlens if c.rope_position_mode == "document" else None
        where = token_positions(x.shape[1], x.device, docs, offset)
        q, k_new = self.rope(q, where), self.rope(k_new, where)
        state = None
        if use_cache:
            k, v, pyramid, state = self._keep(cache, k_new, v_new)
        else:
            pyramid = None
            k, v = ((k_new, v_new) if cache is None else
                    (torch.cat((cache["k"], k_new), 1), torch.cat((cache["v"], v_new), 1)))
        decoding = cache is not None and x.shape[1] == 1
        out = self._mix(q, k, v, pyramid, cu_seqlens, offset, decoding, backend or c.backend)
        if use_cache and past_key_values is not None:
            past_key_values.extend([None] * (self.layer_idx + 1 - len(past_key_values)))
            past_key_values[self.layer_idx] = state
            state = past_key_values
        return self.o_proj(out.flatten(2)), state
