"""MI355X-native PISA block selection and block-sparse attention.

Drop-in for the ``pisa-attention`` operator API of Aphelios-Tang/NlogN_PISA
(``pisa/pisa/__init__.py``): ``select_blocks`` / ``top_k_pyramid_fn``,
``sparse_attention`` / ``sparse_attn_fn``, ``mean_pool`` / ``mean_pooling_fn``
``build_pyramid``, the flat BSA baseline ``bsa_fn``, the decode ``PyramidCache``
and the ``PyramidSparseAttention`` layer, computed by hand-written gfx950 HIP kernels in
``libpisa_hip.so`` (C ABI: ``include/pisa_hip.h``).
"""

from .cache import PyramidCache, TensorCache
from .layer import (PisaLayerConfig, PyramidSparseAttention, RotaryEmbedding, full_attention,
                    rotary, rotary_fn, token_positions)
from .bsa import bsa_fn
from .attention import sparse_attention, sparse_attention_with_lse, sparse_attn_fn
from .pooling import build_pyramid, mean_pool, mean_pooling_fn
from .selection import leaf_scores, routing_geometry, select_blocks, top_k_pyramid_fn
from .validation import packed_queries, query_positions, sequence_slices, validate_qkv

__version__ = "0.1.0"
__all__ = [
    "select_blocks", "top_k_pyramid_fn", "sparse_attention", "sparse_attn_fn",
    "sparse_attention_with_lse", "mean_pool", "mean_pooling_fn", "build_pyramid",
    "routing_geometry", "leaf_scores", "validate_qkv", "query_positions", "packed_queries",
    "sequence_slices", "PyramidCache", "TensorCache", "PisaLayerConfig", "PyramidSparseAttention",
    "RotaryEmbedding", "rotary", "rotary_fn", "token_positions", "full_attention", "bsa_fn",
]
