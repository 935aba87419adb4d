"""Write golden vectors of the reference's flat BSA routing (Torch path).

Run ONCE, in the build container only, with the reference checkout on disk:

    PYTHONPATH=/root/reference/pisa python tests/golden/make_golden_bsa.py

It imports ``pisa`` (Aphelios-Tang/NlogN_PISA, ``pisa/pisa``) and records, as
plain arrays in ``tests/golden/bsa.npz``.  Inputs are not stored: ``case_inputs``
regenerates them from seeded CPU generators and the file keeps the sha256 of each
(fp32 bytes, or the bf16 bit patterns), so a test detects generator drift:

* ``streaming_topk`` (``ops/flash_sparse_attn/bsa/bsa_torch.py:28-58``) on score
  rows full of exact ties (repeated palette values, zeros, -1 padding ids, tails
  that are not a whole tile) - the streaming network's tie order is fixed by
  nothing but the reference itself;
* end-to-end ids of ``bsa_fn(..., backend="torch")`` (``bsa.py:9-25`` ->
  ``bsa_select``, ``bsa_torch.py:61-106``) for fp32 and bf16 inputs, head groups
  1/2/3/4/16, comparison tiles 16-128 (including tiles wider than the block),
  decode and suffix offsets, packed documents, force policies, and keys whose
  block means tie exactly (all-zero keys, repeated blocks).

The fixtures are data only; the GPU box never reads ``/root/reference``.
"""

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def structured_keys(gen, batch, length, kh, dim, block):
    noise = torch.randn(batch, length, kh, dim, generator=gen)
    off = 0.5 * torch.randn(batch, (length + block - 1) // block, kh, dim, generator=gen)
    return noise + off.repeat_interleave(block, 1)[:, :length]


def streaming_cases(streaming_topk):
    gen = torch.Generator().manual_seed(11)
    cases = []
    for tile, topk, length in [(16, 8, 16), (16, 4, 37), (32, 8, 100), (32, 16, 64),
                               (64, 8, 200), (64, 32, 130), (128, 16, 300), (128, 64, 128),
                               (4, 2, 9), (8, 4, 23)]:
        rows = 64
        palette = torch.tensor([4.0, 0.0, 0.5, 0.25, 1.0, 3.0], dtype=torch.float32)
        scores = palette[torch.randint(0, palette.numel(), (rows, length), generator=gen)]
        noise = torch.rand(rows, length, generator=gen)
        use = torch.rand(rows, length, generator=gen) < 0.3
        use[: rows // 2] = False
        scores = torch.where(use, noise, scores)
        # ids: a valid prefix per row (as flat routing produces), -1 beyond it
        limit = torch.randint(0, length, (rows, 1), generator=gen)
        ids = torch.arange(length).expand(rows, length)
        ids = torch.where(ids <= limit, ids, torch.full_like(ids, -1))
        scores = torch.where(ids < 0, torch.zeros_like(scores), scores)
        out = streaming_topk(scores, ids, topk, tile)
        cases.append((tile, topk, scores.numpy(), ids.numpy(), out.numpy()))
    return cases


SHAPES = [
    # name, batch, Tq, N, Hq, Hkv, D, C, offset, key recipe
    ("prefill512", 1, 512, 512, 4, 2, 32, 16, None, "structured"),
    ("tail1000", 2, 1000, 1000, 4, 1, 16, 16, None, "structured"),
    ("gqa16", 1, 512, 512, 16, 1, 32, 16, None, "structured"),
    ("mha", 1, 300, 300, 2, 2, 32, 16, None, "structured"),
    ("g2", 1, 333, 333, 4, 2, 16, 16, None, "structured"),
    ("g3", 1, 256, 256, 6, 2, 16, 16, None, "structured"),
    ("decode", 2, 1, 1000, 4, 2, 32, 16, None, "structured"),
    ("suffix", 1, 64, 777, 4, 2, 32, 16, 600, "structured"),
    ("c32", 1, 1024, 1024, 8, 2, 32, 32, None, "structured"),
    ("c64", 1, 2048, 2048, 4, 1, 32, 64, None, "structured"),
    ("zeros", 1, 256, 256, 4, 2, 16, 16, None, "zeros"),
    ("repeat", 1, 512, 512, 4, 1, 16, 16, None, "repeat"),
]
TOPKS = {"c32": (8, 16), "c64": (8, 32)}
POLICIES = ((True, 1), (True, 2), (False, 1), (False, 0), (True, 0))


def stored(x):
    """fp32 tensors as float32 arrays, 16-bit tensors as their bit patterns (exact)."""
    if x.dtype == torch.float32:
        return x.numpy()
    return x.view(torch.int16).numpy()


def make_keys(gen, recipe, batch, n, kh, dim, block):
    if recipe == "zeros":
        return torch.zeros(batch, n, kh, dim)
    k = structured_keys(gen, batch, n, kh, dim, block)
    if recipe == "repeat":
        # every block repeats the keys of the block four before it: equal means
        blocks = (n + block - 1) // block
        for j in range(4, blocks):
            a, b = j * block, min(n, (j + 1) * block)
            k[:, a:b] = k[:, (j - 4) * block:(j - 4) * block + (b - a)]
    return k


def digest(x):
    return hashlib.sha256(stored(x).tobytes()).hexdigest()


def case_inputs(s_index, dtype_name):
    """q [B, Tq, Hq, D] and k [B, N, Hkv, D] of shape ``SHAPES[s_index]`` in the dtype."""
    name, batch, tq, n, qh, kh, dim, block, offset, recipe = SHAPES[s_index]
    dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    gen = torch.Generator().manual_seed(3000 + 10 * s_index + (dtype_name == "bf16"))
    qf = torch.randn(batch, n, qh, dim, generator=gen)
    kf = make_keys(gen, recipe, batch, n, kh, dim, block)
    q = (qf[:, n - tq:] if offset is None else qf[:, offset:offset + tq]).to(dtype)
    return q.contiguous(), kf.to(dtype)


def packed_inputs(dtype_name):
    """q [1, 512, 4, 32], k [1, 512, 2, 32] of the packed case (documents ``PACKED_CU``)."""
    gen = torch.Generator().manual_seed(3999 + (dtype_name == "bf16"))
    dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}[dtype_name]
    q = torch.randn(1, 512, 4, 32, generator=gen).to(dtype)
    k = structured_keys(gen, 1, 512, 2, 32, 16).to(dtype)
    return q, k


PACKED_CU = (0, 100, 357, 512)


def main():
    from pisa.ops.flash_sparse_attn.bsa import bsa_fn
    from pisa.ops.flash_sparse_attn.bsa.bsa_torch import streaming_topk

    arrays = {}
    for index, (tile, topk, scores, ids, out) in enumerate(streaming_cases(streaming_topk)):
        arrays[f"t{index}_scores"] = scores
        arrays[f"t{index}_ids"] = ids.astype(np.int32)
        arrays[f"t{index}_meta"] = np.array([tile, topk])
        arrays[f"t{index}_out"] = out.astype(np.int32)
    arrays["stream_count"] = np.array(index + 1)

    case = 0
    for s_index, (name, batch, tq, n, qh, kh, dim, block, offset, recipe) in enumerate(SHAPES):
        for dtype_name in ("fp32", "bf16"):
            q, k = case_inputs(s_index, dtype_name)
            arrays[f"in{s_index}{dtype_name}_sha"] = np.array([digest(q), digest(k)])
            for topk in TOPKS.get(name, (4, 8)):
                for force_first, force_recent in POLICIES:
                    out = bsa_fn(q, k, block_size=block, topk=topk, query_offset=offset,
                                 force_first=force_first, force_recent=force_recent,
                                 backend="torch")
                    key = f"s{case}"
                    arrays[key + "_meta"] = np.array(
                        [s_index, dtype_name == "bf16", topk, force_first, force_recent, block,
                         -1 if offset is None else offset, 0], dtype=np.int64)
                    arrays[key + "_out"] = out.numpy().astype(np.int16)
                    case += 1
    # packed documents (cu_seqlens): document-local ids
    cu = torch.tensor(PACKED_CU)
    for dtype_name in ("fp32", "bf16"):
        q, k = packed_inputs(dtype_name)
        arrays[f"packed{dtype_name}_sha"] = np.array([digest(q), digest(k)])
        out = bsa_fn(q, k, block_size=16, topk=8, cu_seqlens=cu, force_first=True,
                     force_recent=2, backend="torch")
        arrays[f"packed{dtype_name}_out"] = out.numpy().astype(np.int16)
    arrays["packed_cu"] = cu.numpy()
    arrays["count"] = np.array(case)
    np.savez_compressed(os.path.join(HERE, "bsa.npz"), **arrays)
    print("streaming cases", arrays["stream_count"], "selection cases", case)


if __name__ == "__main__":
    sys.exit(main())
