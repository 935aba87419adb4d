"""GPU parity of the decode-time ``PyramidCache`` (``attention_cache.py:50-140``).

Bar: after every append, every cached level is bit-exact against the oracle's
full pyramid of the keys appended so far (so the incremental update equals a
rebuild), and ``select_blocks(pyramid=cache)`` returns exactly the ids of
``select_blocks`` building its own pyramid.
"""

import numpy as np
import pytest
import torch

import oracle as O
from parity import structured_qkv, to_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()   # the HIP library must load: no fallback
    return nlogn_pisa_amd


# prefill, single decode tokens, chunks that straddle leaves, and growth of the
# leaf capacity (and with it of the level count) several times over
CHUNKS = [1, 63, 1, 64, 130, 1, 1, 200, 239, 5, 400, 3]


@pytest.mark.parametrize("dtype,branching,block", [("bf16", 2, 64), ("fp32", 2, 16),
                                                   ("fp16", 4, 32), ("bf16", 8, 16)])
def test_append_equals_full_rebuild(P, dtype, branching, block):
    print(f"pyramid cache dtype={dtype} b={branching} C={block}", flush=True)
    _, k = structured_qkv(11, 2, sum(CHUNKS), 4, 2, 64, dtype, value=False)
    cache = P.PyramidCache(block_size=block, branching=branching)
    kg = to_gpu(k, dtype)
    end = 0
    for chunk in CHUNKS:
        cache.append(kg[:, end:end + chunk])
        end += chunk
        assert cache.length == end
        np.testing.assert_array_equal(cache.keys.float().cpu().numpy(), k[:, :end])
        want = O.build_pyramid(k[:, :end], block, branching, None, dtype)
        levels = cache.levels
        assert [x.shape[1] for x in levels] == [x.shape[1] for x in want]
        assert cache.lengths.tolist() == [x.shape[1] for x in want]
        assert cache.offsets.tolist() == list(cache.starts)
        for level, (mine, ref) in enumerate(zip(levels, want)):
            np.testing.assert_array_equal(mine.float().cpu().numpy(), ref,
                                          err_msg=f"after {end} tokens, level {level}")


def test_append_many_leaves_at_once(P):
    """A long prefill appended to a short cache takes the per-level pooling path."""
    print("pyramid cache long append", flush=True)
    _, k = structured_qkv(12, 1, 5000, 4, 4, 128, "bf16", value=False)
    kg = to_gpu(k, "bf16")
    cache = P.PyramidCache.from_keys(kg[:, :70], block_size=64)
    cache.append(kg[:, 70:])
    for mine, ref in zip(cache.levels, O.build_pyramid(k, 64, 2, None, "bf16")):
        np.testing.assert_array_equal(mine.float().cpu().numpy(), ref)


@pytest.mark.parametrize("method", ["pisa", "pisa2", "pisa1"])
def test_decode_selection_with_cache(P, method):
    print(f"decode selection with cache method={method}", flush=True)
    prefill, steps = 1500, 70
    q, k = structured_qkv(13, 2, prefill + steps, 8, 2, 64, "bf16", needles=0.1, value=False,
                          tq=steps)
    qg, kg = to_gpu(q, "bf16"), to_gpu(k, "bf16")
    cache = P.PyramidCache.from_keys(kg[:, :prefill], block_size=64)
    for step in range(steps):
        n = prefill + step + 1
        cache.append(kg[:, n - 1:n])
        query = qg[:, step:step + 1]
        ids = P.select_blocks(query, cache.keys, method=method, block_size=64, topk=8,
                              query_offset=n - 1, pyramid=cache)
        want = P.select_blocks(query, kg[:, :n], method=method, block_size=64, topk=8,
                               query_offset=n - 1)
        assert torch.equal(ids, want), f"decode step {step} ({n} keys)"


def test_decode_selection_with_cache_off_grid_head_dim(P):
    """Head dim 40: the cache's pyramid rows are zero-padded with q and k, and the
    cached selection equals selection over the concatenated keys."""
    print("decode selection with cache, head dim 40", flush=True)
    prefill, steps = 700, 12
    q, k = structured_qkv(17, 1, prefill + steps, 8, 2, 40, "bf16", needles=0.1, value=False,
                          tq=steps)
    qg, kg = to_gpu(q, "bf16"), to_gpu(k, "bf16")
    cache = P.PyramidCache.from_keys(kg[:, :prefill], block_size=64)
    for step in range(steps):
        n = prefill + step + 1
        cache.append(kg[:, n - 1:n])
        query = qg[:, step:step + 1]
        ids = P.select_blocks(query, cache.keys, block_size=64, topk=8, query_offset=n - 1,
                              pyramid=cache)
        want = P.select_blocks(query, kg[:, :n], block_size=64, topk=8, query_offset=n - 1)
        assert torch.equal(ids, want), f"decode step {step} ({n} keys)"
