"""Selection and attention captured in a HIP graph (``torch.cuda.graph``).

The library enqueues only kernels on the caller's stream (no host synchronisation,
no allocation of its own, no memset nodes: scratch is cleared by fill kernels), so a
decode step and a prefill step can be captured once and replayed.  Each test
replays its graph several times on new inputs copied into the captured tensors,
with the same step run eagerly and the device synchronised between replays, and
requires every replay to equal the eager result bit for bit.
"""

import numpy as np
import pytest
import torch

from parity import structured_qkv, to_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()   # the HIP library must load: no fallback
    return nlogn_pisa_amd


def _capture(step):
    """Warm ``step`` up on a side stream (lazy set-up stays out of the graph), then
    capture it; returns the graph and its output tensors."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outputs = step()
    torch.cuda.synchronize()
    return graph, outputs


def _replay_and_compare(graph, outputs, step, feed, rounds):
    for r in range(rounds):
        print(f"graph replay {r}", flush=True)
        feed(r)
        want = [t.clone() for t in step()]         # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outputs, want)):
            assert torch.equal(got, ref), f"replay {r}, output {i}"


def test_decode_step_in_a_graph(P):
    """One decode step: selection through a ``PyramidCache`` (fused route) and the
    direct decode attention, replayed with new query rows."""
    batch, n, qh, kh, dim, block = 2, 5000, 8, 2, 128, 64
    print("graph decode step", flush=True)
    _, k, v = structured_qkv(61, batch, n, qh, kh, dim, "bf16")
    kg, vg = to_gpu(k, "bf16"), to_gpu(v, "bf16")
    cache = P.PyramidCache.from_keys(kg, block_size=block, branching=4)
    rng = np.random.default_rng(62)
    q = torch.zeros(batch, 1, qh, dim, dtype=torch.bfloat16, device="cuda")

    def feed(r):
        q.copy_(torch.from_numpy(rng.standard_normal((batch, 1, qh, dim)).astype(np.float32)))

    def step():
        ids = P.select_blocks(q, cache.keys, method="pisa", block_size=block, topk=16,
                              query_offset=n - 1, pyramid=cache, branching=4, force_recent=1)
        out = P.sparse_attention(q, cache.keys, vg, ids, block, query_offset=n - 1)
        return ids, out

    feed(-1)
    graph, outputs = _capture(step)
    _replay_and_compare(graph, outputs, step, feed, 4)


@pytest.mark.parametrize("method", ["pisa2", "pisa"])
def test_prefill_step_in_a_graph(P, method):
    """A prefill step: grouped selection (dense levels, bucketed leaf scoring) and the
    bucketed attention forward with its combine, replayed with new q and k."""
    batch, n, qh, kh, dim, block = 1, 6000, 16, 4, 128, 64
    print(f"graph prefill step {method}", flush=True)
    rng = np.random.default_rng(63)
    q = torch.zeros(batch, n, qh, dim, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(batch, n, kh, dim, dtype=torch.bfloat16, device="cuda")
    _, _, v = structured_qkv(64, batch, n, qh, kh, dim, "bf16")
    vg = to_gpu(v, "bf16")

    def feed(r):
        qn, kn = structured_qkv(65 + r, batch, n, qh, kh, dim, "bf16", value=False)
        q.copy_(torch.from_numpy(qn))
        k.copy_(torch.from_numpy(kn))

    def step():
        ids = P.select_blocks(q, k, method=method, block_size=block, topk=16, branching=4,
                              force_recent=2)
        out, lse = P.sparse_attention_with_lse(q, k, vg, ids, block)
        return ids, out, lse

    feed(-1)
    graph, outputs = _capture(step)
    _replay_and_compare(graph, outputs, step, feed, 3)
