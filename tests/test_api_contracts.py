"""Host-side contracts of the operator API (no GPU needed): the reference's
ValueError messages (``top_k_pyramid.py:47-59``, ``validation.py``,
``sparse_attn.py:28-34``, ``mean_pooling.py:22-25``), auto-schedule and
geometry helpers, and deterministic synthetic inputs."""

import pytest
import torch

import nlogn_pisa_amd as P
import oracle as O
from nlogn_pisa_amd.inputs import config, make_inputs


def qk(tq=128, n=128, qh=4, kh=2, d=64, dtype=torch.float32):
    return torch.zeros(1, tq, qh, d, dtype=dtype), torch.zeros(1, n, kh, d, dtype=dtype)


@pytest.mark.parametrize("kwargs,message", [
    (dict(method="nope"), "method must be bsa, pisa1, pisa2 or pisa"),
    (dict(backend="cuda"), "backend must be torch, triton or auto"),
    (dict(leaf_tile=3), "leaf_tile must be 1, 2 or 4"),
    (dict(routing_schedule="x"), "routing_schedule must be auto, grouped or fused"),
    (dict(topk=0), "positive block_size/topk and nonnegative force_recent required"),
    (dict(force_recent=0), "causal pyramid routing requires force_recent >= 1"),
])
def test_select_blocks_reference_errors(kwargs, message):
    q, k = qk()
    with pytest.raises(ValueError, match=message):
        P.select_blocks(q, k, **kwargs)


def test_validate_qkv_reference_errors():
    q, k = qk()
    with pytest.raises(ValueError, match=r"q and k must have shape \[batch, tokens, heads, head_dim\]"):
        P.validate_qkv(q[0], k)
    with pytest.raises(ValueError, match="q and k must share batch size and head dimension"):
        P.validate_qkv(q, k[..., :32])
    with pytest.raises(ValueError, match="whole number of query heads per KV head"):
        P.validate_qkv(torch.zeros(1, 8, 3, 64), k)
    with pytest.raises(ValueError, match="q and k must share a floating dtype and device"):
        P.validate_qkv(q, k.double())
    with pytest.raises(ValueError, match="v must share k's batch, length, heads, dtype and device"):
        P.validate_qkv(q, k, k[:, :5])


def test_query_positions_contract():
    q, k = qk(tq=4, n=10)
    assert P.query_positions(q, k).tolist() == [[6, 7, 8, 9]]
    assert P.query_positions(q, k, 2).tolist() == [[2, 3, 4, 5]]
    with pytest.raises(ValueError, match="queries must refer to positions within their key sequence"):
        P.query_positions(q, k, 7)
    with pytest.raises(ValueError, match="one offset per batch element"):
        P.query_positions(q, k, torch.tensor([1, 2]))
    assert (P.query_positions(q, k).numpy() == O.query_positions(1, 4, 10)).all()


def test_packed_query_contracts():
    q, k = qk(tq=10, n=10)
    cu = torch.tensor([0, 4, 10])
    assert P.packed_queries(q, k, cu) == [(0, 4, 0, 4, 0), (4, 10, 4, 10, 0)]
    qd = torch.zeros(1, 2, 4, 64)
    assert P.packed_queries(qd, k, cu) == [(0, 1, 0, 4, 3), (1, 2, 4, 10, 5)]
    with pytest.raises(ValueError, match="cu_seqlens must start at zero and end at the key length"):
        P.sequence_slices(torch.tensor([0, 4]), 10)
    with pytest.raises(ValueError, match="packed sequences must be nonempty and strictly ordered"):
        P.sequence_slices(torch.tensor([0, 4, 4, 10]), 10)
    with pytest.raises(ValueError, match="packed inputs require batch size one"):
        P.packed_queries(torch.zeros(2, 10, 4, 64), torch.zeros(2, 10, 2, 64), cu)


def test_sparse_attention_reference_errors():
    q, k = qk()
    v = torch.zeros_like(k)
    idx = torch.zeros(1, 128, 2, 4, dtype=torch.long)
    with pytest.raises(ValueError, match=r"indices must have shape \[B,Tq,Hkv,K\]"):
        P.sparse_attention(q, k, v, idx[:, :5])
    with pytest.raises(ValueError, match="indices must be integers on the query device"):
        P.sparse_attention(q, k, v, idx.float())
    with pytest.raises(ValueError, match="invalid block_size or attention backend"):
        P.sparse_attention(q, k, v, idx, backend="xla")


def test_cpu_tensors_are_rejected_not_computed():
    """The product has no CPU path: a CPU tensor is an error, never a fallback."""
    q, k = qk()
    with pytest.raises(ValueError, match="runs on a ROCm GPU"):
        P.select_blocks(q, k, force_recent=1)
    with pytest.raises(ValueError, match="runs on a ROCm GPU"):
        P.sparse_attention(q, k, torch.zeros_like(k), torch.zeros(1, 128, 2, 4, dtype=torch.long))
    with pytest.raises(ValueError, match="runs on a ROCm GPU"):
        P.mean_pool(k, 64)
    with pytest.raises(ValueError, match="pool size must be positive"):
        P.mean_pool(k, 0)


def test_routing_geometry_mirror():
    for b in (2, 4, 8):
        for blocks in range(1, 3000, 7):
            assert P.routing_geometry(blocks, 16, b) == O.routing_geometry(blocks, 16, b)


def test_synthetic_inputs_are_deterministic():
    w = config(0)
    a = make_inputs(w, "cpu")
    b = make_inputs(w, "cpu")
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    q, k, v = a
    assert q.shape == (1, 4096, 4, 64) and k.shape == (1, 4096, 4, 64) and q.dtype == torch.float32
    # keys carry the per-64-token offsets: block means differ much more than noise alone
    means = k.reshape(1, 64, 64, 4, 64).mean(2)
    assert means.std() > 0.35
    assert config(2).needles == 0.01 and config(3).per_sequence_seed


def test_tensor_cache_growth_and_errors():
    """``attention_cache.py:8-48``: power-of-two capacity, copy on growth, fixed shape."""
    cache = P.TensorCache()
    with pytest.raises(ValueError, match="the token cache is empty"):
        cache.tensor
    chunks = [torch.randn(2, n, 3, 4) for n in (1, 2, 5, 1, 9)]
    capacities = []
    for chunk in chunks:
        cache.append(chunk)
        capacities.append(cache.buffer.shape[1])
    assert capacities == [1, 4, 8, 16, 32]
    assert torch.equal(cache.tensor, torch.cat(chunks, 1))
    with pytest.raises(ValueError, match=r"nonempty \[B,T,H,D\] floating tensor"):
        cache.append(torch.zeros(2, 0, 3, 4))
    with pytest.raises(ValueError, match=r"nonempty \[B,T,H,D\] floating tensor"):
        cache.append(torch.zeros(2, 1, 3, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="cannot change"):
        cache.append(torch.zeros(2, 1, 3, 5))


def test_pyramid_cache_layout():
    """Level capacities: next power of two of the leaves, divided by b (rounded up) to 1."""
    cache = P.PyramidCache(block_size=64, branching=2)
    cache.reserve(torch.zeros(1, 1, 2, 8), 5)
    assert cache.capacities == (8, 4, 2, 1) and cache.starts == (0, 8, 12, 14)
    assert cache.storage.shape == (1, 15, 2, 8)
    cache.reserve(torch.zeros(1, 1, 2, 8), 8)       # fits: no re-layout
    assert cache.capacities == (8, 4, 2, 1)
    wide = P.PyramidCache(block_size=16, branching=4)
    wide.reserve(torch.zeros(1, 1, 2, 8), 17)
    assert wide.capacities == (32, 8, 2, 1) and wide.starts == (0, 32, 40, 42)
    with pytest.raises(ValueError, match="branching must be at least 2"):
        P.PyramidCache(branching=1)
    with pytest.raises(ValueError, match="runs on a ROCm GPU"):
        P.PyramidCache().append(torch.zeros(1, 4, 2, 8))


def test_layer_config_methods_and_routing_default():
    """``pisa_config.py:63-79``: every attention method of the reference is accepted
    (bsa included), pisa1 defaults to fused prefill routing and the others to grouped;
    the layer itself declines the NSA baseline."""
    for method in ("full", "bsa", "pisa1", "pisa2", "pisa"):
        cfg = P.PisaLayerConfig(attention_method=method)
        assert cfg.prefill_routing == ("fused" if method == "pisa1" else "grouped")
    with pytest.raises(ValueError, match="Unknown attention method"):
        P.PisaLayerConfig(attention_method="dense")
    with pytest.raises(ValueError, match="prefill_routing must be grouped or fused"):
        P.PisaLayerConfig(prefill_routing="flat")
    with pytest.raises(ValueError, match="not provided"):
        P.PyramidSparseAttention(P.PisaLayerConfig(attention_method="nsa"))


def test_token_positions_brute_force():
    """Positions restart at each packed document (``pyramid_sparse_attention.py:6-11``):
    token t of document [a, e) sits at t - a + offset, checked token by token."""
    cu = torch.tensor([0, 3, 3, 10, 17])
    got = P.token_positions(17, "cpu", cu, offset=4)
    bounds = cu.tolist()
    for t in range(17):
        start = max(a for a in bounds[:-1] if a <= t)
        assert int(got[0, t]) == t - start + 4
    assert P.token_positions(5, "cpu", None, 7).tolist() == [[7, 8, 9, 10, 11]]


@pytest.mark.parametrize("dim,base,fraction", [(64, 10000.0, 0.5), (128, 500000.0, 1.0),
                                               (32, 10000.0, 0.25)])
def test_rotary_table_closed_form(dim, base, fraction):
    """The layer's float32 frequency table (``lrpe.py:20-28``, evaluated with torch's
    float32 CPU power as the reference does) is base^(-2i/D) to within one float32 ulp
    of the float64 closed form and of the oracle's table, zero past the fraction."""
    import numpy as np
    import oracle as O
    theta = P.RotaryEmbedding(dim, base, fraction).theta
    assert theta.dtype == torch.float32 and tuple(theta.shape) == (1, dim // 2)
    got = theta.numpy()[0].astype(np.float64)
    count = int(dim // 2 * fraction)
    exact = base ** (-2.0 * np.arange(dim // 2) / dim)
    ulp = np.spacing(np.float32(np.maximum(exact, 1e-30))).astype(np.float64)
    assert (np.abs(got[:count] - exact[:count]) <= ulp[:count]).all()
    assert not got[count:].any()
    oracle = O.rotary_frequency(dim, base, fraction).astype(np.float64)
    assert (np.abs(got - oracle) <= ulp).all()


def test_benchmark_result_files(tmp_path):
    """The selection sweep writes the reference benchmark's files: selection.json with
    metadata and rows, selection.csv with head_dim, length and a "<label> (ms)" column
    per provider (``benchmark.py:13-19`` labels)."""
    import csv
    import json
    from nlogn_pisa_amd import benchmark as B
    res = B.Results(tmp_path, {"seed": 2024}, ["fused", "q4", "bsa"])
    res.add(64, 4096, {"fused": 1.25, "q4": 0.5, "bsa": "ERROR"}, {"bsa": "failed"})
    res.add(128, 8192, {"fused": 2.0, "q4": 1.0, "bsa": 3.0}, {})
    rows = list(csv.reader(open(tmp_path / "selection.csv")))
    assert rows[0] == ["head_dim", "length", "Direct-LSE fused (ms)", "Direct-LSE Q4 (ms)",
                       "BSA Top-K (ms)"]
    assert rows[1] == ["64", "4096", "1.25", "0.5", "ERROR"]
    data = json.load(open(tmp_path / "selection.json"))
    assert data["metadata"] == {"seed": 2024} and len(data["rows"]) == 2
    assert data["rows"][0]["errors"] == {"bsa": "failed"}


@pytest.mark.parametrize("bounds,decode", [([0, 700, 1500, 1536, 2300], False),
                                           ([0, 64, 65, 200, 4096], False),
                                           ([0, 900, 2000, 4096], True)])
def test_packed_key_layout(bounds, decode):
    """One-launch packed attention: every document's local block j is a whole block
    of the launch whose keys are exactly the document's keys [ks + jC, min(ke, ks + (j+1)C)),
    a query's position lies in its own document's blocks at its local offset, and ids
    outside the document's blocks select nothing (``sparse_attn.py:29-54``)."""
    import numpy as np
    from nlogn_pisa_amd.attention import PackedKeys
    C, n = 64, bounds[-1]
    docs = list(zip(bounds[:-1], bounds[1:]))
    tq = len(docs) if decode else n
    q = torch.zeros(1, tq, 2, 8)
    k = torch.zeros(1, n, 1, 8)
    segments = P.packed_queries(q, k, torch.tensor(bounds), None)
    layout = PackedKeys(segments, tq, C, "cpu")
    start, rows = layout.key_start.numpy(), layout.key_rows.numpy()
    positions = layout.positions.numpy()[0]
    nb = [-(-(e - s) // C) for s, e in docs]
    assert layout.blocks == sum(nb)
    local = torch.arange(-2, max(nb) + 2).repeat(tq, 1)[None, :, None, :]   # [1, Tq, 1, ids]
    mapped = layout.block_ids(local).numpy()[0, :, 0]
    for t in range(tq):
        d = t if decode else next(i for i, (s, e) in enumerate(docs) if s <= t < e)
        s, e = docs[d]
        base = sum(nb[:d])
        p = (e - s - 1) if decode else t - s
        assert positions[t] == base * C + p
        for j, g in zip(local[0, t, 0].tolist(), mapped[t].tolist()):
            if 0 <= j < nb[d]:
                assert g == base + j
                assert start[g] == s + j * C and rows[g] == min(C, e - s - j * C)
                assert g * C <= positions[t] or j * C > p      # causal test in block coordinates
            else:
                assert g == -1


def test_bench_refuses_more_than_one_gpu():
    """``bench.py --gpus N`` with N above 1 exits with status 2 and says why (one GPU
    per box; no multi-GPU path), before touching torch or the GPU."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "exactly one GPU" in res.stderr and res.stdout == ""
