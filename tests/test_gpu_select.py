"""GPU parity of pooling and block selection against the CPU oracle and the
reference's golden vectors.

Bar: pooled summaries bit-exact; selected ids bit-exact including slot order,
except rows whose first diverging level swaps ids with oracle scores closer
than 1e-4 x the row's largest real score (``tests/parity.py``).
"""

import os
import zlib

import numpy as np
import pytest
import torch

import oracle as O
import parity
from parity import adjudicate, structured_qkv, to_gpu

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
METHODS = ("pisa", "pisa1", "pisa2")


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()   # the HIP library must load: no fallback
    return nlogn_pisa_amd


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("size", [2, 4, 16, 64])
def test_mean_pool_bit_exact(P, dtype, size):
    print(f"mean_pool dtype={dtype} size={size}", flush=True)
    _, k = structured_qkv(1, 2, 1000, 4, 3, 64, dtype, value=False)
    out = P.mean_pool(to_gpu(k, dtype), size).float().cpu().numpy()
    np.testing.assert_array_equal(out, O.mean_pool(k, size, dtype))


def test_mean_pool_rounds_through_float32(P):
    """fp16 means that are a midpoint plus 2^-30 (``parity.midpoint_blocks``): the
    pooled node is the float32 mean rounded to fp16 (half to even), as the oracle's,
    for the pooling kernel and for the cache's append kernel completing the block."""
    from parity import midpoint_blocks
    keys, h = midpoint_blocks(heads=2)
    kg = to_gpu(keys, "fp16")
    out = P.mean_pool(kg, 128).float().cpu().numpy()
    np.testing.assert_array_equal(out, O.mean_pool(keys, 128, "fp16"))
    np.testing.assert_array_equal(out[0, 0, 0], h)
    cache = P.PyramidCache.from_keys(kg[:, :127], block_size=128)
    cache.append(kg[:, 127:])
    np.testing.assert_array_equal(cache.levels[0].float().cpu().numpy(), out)


@pytest.mark.parametrize("branching", [2, 4, 8])
def test_build_pyramid_bit_exact(P, branching):
    print(f"build_pyramid b={branching}", flush=True)
    _, k = structured_qkv(2, 1, 4000, 4, 2, 128, "bf16", value=False)
    levels = P.build_pyramid(to_gpu(k, "bf16"), 64, branching=branching)
    ref = O.build_pyramid(k, 64, branching, None, "bf16")
    assert len(levels) == len(ref)
    for mine, want in zip(levels, ref):
        np.testing.assert_array_equal(mine.float().cpu().numpy(), want)


def _run_select(P, q, k, dtype, method, block, topk, ff, fr, offset, schedule, branching=2):
    qg, kg = to_gpu(q, dtype), to_gpu(k, dtype)
    ids, trace = P.selection.select_blocks_traced(
        qg, kg, method, block, topk, query_offset=offset, force_first=ff, force_recent=fr,
        routing_schedule=schedule, branching=branching)
    return ids.cpu().numpy(), trace.cpu().numpy()


def _check_against(q, k, dtype, method, block, topk, ff, fr, offset, branching, ids, trace,
                   expected=None, tokens=None):
    """Compare GPU ids with ``expected`` (default: the oracle) and adjudicate mismatches."""
    batch, tq = q.shape[:2]
    pos = O.query_positions(batch, tq, k.shape[1], offset)
    levels = O.build_pyramid(k, block, branching, None, dtype)
    if expected is None:
        expected = O.pyramid_select(q, k, method, block, topk, pos, ff, fr, levels,
                                    branching=branching, tokens=tokens)
    if tokens is not None:
        ids, trace = ids[:, tokens], trace[:, tokens]
    if np.array_equal(ids, expected):
        return 0
    toks = np.arange(tq) if tokens is None else np.asarray(tokens)
    _, otrace = O.pyramid_select(q, k, method, block, topk, pos, ff, fr, levels,
                                 branching=branching, tokens=toks, trace=True)
    heads = ids.shape[2]
    rows, mism, exempt, failures = adjudicate(
        ids.reshape(-1, heads, ids.shape[-1]), trace.reshape(-1, heads, *trace.shape[-2:]),
        expected.reshape(-1, heads, ids.shape[-1]), otrace)
    assert not failures, f"{len(failures)} non-exempt mismatches of {rows} rows, e.g. {failures[:5]}"
    return exempt


def _golden_cases():
    sel = np.load(os.path.join(GOLDEN, "select_b2.npz"))
    for c in range(int(sel["count"])):
        si, isbf, mi, topk, ff, fr, block, off = (int(x) for x in sel[f"s{c}_meta"])
        dt = "bf16" if isbf else "fp32"
        yield dict(q=sel[f"in{si}{dt}_q"], k=sel[f"in{si}{dt}_k"], dtype=dt, method=METHODS[mi],
                   topk=topk, ff=bool(ff), fr=fr, block=block, offset=None if off < 0 else off,
                   out=sel[f"s{c}_out"].astype(np.int64), case=c)


@pytest.mark.parametrize("schedule", ["auto", "grouped", "fused"])
def test_select_matches_reference_goldens(P, schedule):
    """The reference's own Torch-path ids (branching 2, depth >= 2), slot order included."""
    exempt = 0
    for g in _golden_cases():
        print(f"golden case {g['case']} {schedule}", flush=True)
        ids, trace = _run_select(P, g["q"], g["k"], g["dtype"], g["method"], g["block"],
                                 g["topk"], g["ff"], g["fr"], g["offset"], schedule)
        exempt += _check_against(g["q"], g["k"], g["dtype"], g["method"], g["block"], g["topk"],
                                 g["ff"], g["fr"], g["offset"], 2, ids, trace, expected=g["out"])
    print("tie-exempt rows:", exempt)


CONFIGS = [
    # name, B, T(N), Hq, Hkv, D, C, b, K, method, ff, fr, dtype, needles, tq
    ("cfg0", 1, 4096, 4, 4, 64, 64, 4, 8, "pisa", True, 1, "fp32", 0.0, None),
    ("cfg0-pisa1", 1, 4096, 4, 4, 64, 64, 4, 8, "pisa1", True, 1, "fp32", 0.0, None),
    ("cfg1-slice", 1, 4096, 16, 4, 128, 64, 4, 16, "pisa", True, 1, "bf16", 0.0, None),
    ("cfg2-slice", 1, 8192, 8, 2, 128, 64, 4, 32, "pisa2", True, 2, "bf16", 0.01, None),
    ("cfg4-slice", 1, 16384, 16, 2, 128, 128, 8, 16, "pisa", True, 1, "bf16", 0.0, None),
    ("refbench", 1, 8192, 32, 2, 64, 64, 2, 8, "pisa", True, 2, "bf16", 0.0, None),
    ("fp16-b2", 2, 2048, 8, 2, 64, 32, 2, 8, "pisa2", False, 1, "fp16", 0.0, None),
    ("suffix", 1, 4096, 8, 2, 64, 64, 4, 8, "pisa", True, 2, "bf16", 0.0, 100),
    ("d32", 1, 2048, 8, 2, 32, 32, 4, 8, "pisa2", True, 1, "bf16", 0.0, None),
    ("d16-fp32", 1, 1024, 4, 2, 16, 16, 2, 8, "pisa", True, 1, "fp32", 0.0, None),
    # 63 blocks, the last one half full: the last span of four sibling blocks has three
    ("ragged-span", 2, 4000, 8, 2, 128, 64, 4, 8, "pisa", True, 1, "bf16", 0.0, None),
    ("ragged-span2", 1, 3000, 4, 2, 64, 64, 2, 8, "pisa2", True, 2, "bf16", 0.02, None),
    # pairs of 128-key blocks, two waves per block: pisa2 moments with a 112-key tail block
    # and an odd block count (the last span has one block); log-sum-exp in fp16 at D = 64,
    # G = 8, with a 56-key tail block whose second half is empty
    # (at least 16384 (token, kv head) items, where pairs are used)
    ("c128-pisa2-ragged", 1, 9072, 8, 2, 128, 128, 4, 8, "pisa2", True, 1, "bf16", 0.0, None),
    ("c128-lse-fp16-d64", 2, 5048, 16, 2, 64, 128, 2, 8, "pisa", True, 2, "fp16", 0.0, None),
    # shapes outside the fast kernels (top_k_pyramid_triton.py:327-335, :362 pads any head
    # dim and head group): blocks of 256 keys (the leaf in 128-key chunks), head dims 96 and
    # 256 and 32 query heads per kv head (query rows in LDS)
    ("c256", 1, 9000, 8, 2, 64, 256, 4, 8, "pisa", True, 1, "bf16", 0.0, None),
    ("c256-pisa2-fp32", 1, 6000, 4, 2, 32, 256, 2, 8, "pisa2", True, 2, "fp32", 0.0, None),
    # blocks of 1024 and 2048 keys (top_k_pyramid_triton.py:329 sets no upper bound)
    ("c1024", 1, 20000, 8, 2, 64, 1024, 2, 8, "pisa", True, 1, "bf16", 0.0, None),
    ("c2048-pisa2-fp16", 1, 30000, 4, 1, 128, 2048, 4, 4, "pisa2", True, 1, "fp16", 0.0, None),
    ("d96", 1, 4096, 8, 2, 96, 64, 4, 8, "pisa2", True, 2, "bf16", 0.01, None),
    ("d96-lse-fp16", 1, 3000, 4, 1, 96, 32, 2, 8, "pisa", True, 1, "fp16", 0.0, None),
    ("d256", 1, 2048, 8, 2, 256, 64, 2, 8, "pisa", True, 1, "bf16", 0.0, None),
    ("g32", 1, 2048, 64, 2, 64, 64, 4, 8, "pisa", True, 1, "bf16", 0.0, None),
    ("g32-pisa2-d128", 1, 2048, 64, 2, 128, 32, 2, 16, "pisa2", True, 2, "bf16", 0.0, None),
    ("g24-pisa1", 1, 1500, 48, 2, 64, 64, 2, 8, "pisa1", True, 1, "bf16", 0.0, None),
    # 128 query heads per kv head (one kv head; the route's query rows in LDS, 128 KB at D 256)
    ("g128", 1, 1200, 128, 1, 64, 64, 2, 8, "pisa", True, 1, "bf16", 0.0, None),
    ("g128-pisa2-d256", 1, 700, 128, 1, 256, 32, 2, 8, "pisa2", True, 2, "bf16", 0.0, None),
    # head dims off the 16 grid: rows zero-padded to the next multiple of 16, the leaf
    # scaled by the true head dim
    ("d40", 1, 3000, 8, 2, 40, 64, 4, 8, "pisa", True, 1, "bf16", 0.0, None),
    ("d72-pisa2-fp16", 1, 2500, 8, 2, 72, 32, 2, 16, "pisa2", True, 2, "fp16", 0.0, None),
    ("d24-fp32-pisa1", 1, 2000, 4, 1, 24, 64, 4, 8, "pisa1", True, 1, "fp32", 0.0, None),
    ("d100-decode", 2, 20000, 16, 2, 100, 64, 4, 16, "pisa", True, 1, "bf16", 0.01, 1),
]


@pytest.mark.parametrize("cfg", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_select_matches_oracle(P, cfg):
    name, batch, length, qh, kh, dim, block, b, topk, method, ff, fr, dtype, needles, tq = cfg
    print(f"select {name}", flush=True)
    q, k = structured_qkv(zlib.crc32(name.encode()) % 1000, batch, length, qh, kh, dim, dtype, needles=needles,
                          value=False, tq=tq)
    offset = None
    tokens = np.unique(np.linspace(0, q.shape[1] - 1, 256).astype(np.int64))
    for schedule in ("auto", "fused") if method != "pisa1" else ("auto",):
        ids, trace = _run_select(P, q, k, dtype, method, block, topk, ff, fr, offset, schedule, b)
        _check_against(q, k, dtype, method, block, topk, ff, fr, offset, b, ids, trace,
                       tokens=tokens)


@pytest.mark.parametrize("method", ["pisa", "pisa2"])
def test_decode_fused_selection(P, method):
    """Tq = 1 against a long cache (the reference's fused decode route)."""
    print(f"decode {method}", flush=True)
    q, k = structured_qkv(7, 4, 32768, 32, 8, 128, "bf16", needles=0.01, value=False, tq=1)
    ids, trace = _run_select(P, q, k, "bf16", method, 64, 32, True, 1, None, "auto", 4)
    _check_against(q, k, "bf16", method, 64, 32, True, 1, None, 4, ids, trace)
    assert (ids[..., :2] >= 0).all()


def test_select_is_deterministic(P):
    q, k = structured_qkv(8, 1, 16384, 16, 4, 128, "bf16", value=False)
    qg, kg = to_gpu(q, "bf16"), to_gpu(k, "bf16")
    a = P.select_blocks(qg, kg, "pisa", 64, 16, force_recent=1, branching=4)
    b = P.select_blocks(qg, kg, "pisa", 64, 16, force_recent=1, branching=4)
    assert torch.equal(a, b)
    assert a.dtype == torch.int64 and tuple(a.shape) == (1, 16384, 4, 16)


LEAF_SHAPES = [
    # B, T, Hq, Hkv, D, C, dtype
    (2, 2048, 8, 2, 64, 64, "bf16"),
    (1, 1024, 64, 2, 32, 32, "bf16"),     # 32 query heads per kv head: a request spans two units
    (1, 1000, 4, 2, 16, 16, "fp32"),
    (1, 700, 6, 2, 128, 128, "fp16"),     # 3 heads per kv head (padded to 4), tail block
    # key blocks larger than the LDS (200-270 KB): MFMA B loads from the key rows
    (1, 1500, 4, 2, 96, 512, "fp32"),
    (1, 1100, 2, 1, 128, 512, "fp32"),
    (1, 600, 8, 2, 256, 256, "fp32"),
]


@pytest.mark.parametrize("shape", LEAF_SHAPES, ids=[f"{s[-1]}-g{s[2] // s[3]}-d{s[4]}" for s in LEAF_SHAPES])
@pytest.mark.parametrize("method", METHODS)
def test_leaf_scores_match_oracle(P, method, shape):
    batch, length, qh, kh, dim, block, dtype = shape
    print(f"leaf_scores {method} {shape}", flush=True)
    q, k = structured_qkv(9, batch, length, qh, kh, dim, dtype, value=False)
    rng = np.random.default_rng(0)
    blocks = -(-length // block)
    cand = rng.integers(-1, blocks + 2, size=(batch, length, kh, 40)).astype(np.int32)
    pos = O.query_positions(batch, length, length)
    qg, kg = to_gpu(q, dtype), to_gpu(k, dtype)
    out = P.leaf_scores(qg, kg, torch.from_numpy(cand).cuda(), block, method,
                        torch.from_numpy(pos).cuda(), 8, True, 1).cpu().numpy()
    ref = O.leaf_scores(q, k, cand, block, method, pos, 8, True, 1,
                        leaf_means=O.mean_pool(k, block, dtype))
    assert np.array_equal(np.isneginf(out), np.isneginf(ref))
    fin = np.isfinite(ref)
    np.testing.assert_allclose(out[fin], ref[fin], rtol=2e-5, atol=2e-5)


def test_packed_documents(P):
    """cu_seqlens: document-local ids, equal to selecting each document alone."""
    q, k = structured_qkv(10, 1, 3000, 8, 2, 64, "bf16", value=False)
    qg, kg = to_gpu(q, "bf16"), to_gpu(k, "bf16")
    cu = torch.tensor([0, 1000, 1700, 3000], dtype=torch.int32, device="cuda")
    out = P.select_blocks(qg, kg, "pisa", 64, 8, cu_seqlens=cu, force_recent=1)
    for s, e in ((0, 1000), (1000, 1700), (1700, 3000)):
        alone = P.select_blocks(qg[:, s:e], kg[:, s:e], "pisa", 64, 8, force_recent=1)
        assert torch.equal(out[:, s:e], alone)


@pytest.mark.parametrize("method", ["pisa", "pisa1"])
def test_packed_fused_geometry_matches_oracle(P, method):
    """Fused packed routing shares the longest document's geometry
    (``top_k_pyramid.py:73-86``): each document's ids, checked against the oracle run
    with that shared geometry on the document alone (its pyramid padded to the shared
    depth, ``top_k_pyramid_torch.py:147``)."""
    print(f"packed fused geometry {method}", flush=True)
    bounds = [0, 3000, 3300, 9000]
    block, topk, b = 64, 8, 4
    q, k = structured_qkv(13, 1, bounds[-1], 8, 2, 64, "bf16", value=False)
    qg, kg = to_gpu(q, "bf16"), to_gpu(k, "bf16")
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    out = P.select_blocks(qg, kg, method, block, topk, cu_seqlens=cu, force_recent=1,
                          routing_schedule="fused", branching=b).cpu().numpy()
    longest = max(-(-(e - s) // block) for s, e in zip(bounds[:-1], bounds[1:]))
    geometry = O.routing_geometry(longest, topk, b)
    for s, e in zip(bounds[:-1], bounds[1:]):
        qd, kd = q[:, s:e], k[:, s:e]
        alone = -(-(e - s) // block)
        ids, trace = P.selection.select_blocks_traced(
            qg[:, s:e], kg[:, s:e], method, block, topk, force_recent=1,
            routing_schedule="fused", branching=b, geometry=geometry)
        assert np.array_equal(out[:, s:e], ids.cpu().numpy())
        levels = O.build_pyramid(kd, block, b, None, "bf16")
        pos = O.query_positions(1, e - s, e - s)
        tokens = np.unique(np.linspace(0, e - s - 1, 200).astype(np.int64))
        res = parity.selection_parity(qd, kd, ids.cpu().numpy(), trace.cpu().numpy(), tokens,
                                      method, block, topk, True, 1, b, levels, pos,
                                      geometry=geometry)
        print(f"document [{s}, {e}) ({alone} blocks, shared top {geometry[0]}): "
              f"{res['rows']} rows, {res['mismatched']} differ, {res['exempt']} tie-exempt")
        assert not res["failures"]


@pytest.mark.parametrize("method,schedule", [("pisa", "auto"), ("pisa2", "grouped"),
                                             ("pisa", "fused"), ("pisa1", "auto")])
def test_packed_many_documents_batched(P, method, schedule):
    """Forty documents of 1 to 1500 tokens: the packed call equals selecting each
    document alone (its own depth, or the longest document's for fused routing), and
    runs one launch series per (geometry, length class), not one per document."""
    from nlogn_pisa_amd import _lib
    print(f"packed many documents {method} {schedule}", flush=True)
    rng = np.random.default_rng(14)
    lengths = rng.integers(1, 1500, size=40).tolist()
    lengths[3], lengths[7] = 1, 64                      # a one-token and a one-block document
    bounds = np.concatenate([[0], np.cumsum(lengths)]).tolist()
    q, k = structured_qkv(15, 1, bounds[-1], 8, 2, 64, "bf16", value=False)
    qg, kg = to_gpu(q, "bf16"), to_gpu(k, "bf16")
    cu = torch.tensor(bounds, dtype=torch.int64, device="cuda")
    kw = dict(method=method, block_size=32, topk=8, force_recent=1, branching=4,
              routing_schedule=schedule)
    _lib.profile_begin()
    out = P.select_blocks(qg, kg, cu_seqlens=cu, **kw)
    launches = {n: c for n, (c, _) in _lib.profile_end().items()}
    print("launches:", launches)
    assert launches.get("route", 0) <= 16 < len(lengths)
    fused = schedule == "fused" or (schedule == "auto" and method == "pisa1")
    longest = max(-(-n // 32) for n in lengths)
    geometry = O.routing_geometry(longest, 8, 4) if fused else None
    for s, e in zip(bounds[:-1], bounds[1:]):
        alone, _ = P.selection.select_blocks_traced(
            qg[:, s:e], kg[:, s:e], method, 32, 8, force_recent=1, branching=4,
            routing_schedule="fused" if fused else "grouped", geometry=geometry)
        assert torch.equal(out[:, s:e], alone), f"document [{s}, {e})"


def test_packed_decode_batched(P):
    """One decode query per document (``validation.py:72-79``): fused routing with the
    longest document's geometry (``top_k_pyramid.py:64-86``), all documents in one
    batch; each document's ids against the oracle with that geometry."""
    from nlogn_pisa_amd import _lib
    bounds = [0, 900, 2000, 4096, 4100, 6000]
    docs = list(zip(bounds[:-1], bounds[1:]))
    q, k = structured_qkv(16, 1, bounds[-1], 8, 2, 64, "bf16", value=False)
    qd = q[:, :len(docs)]
    qg, kg = to_gpu(qd, "bf16"), to_gpu(k, "bf16")
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    _lib.profile_begin()
    out = P.select_blocks(qg, kg, "pisa", 64, 8, cu_seqlens=cu, force_recent=1,
                          branching=2).cpu().numpy()
    launches = {n: c for n, (c, _) in _lib.profile_end().items()}
    assert launches.get("route", 0) <= 4          # length classes of 4, 1024, 2048, 4096 keys
    geometry = O.routing_geometry(max(-(-(e - s) // 64) for s, e in docs), 8, 2)
    for d, (s, e) in enumerate(docs):
        pos = O.query_positions(1, 1, e - s)
        levels = O.build_pyramid(k[:, s:e], 64, 2, None, "bf16")
        want = O.pyramid_select(qd[:, d:d + 1], k[:, s:e], "pisa", 64, 8, pos, True, 1, levels,
                                branching=2, geometry=geometry)
        if not np.array_equal(out[:, d:d + 1], want):
            ids, trace = P.selection.select_blocks_traced(
                qg[:, d:d + 1], kg[:, s:e], "pisa", 64, 8, force_recent=1,
                routing_schedule="fused", branching=2, geometry=geometry)
            assert np.array_equal(out[:, d:d + 1], ids.cpu().numpy())
            res = parity.selection_parity(qd[:, d:d + 1], k[:, s:e], ids.cpu().numpy(),
                                          trace.cpu().numpy(), np.array([0]), "pisa", 64, 8,
                                          True, 1, 2, levels, pos, geometry=geometry)
            assert not res["failures"], f"document {d}"
