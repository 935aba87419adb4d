"""Property tests on the GPU path: random supported shapes and settings, each
example checked against the CPU oracle to the same bars as the fixed cases
(selection ids bit-exact with tie adjudication, ``tests/parity.py``; attention
within half an output ulp + 2e-2 for 16-bit and 1e-5 for fp32 of float64).  The
attention backward is drawn for head dims up to 128 (the reference's GPU path,
FLA, stops at 128: sparse_attn_fla.py:42-45).

Examples are derandomized, so every run checks the same set.
"""

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle as O
from parity import excess_error, structured_qkv, to_gpu
from test_gpu_select import _check_against, _run_select

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-5, "bf16": 2e-2, "fp16": 2e-2}


def grad_tol(dtype, ref):
    """Gradient bar: TOL, and for float32 gradients larger than 1, 1e-5 of their
    magnitude.  A float32 dK/dV of size ~7 sums ~10^3 products; that sum alone
    carries ~1e-5 of rounding in any order (any float32 implementation, the
    reference's included), and request order within a tile varies, so an
    absolute 1e-5 there measures the order, not the result."""
    if dtype != "fp32":
        return TOL[dtype]
    return TOL[dtype] * max(1.0, float(np.abs(ref).max()))
SETTINGS = dict(deadline=None, derandomize=True, database=None,
                suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large,
                                       HealthCheck.function_scoped_fixture])


def _offsets(kind, seed, batch, tq, length):
    """query_offset forms (``validation.py:38-56``): None (the queries end at the
    keys' end), a scalar, or one offset per batch element; (numpy form for the
    oracle, the form passed to the GPU operators)."""
    if kind == "none" or tq is None:
        return None, None
    rng = np.random.default_rng(seed + 7)
    if kind == "scalar":
        off = int(rng.integers(0, length - tq + 1))
        return off, off
    off = rng.integers(0, length - tq + 1, size=batch).astype(np.int64)
    return off, torch.from_numpy(off).cuda()


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()   # the HIP library must load: no fallback
    return nlogn_pisa_amd


@st.composite
def selection_cases(draw):
    block = draw(st.sampled_from([16, 32, 64, 128, 256, 512, 1024]))
    # up to 400 blocks (routing three or four levels deep at b = 2), the last one ragged
    blocks = draw(st.one_of(st.integers(1, 40), st.integers(41, 400 if block <= 128 else 60)))
    length = max(1, blocks * block - draw(st.integers(0, block - 1)))
    decode = draw(st.booleans())
    tq = 1 if decode else draw(st.sampled_from([None, max(1, length // 3)]))
    ff = draw(st.booleans())
    fr = draw(st.integers(1, 2))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        batch=draw(st.integers(1, 2)),
        length=length,
        tq=tq,
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 3, 4, 8, 16, 32])),
        # off the 16 grid too: rows zero-padded by select_blocks
        dim=draw(st.sampled_from([16, 24, 32, 40, 48, 64, 72, 96, 128, 256])),
        block=block,
        branching=draw(st.sampled_from([2, 4, 8])),
        topk=draw(st.sampled_from([k for k in (2, 4, 8, 16, 32, 64) if k >= int(ff) + fr])),
        method=draw(st.sampled_from(["pisa", "pisa2", "pisa1"])),
        ff=ff,
        fr=fr,
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        schedule=draw(st.sampled_from(["auto", "grouped", "fused"])),
        needles=draw(st.sampled_from([0.0, 0.05])),
        offset=draw(st.sampled_from(["none", "scalar", "per_batch"])),
    )


def _selection_case(P, c):
    """One drawn selection case against the oracle on up to 96 spread tokens."""
    print(f"select property {c}", flush=True)
    q, k = structured_qkv(c["seed"], c["batch"], c["length"], c["group"] * c["kh"], c["kh"], c["dim"],
                          c["dtype"], offset_block=c["block"], needles=c["needles"], value=False,
                          tq=c["tq"])
    tq = q.shape[1] if c["tq"] is not None else None
    off_np, off_gpu = _offsets(c["offset"], c["seed"], c["batch"], tq, c["length"])
    ids, trace = _run_select(P, q, k, c["dtype"], c["method"], c["block"], c["topk"], c["ff"],
                             c["fr"], off_gpu, c["schedule"], c["branching"])
    assert ids.shape == (c["batch"], q.shape[1], c["kh"], c["topk"])
    tokens = np.unique(np.linspace(0, q.shape[1] - 1, min(q.shape[1], 96)).astype(np.int64))
    _check_against(q, k, c["dtype"], c["method"], c["block"], c["topk"], c["ff"], c["fr"], off_np,
                   c["branching"], ids, trace, tokens=tokens)


@settings(max_examples=60, **SETTINGS)
@given(case=selection_cases())
def test_selection_random_shapes(P, case):
    _selection_case(P, case)


@st.composite
def wide_group_selection_cases(draw):
    """33-128 query heads per kv head (the routing keeps a kv head's query rows in
    LDS, eight head slots per lane); q kept under 2^23 elements."""
    block = draw(st.sampled_from([16, 32, 64, 128, 256]))
    blocks = draw(st.one_of(st.integers(1, 40), st.integers(41, 120)))
    length = max(1, blocks * block - draw(st.integers(0, block - 1)))
    group = draw(st.sampled_from([33, 48, 64, 100, 128]))
    dim = draw(st.sampled_from([16, 48, 64, 128, 256]))
    mode = draw(st.sampled_from(["decode", "suffix", "full"]))
    if mode == "full" and length * group * dim > 1 << 23:
        mode = "suffix"
    tq = {"decode": 1, "suffix": max(1, min(length // 3, (1 << 23) // (group * dim))), "full": None}[mode]
    ff = draw(st.booleans())
    fr = draw(st.integers(1, 2))
    return dict(
        seed=draw(st.integers(0, 10_000)), batch=1, length=length, tq=tq, kh=1, group=group,
        dim=dim, block=block, branching=draw(st.sampled_from([2, 4, 8])),
        topk=draw(st.sampled_from([k for k in (2, 4, 8, 16, 32, 64) if k >= int(ff) + fr])),
        method=draw(st.sampled_from(["pisa", "pisa2", "pisa1"])), ff=ff, fr=fr,
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        schedule=draw(st.sampled_from(["auto", "grouped", "fused"])),
        needles=draw(st.sampled_from([0.0, 0.05])),
        offset=draw(st.sampled_from(["none", "scalar"])),
    )


@settings(max_examples=24, **SETTINGS)
@given(case=wide_group_selection_cases())
def test_selection_wide_groups(P, case):
    _selection_case(P, case)


@st.composite
def attention_cases(draw):
    block = draw(st.sampled_from([16, 32, 48, 64, 96, 128, 256]))
    length = draw(st.integers(min_value=1, max_value=12 * block))
    decode = draw(st.booleans())
    # off the 16 grid too: rows zero-padded by sparse_attention
    dim = draw(st.sampled_from([16, 24, 32, 40, 48, 64, 72, 96, 120, 128, 256]))
    backward = draw(st.booleans()) and dim <= 128
    # value rows of another width (forward only, and the backward's padded rows)
    value_dim = draw(st.sampled_from([dim, dim, 32, 64])) if dim <= 128 else dim
    return dict(
        seed=draw(st.integers(0, 10_000)),
        batch=draw(st.integers(1, 2)),
        length=length,
        tq=1 if decode else draw(st.integers(1, length)),
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 3, 4, 8, 16])),
        dim=dim,
        value_dim=value_dim,
        block=block,
        topk=draw(st.integers(1, 8)),
        causal=draw(st.booleans()),
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        duplicates=draw(st.booleans()),
        backward=backward,
        offset=draw(st.sampled_from(["none", "scalar", "per_batch"])),
    )


def _random_ids(rng, batch, tq, kh, topk, blocks, duplicates):
    """Ids in [-1, blocks + 3): padding, blocks past the keys and, when asked,
    a block repeated within a row (its keys then count twice, as in the
    reference's gather)."""
    ids = rng.integers(-1, blocks + 3, size=(batch, tq, kh, topk)).astype(np.int64)
    if duplicates and topk > 1:
        ids[..., -1] = ids[..., 0]
    return ids


def _attention_case(P, c):
    """One drawn attention case (forward, or forward and backward) against the oracle."""
    print(f"attention property {c}", flush=True)
    dt = c["dtype"]
    q, k, v = structured_qkv(c["seed"], c["batch"], c["length"], c["group"] * c["kh"], c["kh"], c["dim"],
                             dt, offset_block=c["block"])
    q = np.ascontiguousarray(q[:, c["length"] - c["tq"]:])
    if c["value_dim"] != c["dim"]:
        v = O.round_storage(np.random.default_rng(c["seed"] + 2).standard_normal(
            (c["batch"], c["length"], c["kh"], c["value_dim"])).astype(np.float32), dt)
    rng = np.random.default_rng(c["seed"] + 1)
    blocks = -(-c["length"] // c["block"])
    ids = _random_ids(rng, c["batch"], c["tq"], c["kh"], c["topk"], blocks, c["duplicates"])
    off_np, off_gpu = _offsets(c["offset"], c["seed"], c["batch"], c["tq"], c["length"])
    pos = O.query_positions(c["batch"], c["tq"], c["length"], off_np)
    ref_o, ref_lse = O.sparse_attention(q, k, v, ids, c["block"], positions=pos, causal=c["causal"])
    ids_gpu = torch.from_numpy(ids).cuda()
    if not c["backward"]:
        out, lse = P.sparse_attention_with_lse(to_gpu(q, dt), to_gpu(k, dt), to_gpu(v, dt), ids_gpu,
                                               c["block"], causal=c["causal"], query_offset=off_gpu)
        assert excess_error(out.float().cpu().numpy(), ref_o, dt) <= TOL[dt]
        lse = lse.cpu().numpy()
        fin = np.isfinite(ref_lse)
        assert np.array_equal(np.isneginf(lse), ~fin)
        if fin.any():
            assert np.abs(lse[fin] - ref_lse[fin]).max() <= max(TOL[dt], 1e-5)
        return
    dout = O.round_storage(rng.standard_normal(ref_o.shape).astype(np.float32), dt)
    qg, kg, vg = (to_gpu(x, dt).requires_grad_(True) for x in (q, k, v))
    out = P.sparse_attention(qg, kg, vg, ids_gpu, c["block"], causal=c["causal"], query_offset=off_gpu)
    out.backward(to_gpu(dout, dt))
    assert excess_error(out.detach().float().cpu().numpy(), ref_o, dt) <= TOL[dt]
    grads = O.sparse_attention_backward(q, k, v, ids, dout, c["block"], positions=pos,
                                        causal=c["causal"])
    for name, mine, ref in zip(("dq", "dk", "dv"), (qg.grad, kg.grad, vg.grad), grads):
        err = excess_error(mine.float().cpu().numpy(), ref, dt)
        assert err <= grad_tol(dt, ref), f"{name} excess error {err}"


@settings(max_examples=60, **SETTINGS)
@given(case=attention_cases())
def test_attention_random_shapes(P, case):
    _attention_case(P, case)


@st.composite
def wide_group_attention_cases(draw):
    """24-128 query heads per kv head (a tile request carries the whole group),
    at most 48 query rows so the float64 oracle stays quick."""
    c = draw(attention_cases())
    c.update(group=draw(st.sampled_from([24, 32, 48, 64, 100, 128])), kh=1, batch=1,
             tq=min(c["tq"], 48))
    return c


@settings(max_examples=24, **SETTINGS)
@given(case=wide_group_attention_cases())
def test_attention_wide_groups(P, case):
    _attention_case(P, case)


# ---------------------------------------------------------------- packed documents

def _bounds(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64).tolist()


def _doc_offsets(kind, seed, docs):
    """Packed decode offsets (``validation.py:70-79``): none (each document's last
    position), one scalar for every document, or one per document; returns the
    per-document local offsets (None: the default) and the query_offset argument."""
    if kind == "none":
        return [None] * len(docs), None
    rng = np.random.default_rng(seed + 11)
    if kind == "scalar":
        off = int(rng.integers(0, min(e - s for s, e in docs)))
        return [off] * len(docs), off
    offs = [int(rng.integers(0, e - s)) for s, e in docs]
    return offs, torch.tensor(offs, dtype=torch.int64, device="cuda")


@st.composite
def packed_selection_cases(draw):
    block = draw(st.sampled_from([16, 32, 64, 128]))
    docs = draw(st.integers(1, 6))
    lengths = draw(st.lists(st.one_of(st.integers(1, 2 * block), st.integers(2 * block, 30 * block)),
                            min_size=docs, max_size=docs))
    ff = draw(st.booleans())
    fr = draw(st.integers(1, 2))
    topk = draw(st.sampled_from([k for k in (2, 4, 8, 16) if k >= int(ff) + fr]))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        lengths=lengths,
        decode=draw(st.booleans()),        # one query per document
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 4, 8])),
        dim=draw(st.sampled_from([16, 32, 64, 128])),
        block=block,
        branching=draw(st.sampled_from([b for b in (2, 4, 8) if b * topk <= 512])),
        topk=topk,
        method=draw(st.sampled_from(["pisa", "pisa2", "pisa1"])),
        ff=ff,
        fr=fr,
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        schedule=draw(st.sampled_from(["auto", "grouped", "fused"])),
        index_dtype=draw(st.sampled_from([torch.int32, torch.int64])),
        doc_offsets=draw(st.sampled_from(["none", "scalar", "per_document"])),
    )


@settings(max_examples=30, **SETTINGS)
@given(case=packed_selection_cases())
def test_packed_selection_random_documents(P, case):
    """cu_seqlens selection (``top_k_pyramid.py:73-86``): every document's ids equal
    its selection alone (own depth, or the longest document's for fused routing),
    and that selection meets the oracle bar."""
    import parity
    c = case
    print(f"packed select property {c}", flush=True)
    dt, block, b = c["dtype"], c["block"], c["branching"]
    bounds = _bounds(c["lengths"])
    docs = list(zip(bounds[:-1], bounds[1:]))
    q, k = structured_qkv(c["seed"], 1, bounds[-1], c["group"] * c["kh"], c["kh"], c["dim"], dt,
                          offset_block=block, value=False)
    if c["decode"]:
        q = np.ascontiguousarray(q[:, :len(docs)])
    qg, kg = to_gpu(q, dt), to_gpu(k, dt)
    cu = torch.tensor(bounds, dtype=c["index_dtype"], device="cuda")
    kw = dict(force_first=c["ff"], force_recent=c["fr"], branching=b)
    decode = q.shape[1] != k.shape[1]
    local, offset = _doc_offsets(c["doc_offsets"] if decode else "none", c["seed"], docs)
    out = P.select_blocks(qg, kg, c["method"], block, c["topk"], cu_seqlens=cu, query_offset=offset,
                          routing_schedule=c["schedule"], **kw).cpu().numpy()
    grouped = c["schedule"] == "grouped" or (c["schedule"] == "auto" and c["method"] != "pisa1"
                                             and not decode)
    longest = max(-(-(e - s) // block) for s, e in docs)
    geometry = None if grouped else O.routing_geometry(longest, c["topk"], b)
    for d, (s, e) in enumerate(docs):
        rows = slice(d, d + 1) if decode else slice(s, e)
        qd, kd = q[:, rows], k[:, s:e]
        ids, trace = P.selection.select_blocks_traced(
            qg[:, rows], kg[:, s:e], c["method"], block, c["topk"], query_offset=local[d],
            routing_schedule="grouped" if grouped else "fused", geometry=geometry, **kw)
        ids, trace = ids.cpu().numpy(), trace.cpu().numpy()
        assert np.array_equal(out[:, rows], ids), f"document {d} [{s}, {e})"
        tq = qd.shape[1]
        tokens = np.unique(np.linspace(0, tq - 1, min(tq, 48)).astype(np.int64))
        levels = O.build_pyramid(kd, block, b, None, dt)
        pos = O.query_positions(1, tq, e - s, local[d])
        res = parity.selection_parity(qd, kd, ids, trace, tokens, c["method"], block, c["topk"],
                                      c["ff"], c["fr"], b, levels, pos, geometry=geometry)
        assert not res["failures"], f"document {d}: {res['failures'][:3]}"


@st.composite
def packed_attention_cases(draw):
    block = draw(st.sampled_from([16, 32, 64, 128]))
    docs = draw(st.integers(1, 5))
    lengths = draw(st.lists(st.integers(1, 10 * block), min_size=docs, max_size=docs))
    dim = draw(st.sampled_from([16, 32, 64, 128, 256]))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        lengths=lengths,
        decode=draw(st.booleans()),
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 4, 8])),
        dim=dim,
        block=block,
        topk=draw(st.integers(1, 8)),
        causal=draw(st.booleans()),
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        duplicates=draw(st.booleans()),
        backward=draw(st.booleans()) and dim <= 128,
        doc_offsets=draw(st.sampled_from(["none", "scalar", "per_document"])),
    )


@settings(max_examples=30, **SETTINGS)
@given(case=packed_attention_cases())
def test_packed_attention_random_documents(P, case):
    """cu_seqlens attention (``sparse_attn.py:29-54``): document-local ids (padding,
    past the document's blocks, repeated) and positions; O, LSE and the gradients
    equal the per-document oracle, concatenated."""
    c = case
    print(f"packed attention property {c}", flush=True)
    dt, block = c["dtype"], c["block"]
    bounds = _bounds(c["lengths"])
    docs = list(zip(bounds[:-1], bounds[1:]))
    qh = c["group"] * c["kh"]
    q, k, v = structured_qkv(c["seed"], 1, bounds[-1], qh, c["kh"], c["dim"], dt, offset_block=block)
    if c["decode"]:
        q = np.ascontiguousarray(q[:, :len(docs)])
    decode = q.shape[1] != k.shape[1]
    local, offset = _doc_offsets(c["doc_offsets"] if decode else "none", c["seed"], docs)
    rng = np.random.default_rng(c["seed"] + 3)
    parts = []
    for s, e in docs:
        tq = 1 if decode else e - s
        parts.append(_random_ids(rng, 1, tq, c["kh"], c["topk"], -(-(e - s) // block), c["duplicates"]))
    ids = np.concatenate(parts, 1)
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    ref_o, ref_l, ref_g = [], [], [[], [], []]
    dout = O.round_storage(rng.standard_normal(q.shape).astype(np.float32), dt)
    for d, (s, e) in enumerate(docs):
        rows = slice(d, d + 1) if decode else slice(s, e)
        pos = O.query_positions(1, rows.stop - rows.start, e - s, local[d])
        o_, l_ = O.sparse_attention(q[:, rows], k[:, s:e], v[:, s:e], ids[:, rows], block,
                                    positions=pos, causal=c["causal"])
        ref_o.append(o_)
        ref_l.append(l_)
        if c["backward"]:
            g_ = O.sparse_attention_backward(q[:, rows], k[:, s:e], v[:, s:e], ids[:, rows],
                                             dout[:, rows], block, positions=pos, causal=c["causal"])
            for j in range(3):
                ref_g[j].append(g_[j])
    ref_o, ref_l = np.concatenate(ref_o, 1), np.concatenate(ref_l, 1)
    ids_gpu = torch.from_numpy(ids).cuda()
    qg, kg, vg = (to_gpu(x, dt).requires_grad_(c["backward"]) for x in (q, k, v))
    out, lse = P.sparse_attention_with_lse(qg, kg, vg, ids_gpu, block, cu_seqlens=cu,
                                           causal=c["causal"], query_offset=offset)
    assert excess_error(out.detach().float().cpu().numpy(), ref_o, dt) <= TOL[dt]
    lse = lse.cpu().numpy()
    fin = np.isfinite(ref_l)
    assert np.array_equal(np.isneginf(lse), ~fin)
    if fin.any():
        assert np.abs(lse[fin] - ref_l[fin]).max() <= max(TOL[dt], 1e-5)
    if c["backward"]:
        out.backward(to_gpu(dout, dt))
        for name, mine, ref in zip(("dq", "dk", "dv"), (qg.grad, kg.grad, vg.grad), ref_g):
            ref = np.concatenate(ref, 1)
            err = excess_error(mine.float().cpu().numpy(), ref, dt)
            assert err <= grad_tol(dt, ref), f"{name} excess error {err}"


# ---------------------------------------------------------------- decode cache

@st.composite
def cache_cases(draw):
    block = draw(st.sampled_from([16, 32, 64, 128]))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        prefill=draw(st.integers(1, 40 * block)),
        chunks=draw(st.lists(st.one_of(st.just(1), st.integers(1, 3 * block)), min_size=1, max_size=8)),
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 4, 8])),
        dim=draw(st.sampled_from([16, 32, 64, 128])),
        block=block,
        branching=draw(st.sampled_from([2, 4, 8])),
        topk=draw(st.sampled_from([4, 8, 16])),
        method=draw(st.sampled_from(["pisa", "pisa2", "pisa1"])),
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        batch=draw(st.integers(1, 2)),
    )


@settings(max_examples=30, **SETTINGS)
@given(case=cache_cases())
def test_cache_random_appends(P, case):
    """``PyramidCache`` (``attention_cache.py:50-140``) under a random prefill and
    append sequence: every level bit-exact against a rebuild after each append, and
    a decode selection through the cache equal to one that builds its own pyramid,
    which meets the oracle bar."""
    c = case
    print(f"cache property {c}", flush=True)
    dt, block, b = c["dtype"], c["block"], c["branching"]
    total = c["prefill"] + sum(c["chunks"])
    q, k = structured_qkv(c["seed"], c["batch"], total, c["group"] * c["kh"], c["kh"], c["dim"], dt,
                          offset_block=block, value=False, tq=1)
    kg, qg = to_gpu(k, dt), to_gpu(q, dt)
    cache = P.PyramidCache.from_keys(kg[:, :c["prefill"]], block_size=block, branching=b)
    end = c["prefill"]
    for chunk in c["chunks"]:
        cache.append(kg[:, end:end + chunk])
        end += chunk
        assert cache.length == end
        want = O.build_pyramid(k[:, :end], block, b, None, dt)
        assert cache.lengths.tolist() == [x.shape[1] for x in want]
        for level, (mine, ref) in enumerate(zip(cache.levels, want)):
            np.testing.assert_array_equal(mine.float().cpu().numpy(), ref,
                                          err_msg=f"after {end} tokens, level {level}")
    kw = dict(method=c["method"], block_size=block, topk=c["topk"], query_offset=total - 1,
              force_first=True, force_recent=1, branching=b)
    ids = P.select_blocks(qg, cache.keys, pyramid=cache, **kw)
    alone = P.select_blocks(qg, kg, **kw)
    assert torch.equal(ids, alone)
    traced, trace = _run_select(P, q, k, dt, c["method"], block, c["topk"], True, 1, total - 1,
                                "auto", b)
    assert np.array_equal(traced, ids.cpu().numpy())
    _check_against(q, k, dt, c["method"], block, c["topk"], True, 1, total - 1, b, traced, trace)


# ---------------------------------------------------------------- flat BSA selection

@st.composite
def bsa_cases(draw):
    block = draw(st.sampled_from([4, 8, 16, 32, 64, 128]))
    blocks = draw(st.one_of(st.integers(1, 40), st.integers(41, 300)))
    length = max(1, blocks * block - draw(st.integers(0, block - 1)))
    kind = draw(st.sampled_from(["prefill", "decode", "suffix"]))
    ff = draw(st.booleans())
    fr = draw(st.integers(1, 3))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        batch=draw(st.integers(1, 2)),
        length=length,
        kind=kind,
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 3, 4, 8, 16, 32])),
        dim=draw(st.sampled_from([16, 32, 48, 64, 96, 128, 160, 256])),
        block=block,
        topk=draw(st.sampled_from([k for k in (2, 4, 8, 16, 32, 64) if k >= int(ff) + fr])),
        ff=ff,
        fr=fr,
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        per_batch=draw(st.booleans()),
    )


@settings(max_examples=60, **SETTINGS)
@given(case=bsa_cases())
def test_bsa_random_shapes(P, case):
    """``bsa_fn`` (``bsa_torch.py:8-106``) on random supported shapes against the
    oracle: ids bit-exact including slot order, ties within 1e-4 adjudicated."""
    from parity import adjudicate_flat
    c = case
    print(f"bsa property {c}", flush=True)
    dt, n = c["dtype"], c["length"]
    q, k = structured_qkv(c["seed"], c["batch"], n, c["group"] * c["kh"], c["kh"], c["dim"], dt,
                          offset_block=c["block"], value=False)
    offset = off_gpu = None
    if c["kind"] == "decode":
        q = np.ascontiguousarray(q[:, n - 1:])
    elif c["kind"] == "suffix" and n > 2:
        offset = off_gpu = n // 3
        q = np.ascontiguousarray(q[:, offset:offset + max(1, n // 3)])
    if c["per_batch"] and c["kind"] != "prefill":
        offset, off_gpu = _offsets("per_batch", c["seed"], c["batch"], q.shape[1], n)
    got = P.bsa_fn(to_gpu(q, dt), to_gpu(k, dt), c["block"], c["topk"], query_offset=off_gpu,
                   force_first=c["ff"], force_recent=c["fr"]).cpu().numpy()
    assert got.shape == (c["batch"], q.shape[1], c["kh"], c["topk"])
    tokens = np.unique(np.linspace(0, q.shape[1] - 1, min(q.shape[1], 128)).astype(np.int64))
    pos = O.query_positions(c["batch"], q.shape[1], n, offset)[:, tokens]
    qs, got = q[:, tokens], got[:, tokens]
    want = O.bsa_select(qs, k, c["block"], c["topk"], pos, c["ff"], c["fr"], dt)
    if not np.array_equal(got, want):
        scores, ids, _ = O.bsa_scores(qs, k, c["block"], pos, c["ff"], c["fr"], dt)
        differ, exempt, failures = adjudicate_flat(got, want, scores, ids)
        assert not failures, f"{len(failures)} of {differ} differing rows, e.g. {failures[:3]}"


# ---------------------------------------------------------------- pooling

@st.composite
def pooling_cases(draw):
    dtype = draw(st.sampled_from(["fp32", "bf16", "fp16"]))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        batch=draw(st.integers(1, 3)),
        length=draw(st.one_of(st.integers(1, 64), st.integers(64, 3000))),
        kh=draw(st.integers(1, 4)),
        dim=draw(st.sampled_from([8, 16, 24, 64, 96, 128, 256])),
        size=draw(st.sampled_from([2, 3, 4, 16, 64, 100, 128, 512])),
        branching=draw(st.sampled_from([2, 3, 4, 8])),
        dtype=dtype,
        # magnitudes over 10^(+-spread): float64 sums of fp16 keys are exact at any
        # magnitude (multiples of 2^-24 below 2^16); bf16 and fp32 keys spread over
        # twelve decades have no order-independent sum, so they stay within 10^+-1
        spread=draw(st.sampled_from([1.0, 6.0])) if dtype == "fp16" else 1.0,
    )


@settings(max_examples=40, **SETTINGS)
@given(case=pooling_cases())
def test_pooling_random_shapes(P, case):
    """``mean_pool`` and ``build_pyramid`` (``mean_pooling.py:35-52``) bit-exact against
    the oracle on random shapes, pool sizes, branching factors and keys spread over
    many binades (exact sums, one rounding to float32, then the dtype)."""
    c = case
    print(f"pooling property {c}", flush=True)
    rng = np.random.default_rng(c["seed"])
    shape = (c["batch"], c["length"], c["kh"], c["dim"])
    raw = rng.standard_normal(shape) * 10.0 ** rng.uniform(-c["spread"], c["spread"], shape)
    limit = {"fp16": 6.0e4, "bf16": 1e30, "fp32": 1e30}[c["dtype"]]
    keys = O.round_storage(np.clip(raw, -limit, limit).astype(np.float32), c["dtype"])
    kg = to_gpu(keys, c["dtype"])
    got = P.mean_pool(kg, c["size"]).float().cpu().numpy()
    np.testing.assert_array_equal(got, O.mean_pool(keys, c["size"], c["dtype"]))
    levels = P.build_pyramid(kg, c["size"], branching=c["branching"])
    want = O.build_pyramid(keys, c["size"], c["branching"], None, c["dtype"])
    assert len(levels) == len(want)
    for level, (mine, ref) in enumerate(zip(levels, want)):
        np.testing.assert_array_equal(mine.float().cpu().numpy(), ref, err_msg=f"level {level}")


# ---------------------------------------------------------------- leaf scoring and packed BSA

@st.composite
def leaf_cases(draw):
    block = draw(st.sampled_from([16, 32, 64, 128, 256, 512]))
    ff = draw(st.booleans())
    fr = draw(st.integers(1, 2))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        batch=draw(st.integers(1, 2)),
        length=draw(st.one_of(st.integers(1, 2 * block), st.integers(2 * block, 12 * block))),
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 3, 4, 8, 16])),
        dim=draw(st.sampled_from([16, 32, 48, 64, 96, 128, 256])),
        block=block,
        width=draw(st.integers(1, 48)),
        topk=draw(st.sampled_from([k for k in (2, 4, 8, 16) if k >= int(ff) + fr])),
        method=draw(st.sampled_from(["pisa", "pisa2", "pisa1"])),
        ff=ff,
        fr=fr,
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
    )


@settings(max_examples=40, **SETTINGS)
@given(case=leaf_cases())
def test_leaf_scores_random_shapes(P, case):
    """``leaf_scores`` (``leaf_triton.py:144-232``): random candidates (padding, blocks
    past the keys, repeats) on random shapes against the oracle: the same slots
    scored, scores within 2e-5 (float32 sums in another order)."""
    c = case
    print(f"leaf property {c}", flush=True)
    dt, n = c["dtype"], c["length"]
    q, k = structured_qkv(c["seed"], c["batch"], n, c["group"] * c["kh"], c["kh"], c["dim"], dt,
                          offset_block=c["block"], value=False)
    # the oracle scores every candidate on the CPU: bound its work (q . k products)
    budget = 3e9 / (c["batch"] * c["kh"] * c["width"] * c["block"] * c["dim"] * c["group"])
    if n > budget:
        n = max(1, int(budget))
        q, k = np.ascontiguousarray(q[:, :n]), np.ascontiguousarray(k[:, :n])
    rng = np.random.default_rng(c["seed"] + 5)
    blocks = -(-n // c["block"])
    cand = rng.integers(-1, blocks + 2, size=(c["batch"], n, c["kh"], c["width"])).astype(np.int32)
    pos = O.query_positions(c["batch"], n, n)
    out = P.leaf_scores(to_gpu(q, dt), to_gpu(k, dt), torch.from_numpy(cand).cuda(), c["block"],
                        c["method"], torch.from_numpy(pos).cuda(), c["topk"], c["ff"],
                        c["fr"]).cpu().numpy()
    ref = O.leaf_scores(q, k, cand, c["block"], c["method"], pos, c["topk"], c["ff"], c["fr"],
                        leaf_means=O.mean_pool(k, c["block"], dt))
    assert np.array_equal(np.isneginf(out), np.isneginf(ref))
    fin = np.isfinite(ref)
    np.testing.assert_allclose(out[fin], ref[fin], rtol=2e-5, atol=2e-5)


@st.composite
def packed_bsa_cases(draw):
    block = draw(st.sampled_from([4, 8, 16, 32, 64, 128]))
    docs = draw(st.integers(1, 6))
    ff = draw(st.booleans())
    fr = draw(st.integers(1, 3))
    return dict(
        seed=draw(st.integers(0, 10_000)),
        lengths=draw(st.lists(st.one_of(st.integers(1, 2 * block), st.integers(2 * block, 30 * block)),
                              min_size=docs, max_size=docs)),
        decode=draw(st.booleans()),
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 4, 16])),
        dim=draw(st.sampled_from([16, 64, 96, 128])),
        block=block,
        topk=draw(st.sampled_from([k for k in (2, 4, 8, 16) if k >= int(ff) + fr])),
        ff=ff,
        fr=fr,
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
    )


@settings(max_examples=30, **SETTINGS)
@given(case=packed_bsa_cases())
def test_packed_bsa_random_documents(P, case):
    """``bsa_fn`` with ``cu_seqlens`` (``bsa.py:26-52``): each document's ids equal the
    oracle's on that document alone (prefill, or one decode query per document)."""
    from parity import adjudicate_flat
    c = case
    print(f"packed bsa property {c}", flush=True)
    dt, block = c["dtype"], c["block"]
    bounds = _bounds(c["lengths"])
    docs = list(zip(bounds[:-1], bounds[1:]))
    q, k = structured_qkv(c["seed"], 1, bounds[-1], c["group"] * c["kh"], c["kh"], c["dim"], dt,
                          offset_block=block, value=False)
    if c["decode"]:
        q = np.ascontiguousarray(q[:, :len(docs)])
    decode = q.shape[1] != k.shape[1]
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    got = P.bsa_fn(to_gpu(q, dt), to_gpu(k, dt), block, c["topk"], cu_seqlens=cu,
                   force_first=c["ff"], force_recent=c["fr"]).cpu().numpy()
    for d, (s, e) in enumerate(docs):
        rows = slice(d, d + 1) if decode else slice(s, e)
        qd, kd, mine = q[:, rows], k[:, s:e], got[:, rows]
        tokens = np.unique(np.linspace(0, qd.shape[1] - 1, min(qd.shape[1], 64)).astype(np.int64))
        pos = O.query_positions(1, qd.shape[1], e - s)[:, tokens]
        want = O.bsa_select(qd[:, tokens], kd, block, c["topk"], pos, c["ff"], c["fr"], dt)
        if not np.array_equal(mine[:, tokens], want):
            scores, ids, _ = O.bsa_scores(qd[:, tokens], kd, block, pos, c["ff"], c["fr"], dt)
            differ, exempt, failures = adjudicate_flat(mine[:, tokens], want, scores, ids)
            assert not failures, f"document {d}: {len(failures)} of {differ} differing rows"


# ---------------------------------------------------------------- the attention layer

@st.composite
def layer_cases(draw):
    ff = draw(st.booleans())
    fr = draw(st.integers(1, 2))
    packed = draw(st.booleans())
    docs = draw(st.integers(1, 4)) if packed else 1
    return dict(
        seed=draw(st.integers(0, 10_000)),
        batch=1 if packed else draw(st.integers(1, 2)),
        lengths=draw(st.lists(st.integers(1, 400), min_size=docs, max_size=docs)),
        packed=packed,
        hidden=draw(st.sampled_from([32, 64, 96])),
        kh=draw(st.integers(1, 2)),
        group=draw(st.sampled_from([1, 2, 4])),
        dim=draw(st.sampled_from([16, 32, 64])),
        block=draw(st.sampled_from([16, 32, 64])),
        method=draw(st.sampled_from(["pisa", "pisa2", "pisa1", "bsa", "full"])),
        topk=draw(st.sampled_from([k for k in (4, 8) if k >= int(ff) + fr])),
        ff=ff,
        fr=fr,
        branching=draw(st.sampled_from([2, 4])),
        rope_fraction=draw(st.sampled_from([0.0, 0.5, 1.0])),
        rope_theta=draw(st.sampled_from([10000.0, 500000.0])),
        rope_mode=draw(st.sampled_from(["document", "sequence"])),
        bias=draw(st.booleans()),
    )


@settings(max_examples=30, **SETTINGS)
@given(case=layer_cases())
def test_layer_random_configs(P, case):
    """``PyramidSparseAttention`` (``pyramid_sparse_attention.py:71-222``) in float32 on
    random configurations, packed or not: its output equals the float64 composition of
    the oracle's rotary and attention over the ids the layer's own selection picks
    (projections, rotary positions per document or per sequence, block-sparse or
    dense causal attention, output projection), within 1e-4."""
    c = case
    print(f"layer property {c}", flush=True)
    torch.manual_seed(c["seed"])
    qh, kh, dim = c["group"] * c["kh"], c["kh"], c["dim"]
    cfg = P.PisaLayerConfig(hidden_size=c["hidden"], num_attention_heads=qh, num_key_value_heads=kh,
                            head_dim=dim, attention_method=c["method"], block_size=c["block"],
                            topk=c["topk"], force_first=c["ff"], force_recent=c["fr"],
                            branching=c["branching"], rope_fraction=c["rope_fraction"],
                            rope_theta=c["rope_theta"], rope_position_mode=c["rope_mode"],
                            bias=c["bias"])
    layer = P.PyramidSparseAttention(cfg).cuda()
    bounds = _bounds(c["lengths"])
    n = bounds[-1]
    x = torch.randn(c["batch"], n, c["hidden"], device="cuda")
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda") if c["packed"] else None
    with torch.no_grad():
        out, _ = layer(x, cu_seqlens=cu)
        where = P.token_positions(n, x.device, cu if c["rope_mode"] == "document" else None)
        q = layer.rope(layer.q_proj(x).view(c["batch"], n, qh, dim), where)
        k = layer.rope(layer.k_proj(x).view(c["batch"], n, kh, dim), where)
        if c["method"] == "full":
            ids = None
        else:
            routing = {} if c["method"] == "bsa" else dict(
                routing_schedule=cfg.prefill_routing, leaf_tile=cfg.leaf_tile, branching=c["branching"])
            ids = P.select_blocks(q, k, method=c["method"], block_size=c["block"], topk=c["topk"],
                                  cu_seqlens=cu, force_first=c["ff"], force_recent=c["fr"],
                                  **routing).cpu().numpy()
    w = {name: p.detach().double().cpu().numpy() for name, p in layer.named_parameters()}
    xn = x.double().cpu().numpy()
    theta = layer.rope.theta.cpu().numpy()
    pos = where.cpu().numpy()

    def project(name, heads):
        y = xn @ w[f"{name}.weight"].T + (w[f"{name}.bias"] if c["bias"] else 0.0)
        return y.reshape(c["batch"], n, heads, dim)

    qn = O.rotary(project("q_proj", qh), theta, pos)
    kn = O.rotary(project("k_proj", kh), theta, pos)
    vn = project("v_proj", kh)
    parts = []
    for s, e in zip(bounds[:-1], bounds[1:]):
        docs_ids = (np.broadcast_to(np.arange(-(-(e - s) // c["block"])), (c["batch"], e - s, kh,
                                                                      -(-(e - s) // c["block"])))
                    if ids is None else ids[:, s:e])
        o, _ = O.sparse_attention(qn[:, s:e], kn[:, s:e], vn[:, s:e], np.ascontiguousarray(docs_ids),
                                  c["block"])
        parts.append(o)
    mixed = np.concatenate(parts, 1).reshape(c["batch"], n, qh * dim)
    ref = mixed @ w["o_proj.weight"].T + (w["o_proj.bias"] if c["bias"] else 0.0)
    err = np.abs(out.double().cpu().numpy() - ref).max()
    assert err <= 1e-4 * max(1.0, np.abs(ref).max()), f"max-abs error {err}"


# ---------------------------------------------------------------- flat BSA selection

@st.composite
def bsa_cases(draw):
    """Shapes ``bsa_fn`` takes on the GPU (block_size <= 128, topk <= 64): any block
    size, a ragged last block, 1-128 query heads per kv head (above 32 in chunks),
    head dims 16-256 (padded ones included; fp32 also off the 8 grid), decode /
    suffix / full prefill."""
    block = draw(st.sampled_from([1, 3, 4, 8, 16, 24, 32, 48, 64, 100, 128]))
    nblocks = draw(st.integers(1, 120))
    length = max(1, nblocks * block - draw(st.integers(0, block - 1)))
    blocks = -(-length // block)
    ff = draw(st.booleans())
    fr = draw(st.integers(0, 3))
    batch = draw(st.integers(1, 2))
    group = draw(st.sampled_from([1, 2, 3, 4, 8, 16, 24, 32, 48, 64, 100, 128]))
    kh = draw(st.sampled_from([1, 2]))
    dtype = draw(st.sampled_from(["fp32", "bf16", "fp16"]))
    dims = [16, 24, 32, 40, 48, 64, 72, 80, 96, 128, 160, 200, 256]
    dim = draw(st.sampled_from(dims + ([17, 33, 100, 131] if dtype == "fp32" else [])))
    mode = draw(st.sampled_from(["decode", "suffix", "full"]))
    row = batch * group * kh * dim
    if mode == "full" and length * row > 1 << 23:
        mode = "suffix"
    tq = {"decode": 1, "suffix": max(1, min(length // 3, (1 << 23) // row)), "full": None}[mode]
    return dict(
        seed=draw(st.integers(0, 10_000)), batch=batch, length=length, block=block,
        topk=draw(st.sampled_from([k for k in (1, 2, 4, 8, 16, 32, 64) if k >= min(blocks, int(ff) + fr)])),
        ff=ff, fr=fr, group=group, kh=kh, dim=dim, tq=tq, dtype=dtype,
        offset=draw(st.sampled_from(["none", "scalar", "per_batch"])),
    )


@settings(max_examples=60, **SETTINGS)
@given(case=bsa_cases())
def test_bsa_random_shapes(P, case):
    from test_gpu_bsa import _check as check_bsa
    c = case
    print(f"bsa property {c}", flush=True)
    q, k = structured_qkv(c["seed"], c["batch"], c["length"], c["group"] * c["kh"], c["kh"],
                          c["dim"], c["dtype"], offset_block=c["block"], value=False, tq=c["tq"])
    tq = q.shape[1] if c["tq"] is not None else None
    off_np, off_gpu = _offsets(c["offset"], c["seed"], c["batch"], tq, c["length"])
    got = P.bsa_fn(to_gpu(q, c["dtype"]), to_gpu(k, c["dtype"]), c["block"], c["topk"],
                   query_offset=off_gpu, force_first=c["ff"], force_recent=c["fr"]).cpu().numpy()
    assert got.shape == (c["batch"], q.shape[1], c["kh"], c["topk"])
    tokens = np.unique(np.linspace(0, q.shape[1] - 1, min(q.shape[1], 64)).astype(np.int64))
    check_bsa(q, k, c["dtype"], c["block"], c["topk"], c["ff"], c["fr"], off_np, got, tokens=tokens)
