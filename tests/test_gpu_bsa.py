"""GPU parity of the flat BSA selection (``bsa_fn``) against the reference's golden
vectors and the CPU oracle.

Bar: ids bit-exact including slot order, except rows whose differing slots hold
blocks the oracle scores within 1e-4 of the row's largest score
(``parity.adjudicate_flat``).
"""

import os
import zlib

import numpy as np
import pytest
import torch

import oracle as O
from parity import adjudicate_flat, structured_qkv, to_gpu
from tests.golden.make_golden_bsa import PACKED_CU, SHAPES, case_inputs, packed_inputs

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bsa.npz")


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()   # the HIP library must load: no fallback
    return nlogn_pisa_amd


def _check(q, k, dtype, block, topk, ff, fr, offset, got, want=None, tokens=None):
    """Compare GPU ids with ``want`` (default: the oracle); returns the exempt rows."""
    batch, tq = q.shape[:2]
    pos = O.query_positions(batch, tq, k.shape[1], offset)
    if tokens is not None:
        q, pos, got = q[:, tokens], pos[:, tokens], got[:, tokens]
        want = None if want is None else want[:, tokens]
    if want is None:
        want = O.bsa_select(q, k, block, topk, pos, ff, fr, dtype)
    if np.array_equal(got, want):
        return 0
    scores, ids, _ = O.bsa_scores(q, k, block, pos, ff, fr, dtype)
    differ, exempt, failures = adjudicate_flat(got, want, scores, ids)
    assert not failures, f"{len(failures)} non-exempt rows of {differ} differing, e.g. {failures[:5]}"
    return exempt


def test_bsa_matches_reference_goldens(P):
    g = np.load(GOLDEN)
    inputs, rows, exempt = {}, 0, 0
    for c in range(int(g["count"])):
        s_index, bf16, topk, ff, fr, block, offset, _ = (int(x) for x in g[f"s{c}_meta"])
        dtype = "bf16" if bf16 else "fp32"
        print(f"golden case {c} ({SHAPES[s_index][0]}, {dtype}, K={topk}, ff={ff}, fr={fr})",
              flush=True)
        if (s_index, dtype) not in inputs:
            inputs[(s_index, dtype)] = case_inputs(s_index, dtype)
        q, k = inputs[(s_index, dtype)]
        off = None if offset < 0 else offset
        got = P.bsa_fn(q.cuda(), k.cuda(), block, topk, query_offset=off, force_first=bool(ff),
                       force_recent=fr).cpu().numpy()
        exempt += _check(q.float().numpy(), k.float().numpy(), dtype, block, topk, bool(ff), fr,
                         off, got, want=g[f"s{c}_out"].astype(np.int64))
        rows += got.size // topk
    assert exempt <= 1e-3 * rows


def test_bsa_packed_matches_reference_goldens(P):
    g = np.load(GOLDEN)
    cu = torch.tensor(PACKED_CU, dtype=torch.int32, device="cuda")
    for dtype in ("fp32", "bf16"):
        print(f"packed {dtype}", flush=True)
        q, k = packed_inputs(dtype)
        got = P.bsa_fn(q.cuda(), k.cuda(), 16, 8, cu_seqlens=cu, force_first=True,
                       force_recent=2).cpu().numpy()
        want = g[f"packed{dtype}_out"].astype(np.int64)
        if not np.array_equal(got, want):
            for a, b in zip(PACKED_CU[:-1], PACKED_CU[1:]):
                _check(q[:, a:b].float().numpy(), k[:, a:b].float().numpy(), dtype, 16, 8, True,
                       2, None, got[:, a:b], want=want[:, a:b])


CASES = [
    # name, dtype, batch, n, tq, Hq, Hkv, D, C, K, ff, fr, offset
    ("g8-d128", "bf16", 1, 3000, None, 16, 2, 128, 64, 8, True, 2, None),
    ("g32", "bf16", 1, 1500, None, 32, 1, 64, 32, 16, True, 1, None),
    ("g1-fp16", "fp16", 2, 700, None, 3, 3, 32, 16, 8, False, 1, None),
    ("w128", "bf16", 1, 4000, None, 8, 2, 64, 128, 16, True, 2, None),
    ("k64", "bf16", 1, 9000, None, 4, 1, 64, 64, 64, True, 3, None),
    ("w4", "fp32", 1, 90, None, 4, 2, 16, 4, 2, True, 1, None),
    ("w8", "fp32", 1, 200, None, 2, 1, 32, 8, 4, False, 2, None),
    ("decode", "bf16", 3, 20000, 1, 32, 2, 64, 64, 8, True, 2, None),
    ("suffix", "bf16", 2, 5000, 77, 4, 2, 128, 64, 8, True, 2, 4000),
    # head dims outside 16/32/64/128: zero-padded products
    ("d48", "bf16", 1, 2000, None, 8, 2, 48, 32, 8, True, 2, None),
    ("d96-fp32", "fp32", 1, 1500, None, 4, 1, 96, 64, 8, True, 1, None),
    ("d80-g32", "fp16", 1, 1200, None, 32, 1, 80, 16, 16, True, 2, None),
    ("d256", "bf16", 2, 3000, None, 16, 2, 256, 64, 16, True, 2, None),
    ("d160-fp32-decode", "fp32", 2, 5000, 1, 8, 2, 160, 64, 8, False, 2, None),
    # head dims off the 16 grid: 16-bit multiples of 8, any fp32 head dim
    ("d40", "bf16", 1, 1500, None, 8, 2, 40, 32, 8, True, 2, None),
    ("d24-fp16-g64", "fp16", 1, 900, None, 64, 1, 24, 16, 8, True, 1, None),
    ("d72-suffix", "bf16", 2, 2000, 50, 16, 2, 72, 64, 16, True, 2, 1500),
    ("d17-fp32", "fp32", 1, 700, None, 4, 2, 17, 16, 8, False, 2, None),
    ("d200-fp32-decode", "fp32", 2, 4000, 1, 8, 1, 200, 64, 8, True, 2, None),
    # more than 32 query heads per kv head: head chunks of 32 summed per tile
    ("g64", "bf16", 1, 1500, None, 64, 1, 64, 32, 16, True, 1, None),
    ("g48-fp32", "fp32", 1, 800, None, 96, 2, 32, 16, 8, False, 2, None),
    ("g100-fp16-d80", "fp16", 1, 1000, None, 100, 1, 80, 64, 8, True, 2, None),
    ("g128-decode", "bf16", 2, 6000, 1, 128, 1, 128, 64, 8, True, 2, None),
    ("g128-d256-suffix", "bf16", 1, 3000, 40, 128, 1, 256, 64, 16, True, 2, 2500),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_bsa_matches_oracle(P, case):
    name, dtype, batch, n, tq, qh, kh, dim, block, topk, ff, fr, offset = case
    print(f"bsa {name}", flush=True)
    q, k = structured_qkv(zlib.crc32(name.encode()) % 1000, batch, n, qh, kh, dim, dtype, value=False)
    if tq is not None:
        start = n - tq if offset is None else offset
        q = q[:, start:start + tq].copy()
    got = P.bsa_fn(to_gpu(q, dtype), to_gpu(k, dtype), block, topk, query_offset=offset,
                   force_first=ff, force_recent=fr).cpu().numpy()
    tokens = None
    if q.shape[1] > 600:
        rng = np.random.default_rng(1)
        tokens = np.sort(np.concatenate([np.arange(64), q.shape[1] - 1 - np.arange(64),
                                         rng.choice(q.shape[1], 256, replace=False)]))
        tokens = np.unique(tokens)
    _check(q, k, dtype, block, topk, ff, fr, offset, got, tokens=tokens)


def test_bsa_reference_benchmark_shape_sampled(P):
    """The reference benchmark's shape (bf16, Hq=32, Hkv=2, D=64, C=64, K=8) at 16K
    tokens: 384 sampled tokens against the oracle with the full block means."""
    n = 16384
    gen = torch.Generator().manual_seed(2024)
    q = torch.randn(1, n, 32, 64, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, n, 2, 64, generator=gen).to(torch.bfloat16)
    got = P.bsa_fn(q.cuda(), k.cuda(), 64, 8).cpu().numpy()
    tokens = np.unique(np.concatenate([np.arange(0, n, 64), np.arange(n - 128, n)]))
    _check(q.float().numpy(), k.float().numpy(), "bf16", 64, 8, True, 2, None, got,
           tokens=tokens)


def test_select_blocks_bsa_method_is_bsa_fn(P):
    q, k = structured_qkv(9, 1, 777, 8, 2, 64, "bf16", value=False)
    qg, kg = to_gpu(q, "bf16"), to_gpu(k, "bf16")
    a = P.select_blocks(qg, kg, method="bsa", block_size=32, topk=8, force_recent=1)
    b = P.bsa_fn(qg, kg, 32, 8, force_recent=1)
    assert torch.equal(a, b)


def test_bsa_errors(P):
    q = torch.zeros(1, 64, 4, 32, device="cuda", dtype=torch.bfloat16)
    k = torch.zeros(1, 64, 2, 32, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="topk cannot hold all required blocks"):
        P.bsa_fn(q, k, 8, 2, force_first=True, force_recent=3)
    with pytest.raises(ValueError, match="block_size <= 128"):
        P.bsa_fn(q, k, 256, 8)
    with pytest.raises(P._lib.PisaError, match="at most 128 query heads"):
        P.bsa_fn(torch.zeros(1, 64, 129, 32, device="cuda", dtype=torch.bfloat16),
                 torch.zeros(1, 64, 1, 32, device="cuda", dtype=torch.bfloat16), 16, 4)
    with pytest.raises(P._lib.PisaError, match="multiples of 8 for 16-bit"):
        P.bsa_fn(torch.zeros(1, 64, 4, 36, device="cuda", dtype=torch.bfloat16),
                 torch.zeros(1, 64, 2, 36, device="cuda", dtype=torch.bfloat16), 16, 4)
    with pytest.raises(P._lib.PisaError, match="up to 256"):
        P.bsa_fn(torch.zeros(1, 64, 4, 264, device="cuda", dtype=torch.float32),
                 torch.zeros(1, 64, 2, 264, device="cuda", dtype=torch.float32), 16, 4)
