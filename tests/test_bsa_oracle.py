"""The flat BSA routing oracle (``oracle.bsa_select`` and its parts) pinned on the CPU.

streaming_topk   reference golden vectors on tie-heavy rows (tests/golden/bsa.npz) and,
                 for distinct scores, the textbook top-K in descending order
bsa_scores       a per-token brute-force restatement in float64 loops (closed form of
                 the probabilities, the normaliser and the forced-block rule)
bsa_select       reference golden vectors end to end: 240 cases (fp32/bf16, head groups
                 1-16, tiles 16-128, offsets, force policies, exact ties) + packed documents
"""

import math
import os

import numpy as np
import pytest
import torch

import oracle as O
from tests.parity import adjudicate_flat
from tests.golden.make_golden_bsa import (PACKED_CU, SHAPES, case_inputs, digest,
                                          packed_inputs)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bsa.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


def test_streaming_topk_matches_reference_goldens(golden):
    for c in range(int(golden["stream_count"])):
        tile, topk = (int(x) for x in golden[f"t{c}_meta"])
        out = O.streaming_topk(golden[f"t{c}_scores"], golden[f"t{c}_ids"], topk, tile)
        np.testing.assert_array_equal(out, golden[f"t{c}_out"], err_msg=f"case {c}")


@pytest.mark.parametrize("tile,topk,length", [(16, 8, 50), (64, 8, 300), (128, 32, 129), (4, 2, 7)])
def test_streaming_topk_is_sorted_topk_for_distinct_scores(tile, topk, length):
    rng = np.random.default_rng(tile + length)
    rows = 40
    scores = rng.permutation(rows * length).reshape(rows, length).astype(np.float32) + 1
    limit = rng.integers(0, length, (rows, 1))
    ids = np.where(np.arange(length) <= limit, np.arange(length), -1)
    scores = np.where(ids < 0, 0, scores)
    out = O.streaming_topk(scores, ids, topk, tile)
    for r in range(rows):
        valid = np.flatnonzero(ids[r] >= 0)
        order = valid[np.argsort(-scores[r, valid], kind="stable")][:topk]
        expect = np.full(topk, -1)
        expect[:order.size] = order
        np.testing.assert_array_equal(out[r], expect)


def test_streaming_topk_rejects_narrow_tiles():
    with pytest.raises(ValueError, match="tile_size"):
        O.streaming_topk(np.zeros((1, 8)), np.zeros((1, 8), int), 5, 8)


def _brute_scores(q, k, block, position, force_first, force_recent, dtype):
    """One token, one kv head group: the BSA score of every block from the formula."""
    heads_q, dim = q.shape
    n = k.shape[0]
    blocks = -(-n // block)
    means = []
    for j in range(blocks):
        rows = k[j * block:min(n, (j + 1) * block)].astype(np.float64)
        means.append(O.round_storage(np.float32(rows.sum(0) / rows.shape[0]), dtype))
    scale = np.float32(dim ** -0.5)
    query = O.round_storage(q.astype(np.float32) * scale, dtype).astype(np.float64)
    current, complete = position // block, (position + 1) // block
    scores = np.zeros(blocks)
    for h in range(heads_q):
        logits = [float(np.dot(query[h], means[j].astype(np.float64))) for j in range(blocks)]
        if complete > 0:
            peak = max(logits[:complete])
            norm = peak + math.log(sum(math.exp(x - peak) for x in logits[:complete]))
        else:
            norm = 0.0
        for j in range(blocks):
            forced = (force_first and j == 0) or 0 <= current - j < force_recent
            if forced:
                scores[j] += 1.0
            elif j < current:
                scores[j] += math.exp(logits[j] - norm)
    return scores


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("force_first,force_recent", [(True, 2), (False, 0), (False, 1)])
def test_bsa_scores_brute_force(dtype, force_first, force_recent):
    rng = np.random.default_rng(5)
    batch, n, qh, kh, dim, block = 2, 70, 4, 2, 8, 8
    q = O.round_storage(rng.standard_normal((batch, n, qh, dim)), dtype)
    k = O.round_storage(rng.standard_normal((batch, n, kh, dim)) + 0.5, dtype)
    positions = O.query_positions(batch, n, n)
    scores, ids, _ = O.bsa_scores(q, k, block, positions, force_first, force_recent, dtype)
    group = qh // kh
    for b in range(batch):
        for t in range(0, n, 3):
            for h in range(kh):
                expect = _brute_scores(q[b, t, h * group:(h + 1) * group], k[b, :, h], block,
                                       t, force_first, force_recent, dtype)
                np.testing.assert_allclose(scores[b, t, h], expect, rtol=2e-5, atol=1e-7)
                valid = np.arange(expect.size) <= t // block
                np.testing.assert_array_equal(ids[b, t, h], np.where(valid, np.arange(expect.size), -1))


def test_bsa_select_rejects_too_many_required_blocks():
    q = np.zeros((1, 64, 2, 8), np.float32)
    k = np.zeros((1, 64, 1, 8), np.float32)
    with pytest.raises(ValueError, match="required distinct blocks"):
        O.bsa_select(q, k, 4, 2, O.query_positions(1, 64, 64), True, 3)


def _to_numpy(x):
    return x.float().numpy()


def test_bsa_select_matches_reference_goldens(golden):
    """Bit-exact ids (slot order included) except rows whose differing slots hold blocks
    the oracle scores within 1e-4 of the row's largest score."""
    inputs = {}
    total_rows = total_exempt = 0
    for c in range(int(golden["count"])):
        s_index, bf16, topk, first, recent, block, offset, _ = (int(x) for x in golden[f"s{c}_meta"])
        dtype = "bf16" if bf16 else "fp32"
        key = (s_index, dtype)
        if key not in inputs:
            q, k = case_inputs(s_index, dtype)
            assert list(golden[f"in{s_index}{dtype}_sha"]) == [digest(q), digest(k)], \
                "generator drift: regenerated inputs differ from the golden inputs"
            inputs[key] = (_to_numpy(q), _to_numpy(k))
        q, k = inputs[key]
        positions = O.query_positions(q.shape[0], q.shape[1], k.shape[1],
                                      None if offset < 0 else offset)
        out = O.bsa_select(q, k, block, topk, positions, bool(first), recent, dtype)
        scores, ids, _ = O.bsa_scores(q, k, block, positions, bool(first), recent, dtype)
        differ, exempt, failures = adjudicate_flat(out, golden[f"s{c}_out"], scores, ids)
        assert not failures, f"case {c} ({SHAPES[s_index][0]}, {dtype}): rows {failures[:5]}"
        total_rows += out.size // topk
        total_exempt += exempt
    # pooling sums in float32 (reference) or exactly (oracle) move near-tied blocks only
    assert total_exempt <= 1e-3 * total_rows


def test_bsa_select_packed_matches_reference_goldens(golden):
    for dtype in ("fp32", "bf16"):
        q, k = packed_inputs(dtype)
        assert list(golden[f"packed{dtype}_sha"]) == [digest(q), digest(k)]
        q, k = _to_numpy(q), _to_numpy(k)
        pieces = []
        for a, b in zip(PACKED_CU[:-1], PACKED_CU[1:]):
            positions = O.query_positions(1, b - a, b - a)
            pieces.append(O.bsa_select(q[:, a:b], k[:, a:b], 16, 8, positions, True, 2, dtype))
        np.testing.assert_array_equal(np.concatenate(pieces, 1), golden[f"packed{dtype}_out"])
