"""Pins the CPU oracle (``oracle/pisa_oracle.py``) before it is trusted.

What pins each oracle function (no function is left "parity unpinned"):

=====================  ==========================================================
function               pinned by
=====================  ==========================================================
network_topk           reference golden vectors (tie order, tests/golden/network_topk.npz);
                       sortedness + textbook top-k on distinct scores
pyramid_select         reference golden vectors at b=2 (180 cases, slot order, per-level
                       traces); flat top-k when top == 0; identity rule; brute force
mean_pool/build_*      brute-force loops (tails, valid counts); bf16 rounding vs torch
routing_geometry       independent closed form over an exhaustive grid
masks                  brute-force per-id loops
scores                 closed forms: LSE, mean+var/2, binary pisa2 == general form at S=2,
                       one valid child -> z
sparse_attention       dense textbook attention (union mask), torch fp64 autograd,
                       finite differences for the gradients, LSE closed form
rotary_frequency       closed form base^(-2i/d) within float32 rounding, zero tail count
rotary                 closed form of a unit vector's turn (sign), invariants: pair norms kept, identity at position 0, turns compose
                       (p1 then p2 == p1 + p2), negated frequencies undo the turn
=====================  ==========================================================
"""

import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
SHAPES = [("prefill256", None), ("tail1000", None), ("gqa16", None), ("decode", None), ("suffix", 600)]
METHODS = ("pisa", "pisa1", "pisa2")


# ----------------------------------------------------------------- golden vectors

def test_network_topk_matches_reference_goldens():
    net = np.load(os.path.join(GOLDEN, "network_topk.npz"))
    for i in range(int(net["count"])):
        out = O.network_topk(net[f"c{i}_scores"], net[f"c{i}_ids"].astype(np.int64),
                             int(net[f"c{i}_topk"]))
        np.testing.assert_array_equal(out, net[f"c{i}_out"], err_msg=f"case {i}")


def _golden_case(sel, c):
    si, isbf, mi, topk, ff, fr, block, off = (int(x) for x in sel[f"s{c}_meta"])
    dt = "bf16" if isbf else "fp32"
    q, k = sel[f"in{si}{dt}_q"], sel[f"in{si}{dt}_k"]
    pos = O.query_positions(q.shape[0], q.shape[1], k.shape[1], None if off < 0 else off)
    return dict(q=q, k=k, dt=dt, method=METHODS[mi], topk=topk, ff=bool(ff), fr=fr,
                block=block, pos=pos)


def test_pyramid_select_matches_reference_goldens():
    sel = np.load(os.path.join(GOLDEN, "select_b2.npz"))
    checked = 0
    for c in range(int(sel["count"])):
        g = _golden_case(sel, c)
        levels = O.build_pyramid(g["k"], g["block"], 2, None, g["dt"])
        out = O.pyramid_select(g["q"], g["k"], g["method"], g["block"], g["topk"], g["pos"],
                               g["ff"], g["fr"], levels)
        np.testing.assert_array_equal(out, sel[f"s{c}_out"], err_msg=f"case {c}")
        checked += out.size
    assert checked > 100_000


def test_pyramid_select_level_traces_match_reference():
    sel = np.load(os.path.join(GOLDEN, "select_b2.npz"))
    traced = 0
    for c in range(int(sel["count"])):
        if f"s{c}_trace" not in sel:
            continue
        g = _golden_case(sel, c)
        tokens = sel[f"s{c}_trace_tokens"]
        levels = O.build_pyramid(g["k"], g["block"], 2, None, g["dt"])
        _, trace = O.pyramid_select(g["q"], g["k"], g["method"], g["block"], g["topk"], g["pos"],
                                    g["ff"], g["fr"], levels, tokens=tokens, trace=True)
        ref = sel[f"s{c}_trace"]                       # [B, tokens, H, levels, K]
        batch = ref.shape[0]
        for j, entry in enumerate(trace):
            mine = entry["selected"].reshape(batch, len(tokens), -1, g["topk"])
            np.testing.assert_array_equal(mine, ref[:, :, :, j], err_msg=f"case {c} level {j}")
        traced += 1
    assert traced >= 30


# ----------------------------------------------------------------- network invariants

def test_network_sorts_descending_and_matches_textbook_topk():
    rng = np.random.default_rng(0)
    for width in (16, 32, 64, 128, 256, 512, 48):
        scores = rng.standard_normal((50, width)).astype(np.float32)
        ids = np.broadcast_to(np.arange(width), scores.shape).copy()
        out = O.network_topk(scores, ids, 8)
        expect = np.argsort(-scores, axis=-1, kind="stable")[:, :8]
        np.testing.assert_array_equal(out, expect)


# ----------------------------------------------------------------- pooling

def _brute_mean_pool(keys, size):
    b, n, h, d = keys.shape
    blocks = (n + size - 1) // size
    out = np.zeros((b, blocks, h, d))
    for j in range(blocks):
        rows = keys[:, j * size:min(n, (j + 1) * size)].astype(np.float64)
        out[:, j] = rows.sum(1) / rows.shape[1]
    return out


@pytest.mark.parametrize("n,size", [(64, 16), (70, 16), (1, 16), (130, 64), (9, 2), (10, 4)])
def test_mean_pool_brute_force(n, size):
    rng = np.random.default_rng(n * 31 + size)
    keys = rng.standard_normal((2, n, 3, 8)).astype(np.float32)
    np.testing.assert_allclose(O.mean_pool(keys, size, "fp32"), _brute_mean_pool(keys, size),
                               rtol=1e-6, atol=1e-7)


def test_mean_pool_rounds_through_float32():
    """A node is the float32 mean cast to the storage dtype (two roundings,
    ``mean_pooling_torch.py:7-14``): on means that are an fp16 midpoint plus 2^-30
    the oracle returns the even neighbour h, as the reference's eager float32
    mean does, not h + ulp (one rounding)."""
    from parity import midpoint_blocks
    keys, h = midpoint_blocks()
    out = O.mean_pool(keys, 128, "fp16")
    np.testing.assert_array_equal(out[0, 0, 0], h)
    eager = torch.from_numpy(keys).half().float().mean(1).half().float().numpy()
    np.testing.assert_array_equal(out[0, 0], eager[0])


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(100_000) * 10 ** rng.uniform(-6, 6, 100_000)).astype(np.float32)
    mine = O.round_storage(x, "bf16")
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(mine, ref)


@pytest.mark.parametrize("branching", [2, 3, 4, 8])
def test_build_pyramid_levels(branching):
    rng = np.random.default_rng(branching)
    keys = rng.standard_normal((1, 1000, 2, 16)).astype(np.float32)
    levels = O.build_pyramid(keys, 16, branching, None, "bf16")
    assert levels[-1].shape[1] == 1
    assert levels[0].shape[1] == 63
    for lower, upper in zip(levels, levels[1:]):
        expect = O.round_storage(_brute_mean_pool(lower, branching), "bf16")
        np.testing.assert_array_equal(upper, expect)
    capped = O.build_pyramid(keys, 16, branching, 1, "bf16")
    assert len(capped) == 2


# ----------------------------------------------------------------- geometry and masks

def _geometry_closed_form(blocks, topk, branching):
    sizes = [blocks]
    while sizes[-1] > topk:
        parent = -(-sizes[-1] // branching)
        if parent < topk or parent == sizes[-1]:
            break
        sizes.append(parent)
    width = max(sizes[-1], topk)
    return len(sizes) - 1, max(16, 2 ** int(np.ceil(np.log2(width))) if width > 1 else 1)


def test_routing_geometry_exhaustive():
    for branching in (2, 4, 8):
        for topk in (8, 16, 32, 64):
            for blocks in range(1, 4097):
                assert O.routing_geometry(blocks, topk, branching) == \
                    _geometry_closed_form(blocks, topk, branching), (blocks, topk, branching)


def test_force_and_routing_masks_brute_force():
    for branching in (2, 4):
        for level in range(3):
            ids = np.arange(-1, 40)[None, :].repeat(64, 0)
            pos = np.arange(0, 64 * 37, 37)
            valid, forced, scoreable = O.routing_masks(ids, pos, 16, 64, True, 2, level, branching)
            for r, p in enumerate(pos):
                leaf = p // 16
                for c, i in enumerate(ids[r]):
                    v = i >= 0 and i * 16 * branching ** level <= p
                    f = v and (i == 0 or any(leaf - t >= 0 and i == (leaf - t) // branching ** level
                                             for t in range(2)))
                    assert valid[r, c] == v and forced[r, c] == f


# ----------------------------------------------------------------- score closed forms

def test_support_scores_closed_forms():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 3, 8)).astype(np.float32)      # B=1, Hq=3 (G=3), D=8
    src = rng.standard_normal((1, 10, 1, 8)).astype(np.float32)
    ids = np.array([[[0, 1, 2, 4]]])
    scale = 8 ** -0.5
    lse = O.block_scores(q, src, ids, 2, "pisa", scale)
    p2 = O.block_scores(q, src, ids, 2, "pisa2", scale)
    p1 = O.block_scores(q, src, ids, 1, "pisa1", 1.0)
    for w, node in enumerate(ids[0, 0]):
        children = src[0, 2 * node:2 * node + 2, 0].astype(np.float64)
        z = q[0].astype(np.float64) @ children.T * scale          # [G, 2]
        expect_lse = np.log(np.exp(z).sum(-1)).sum()
        expect_p2 = (z.mean(-1) + 0.5 * z.var(-1)).sum()
        assert abs(lse[0, 0, w] - expect_lse) < 1e-5 * max(1, abs(expect_lse))
        assert abs(p2[0, 0, w] - expect_p2) < 1e-5 * max(1, abs(expect_p2))
        assert abs(p1[0, 0, w] - (q[0] @ src[0, node, 0]).sum()) < 1e-5
    # the general second-order branch equals the binary form at support two
    gen = O.block_scores(q, src, ids, 2, "pisa2", scale)
    np.testing.assert_allclose(gen, p2, rtol=1e-6)
    # one valid child (node 4 at support 2 over 10 rows has both; node with one: id 4 of 9 rows)
    src9 = src[:, :9]
    one = O.block_scores(q, src9, np.array([[[4]]]), 2, "pisa", scale)
    z = (q[0].astype(np.float64) @ src9[0, 8, 0].astype(np.float64)) * scale
    assert abs(one[0, 0, 0] - z.sum()) < 1e-5
    for method in ("pisa2",):
        one2 = O.block_scores(q, src9, np.array([[[4]]]), 2, method, scale)
        assert abs(one2[0, 0, 0] - z.sum()) < 1e-5


def test_leaf_second_order_closed_form():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 2, 16)).astype(np.float32)
    k = rng.standard_normal((1, 100, 1, 16)).astype(np.float32)
    scale = 16 ** -0.5
    out = O.block_scores(q, k, np.array([[[0, 3, 6]]]), 16, "pisa2", scale)
    for w, node in enumerate((0, 3, 6)):
        rows = k[0, node * 16:min(100, node * 16 + 16), 0].astype(np.float64)
        p = q[0].astype(np.float64) @ rows.T
        expect = (scale * p.mean(-1) + 0.5 * scale * scale * p.var(-1)).sum()
        assert abs(out[0, 0, w] - expect) < 1e-5 * max(1, abs(expect))


# ----------------------------------------------------------------- selection special cases

def _structured(seed, b, t, qh, kh, d, block=16):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, t, qh, d)).astype(np.float32)
    off = 0.5 * rng.standard_normal((b, -(-t // block), kh, d))
    k = (rng.standard_normal((b, t, kh, d)) + np.repeat(off, block, 1)[:, :t]).astype(np.float32)
    return q, k


@pytest.mark.parametrize("method", METHODS)
def test_flat_selection_when_top_is_zero(method):
    """top == 0: the network ranks exhaustive leaf scores of the visible blocks."""
    q, k = _structured(1, 1, 256, 4, 2, 16)
    topk = 8
    levels = O.build_pyramid(k, 16, 4, None, "fp32")
    assert O.routing_geometry(levels[0].shape[1], topk, 4)[0] == 0
    pos = O.query_positions(1, 256, 256)
    out = O.pyramid_select(q, k, method, 16, topk, pos, True, 1, levels, branching=4)
    cand = np.broadcast_to(np.arange(16), (1, 256, 2, 16))
    scores = O.leaf_scores(q, k, cand, 16, method, pos, topk, True, 1,
                           leaf_means=levels[0])
    for t in range(0, 256, 17):
        for h in range(2):
            leaf = t // 16
            visible = [j for j in range(leaf + 1)]
            if len(visible) <= topk and method != "pisa1":
                assert sorted(x for x in out[0, t, h] if x >= 0) == visible
                continue
            forced = {0, leaf}
            rest = sorted((j for j in visible if j not in forced),
                          key=lambda j: -scores[0, t, h, j])
            want = forced | set(rest[:topk - len(forced)])
            assert set(x for x in out[0, t, h] if x >= 0) == want


@pytest.mark.parametrize("branching", [2, 4, 8])
def test_selection_brute_force_small(branching):
    """Each level keeps the top-K children by exact score (brute force per row)."""
    q, k = _structured(2, 1, 512, 8, 2, 16)
    topk = 8
    levels = O.build_pyramid(k, 16, branching, None, "fp32")
    pos = O.query_positions(1, 512, 512)
    tokens = np.arange(300, 512, 13)
    out, trace = O.pyramid_select(q, k, "pisa", 16, topk, pos, True, 2, levels,
                                  branching=branching, tokens=tokens, trace=True)
    for entry in trace:
        ids, scores, selected = entry["ids"], entry["scores"], entry["selected"]
        for r in range(ids.shape[0]):
            for h in range(ids.shape[1]):
                best = np.sort(scores[r, h])[::-1][:topk]
                lookup = dict(zip(ids[r, h].tolist(), scores[r, h].tolist()))
                chosen = [lookup[i] for i in selected[r, h].tolist()]
                # the selected slots carry exactly the K largest scores, in descending order
                np.testing.assert_array_equal(np.array(chosen, np.float32), best)


# ----------------------------------------------------------------- attention

def _attn_case(seed, b=1, t=96, qh=4, kh=2, d=16, block=16, topk=3, distinct=True):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, t, qh, d))
    k = rng.standard_normal((b, t, kh, d))
    v = rng.standard_normal((b, t, kh, d))
    blocks = -(-t // block)
    idx = np.full((b, t, kh, topk), -1, dtype=np.int64)
    for bb in range(b):
        for tt in range(t):
            for h in range(kh):
                pick = rng.permutation(blocks)[:topk] if distinct else rng.integers(0, blocks, topk)
                idx[bb, tt, h] = pick
    idx[0, 0, 0] = -1                                           # an empty row
    return q, k, v, idx


@pytest.mark.parametrize("causal", [True, False])
def test_attention_gather_equals_dense_textbook(causal):
    q, k, v, idx = _attn_case(0)
    o1, l1 = O.sparse_attention(q, k, v, idx, 16, causal=causal)
    o2, l2 = O.sparse_attention_dense(q, k, v, idx, 16, causal=causal)
    np.testing.assert_allclose(o1, o2, atol=1e-12)
    np.testing.assert_allclose(l1, l2, atol=1e-12)
    assert np.isneginf(l1[0, 0, 0]) and (o1[0, 0, 0] == 0).all()


def test_attention_matches_torch_autograd_and_finite_differences():
    q, k, v, idx = _attn_case(1, t=48, block=8, topk=2)
    dout = np.random.default_rng(9).standard_normal(q.shape)
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    pos = torch.arange(48)
    tokens = (torch.tensor(idx)[..., None] * 8 + torch.arange(8)).flatten(-2)
    valid = (tokens >= 0) & (tokens < 48) & (tokens <= pos[None, :, None, None])
    tokens = tokens.clamp(0, 47)
    bi = torch.arange(1)[:, None, None, None]
    hi = torch.arange(2)[None, None, :, None]
    keys, values = kt[bi, tokens, hi], vt[bi, tokens, hi]
    query = qt.reshape(1, 48, 2, 2, 16)
    logits = torch.einsum("bthgd,bthsd->bthgs", query, keys) * 16 ** -0.5
    masked = logits.masked_fill(~valid[..., None, :], -torch.inf)
    masked = torch.where(valid.any(-1)[..., None, None], masked, torch.zeros_like(masked))
    prob = masked.softmax(-1) * valid[..., None, :]
    out = torch.einsum("bthgs,bthsv->bthgv", prob, values).reshape(1, 48, 4, 16)
    out.backward(torch.tensor(dout))
    o, _ = O.sparse_attention(q, k, v, idx, 8)
    np.testing.assert_allclose(o, out.detach().numpy(), atol=1e-12)
    dq, dk, dv = O.sparse_attention_backward(q, k, v, idx, dout, 8)
    np.testing.assert_allclose(dq, qt.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dk, kt.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dv, vt.grad.numpy(), atol=1e-10)
    # finite differences on a few coordinates
    eps = 1e-6
    for arr, grad, coord in ((q, dq, (0, 20, 1, 3)), (k, dk, (0, 9, 1, 5)), (v, dv, (0, 17, 0, 2))):
        plus, minus = arr.copy(), arr.copy()
        plus[coord] += eps
        minus[coord] -= eps
        args_p = [plus if a is arr else a for a in (q, k, v)]
        args_m = [minus if a is arr else a for a in (q, k, v)]
        fp = (O.sparse_attention(*args_p, idx, 8)[0] * dout).sum()
        fm = (O.sparse_attention(*args_m, idx, 8)[0] * dout).sum()
        assert abs((fp - fm) / (2 * eps) - grad[coord]) < 1e-6


def test_attention_lse_closed_form():
    q, k, v, idx = _attn_case(2)
    _, lse = O.sparse_attention(q, k, v, idx, 16)
    t, hq = 77, 3
    h = hq // 2
    keys = sorted({j for i in idx[0, t, h] if i >= 0 for j in range(i * 16, i * 16 + 16) if j <= t})
    z = k[0, keys, h] @ q[0, t, hq] * 16 ** -0.5
    assert abs(lse[0, t, hq] - np.log(np.exp(z).sum())) < 1e-12


# ----------------------------------------------------------------- rotary encoding

@pytest.mark.parametrize("dim,fraction", [(64, 0.5), (128, 1.0), (32, 0.25)])
def test_rotary_frequency_closed_form(dim, fraction):
    theta = O.rotary_frequency(dim, 10000.0, fraction)
    count = int(dim // 2 * fraction)
    exact = 10000.0 ** (-2.0 * np.arange(dim // 2) / dim)
    assert theta.dtype == np.float32 and theta.shape == (dim // 2,)
    np.testing.assert_allclose(theta[:count], exact[:count], rtol=2e-6)
    assert not theta[count:].any()


def test_rotary_invariants():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 40, 3, 64))
    freq = O.rotary_frequency(64, 10000.0, 1.0)
    pos = np.stack([np.arange(40), np.arange(40) + 977])
    y = O.rotary(x, freq, pos)
    half = 32
    norm = lambda a: a[..., :half] ** 2 + a[..., half:] ** 2
    np.testing.assert_allclose(norm(y), norm(x), rtol=1e-12)
    np.testing.assert_allclose(O.rotary(x, freq, np.zeros((1, 40)))[0], x[0], rtol=0, atol=0)
    # turns compose: p1 then p2 equals p1 + p2 (small integer positions: exact float32 angles)
    p1, p2 = np.full((1, 40), 3), np.full((1, 40), 5)
    np.testing.assert_allclose(O.rotary(O.rotary(x, freq, p1), freq, p2), O.rotary(x, freq, p1 + p2),
                               atol=1e-6)
    # negated frequencies undo the turn
    np.testing.assert_allclose(O.rotary(y, -freq, pos), x, atol=1e-9)



def test_rotary_sign_closed_form():
    """Pins the direction of the turn (``rotary_torch.py:5-10``): a unit vector at
    feature f, turned by theta = p * frequency[f], becomes cos(theta) at f and
    +sin(theta) at f + D/2; a unit vector at f + D/2 becomes -sin(theta) at f and
    cos(theta) at f + D/2.  A flipped sign fails both."""
    dim, half = 16, 8
    freq = O.rotary_frequency(dim, 10000.0, 1.0)
    pos = np.array([[0, 1, 7, 300]])
    for f in range(half):
        theta = (pos[0].astype(np.float32) * freq[f]).astype(np.float64)
        lo = np.zeros((1, 4, 1, dim))
        lo[..., f] = 1.0
        y = O.rotary(lo, freq, pos)[0, :, 0]
        np.testing.assert_allclose(y[:, f], np.cos(theta), atol=1e-15)
        np.testing.assert_allclose(y[:, f + half], np.sin(theta), atol=1e-15)
        hi = np.zeros((1, 4, 1, dim))
        hi[..., f + half] = 1.0
        y = O.rotary(hi, freq, pos)[0, :, 0]
        np.testing.assert_allclose(y[:, f], -np.sin(theta), atol=1e-15)
        np.testing.assert_allclose(y[:, f + half], np.cos(theta), atol=1e-15)
        others = [i for i in range(dim) if i not in (f, f + half)]
        assert not y[:, others].any()
