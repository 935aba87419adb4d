"""GPU parity at the benchmark configurations' full sizes.

Each test builds a configuration's seeded inputs (``nlogn_pisa_amd.inputs``),
runs the product path at its real shape, and checks it against the CPU oracle:

* selection: every id, slot order included, on >= 1024 stratified (batch, token)
  rows against ``oracle.pyramid_select`` with the full pyramid; a differing row is
  exempt only as ``parity.adjudicate`` allows (oracle score gap < 1e-4 of the
  row's largest at the first diverging level);
* attention: O and LSE on sampled rows against the float64 oracle
  (``sparse_attn_torch.py:6-35`` restated), and for the training configuration
  O, LSE, dQ, dK and dV over the whole tensors against a float32 torch
  restatement of the same equations on the GPU (``parity.torch_sparse_attention``);
  max-abs error <= 2e-2 beyond the final bf16 rounding.

The shapes exercise what the small cases cannot: several 128 MiB query windows
in the leaf scoring and the attention forward (config 1: 2, config 2: 4),
routing depth 2 with both upper levels scored densely (config 2), depth 3 over
131,072 keys with and without a ``PyramidCache`` (config 3), and 128-key blocks
with branching 8 from 4K to 256K tokens (config 4).
"""

import numpy as np
import pytest
import torch

import oracle as O
from parity import (excess_error, needle_recall, selection_parity, stratified_tokens,
                    torch_sparse_attention)

pytestmark = pytest.mark.gpu

TOL = 2e-2          # bf16 outputs and gradients (north star)
SAMPLE = 1024       # selection rows checked per configuration


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()
    return nlogn_pisa_amd


def _numpy(x):
    return x.float().cpu().numpy()


def _select(P, w, q, k, pyramid=None):
    """The product call, then the traced call (same kernels plus the per-level ids)."""
    kw = dict(method=w.method, block_size=w.block_size, topk=w.topk, force_first=w.force_first,
              force_recent=w.force_recent, branching=w.branching)
    ids = P.select_blocks(q, k, backend="auto", pyramid=pyramid, **kw)
    traced, trace = P.selection.select_blocks_traced(q, k, pyramid=pyramid, **kw)
    assert torch.equal(ids, traced), "the traced selection differs from select_blocks"
    return ids, trace


def _check_selection(w, qn, kn, ids, trace, tokens, label):
    positions = O.query_positions(qn.shape[0], qn.shape[1], kn.shape[1])
    levels = O.build_pyramid(kn, w.block_size, w.branching, None, "bf16")
    res = selection_parity(qn, kn, ids, trace, tokens, w.method, w.block_size, w.topk,
                           w.force_first, w.force_recent, w.branching, levels, positions)
    print(f"{label}: {res['rows']} rows, {res['mismatched']} differ, {res['exempt']} tie-exempt",
          flush=True)
    assert not res["failures"], \
        f"{len(res['failures'])} non-exempt mismatches, e.g. {res['failures'][:5]}"
    return res, positions


def _check_rows(label, out, lse, ref_o, ref_lse):
    err = excess_error(out, ref_o, "bf16")
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(lse), ~fin)
    lse_err = float(np.abs(lse[fin] - ref_lse[fin]).max()) if fin.any() else 0.0
    raw = float(np.abs(out - ref_o).max())
    print(f"{label}: O max-abs {raw:.3e} (beyond bf16 rounding {err:.3e}), LSE {lse_err:.3e}",
          flush=True)
    assert err <= TOL and lse_err <= TOL


# ---------------------------------------------------------------- config 2

@pytest.fixture(scope="module")
def cfg2(P):
    from nlogn_pisa_amd.inputs import config, make_inputs
    w = config(2)
    print(f"generating {w.name}", flush=True)
    needles = []
    q, k, v = make_inputs(w, "cuda", needles=needles)
    ids, trace = _select(P, w, q, k)
    print("config 2 selected", flush=True)
    return w, q, k, v, ids, trace, needles


def test_cfg2_selection(P, cfg2):
    """64K tokens, 32 query / 8 kv heads, pisa2, b = 4: routing depth 2 with both
    upper levels dense, four leaf-scoring windows; plus the needle recall."""
    w, q, k, v, ids, trace, needles = cfg2
    assert tuple(ids.shape) == (1, 65536, 8, 32)
    qn, kn = _numpy(q), _numpy(k)
    tokens = stratified_tokens(w.tokens, SAMPLE, seed=2)
    ids_n = ids.cpu().numpy()
    res, positions = _check_selection(w, qn, kn, ids_n, trace.cpu().numpy(), tokens, "config 2")
    hits, total = needle_recall(qn, kn, ids_n[:, tokens], tokens, needles, w.block_size, w.topk,
                                w.force_first, w.force_recent, positions)
    recall = hits / max(total, 1)
    print(f"config 2 needle recall: {hits} / {total} = {recall:.4f}", flush=True)
    assert total > 1000 and recall >= 0.9


def test_cfg2_attention_forward(P, cfg2):
    """O and LSE of the 64K prefill (four attention windows) on 512 sampled rows."""
    w, q, k, v, ids, trace, needles = cfg2
    out, lse = P.sparse_attention_with_lse(q, k, v, ids, block_size=w.block_size)
    rows = stratified_tokens(w.tokens, 512, seed=3)
    pos = O.query_positions(1, w.tokens, w.keys)
    ref_o, ref_lse = O.sparse_attention(_numpy(q[:, rows]), _numpy(k), _numpy(v),
                                        ids[:, rows].cpu().numpy(), w.block_size,
                                        positions=pos[:, rows], chunk=8)
    _check_rows("config 2 attention", _numpy(out[:, rows]), lse[:, rows].cpu().numpy(),
                ref_o, ref_lse)


# ---------------------------------------------------------------- config 1

@pytest.fixture(scope="module")
def cfg1(P):
    from nlogn_pisa_amd.inputs import config, make_inputs
    w = config(1)
    print(f"generating {w.name}", flush=True)
    q, k, v, dout = make_inputs(w, "cuda")
    ids, trace = _select(P, w, q, k)
    print("config 1 selected", flush=True)
    return w, q, k, v, dout, ids, trace


def test_cfg1_selection(P, cfg1):
    """4 x 16K tokens, 16 / 4 heads, pisa, b = 4, depth 2: two leaf windows, the
    first covering two sequences."""
    w, q, k, v, dout, ids, trace = cfg1
    tokens = stratified_tokens(w.tokens, SAMPLE // w.batch, seed=1)
    _check_selection(w, _numpy(q), _numpy(k), ids.cpu().numpy(), trace.cpu().numpy(), tokens,
                     "config 1")


def test_cfg1_attention_forward_backward(P, cfg1):
    """Forward and backward of the training step on the selected ids: every element
    of O, LSE, dQ, dK and dV against the float32 restatement, and O, LSE and dQ of
    sampled rows against the float64 oracle."""
    w, q, k, v, dout, ids, trace = cfg1
    leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v)]
    out, lse = P.sparse_attention_with_lse(*leaves, ids, block_size=w.block_size)
    out.backward(dout)
    positions = torch.arange(w.tokens, device=q.device).expand(w.batch, w.tokens)
    ref = torch_sparse_attention(q, k, v, ids, w.block_size, positions, dout=dout, chunk=128)
    lse_ref = ref[1]
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isneginf(lse), ~fin)
    lse_err = float((lse[fin] - lse_ref[fin]).abs().max())
    print(f"config 1 LSE max-abs {lse_err:.3e}", flush=True)
    assert lse_err <= TOL
    for name, mine, want in (("O", out.detach(), ref[0]), ("dQ", leaves[0].grad, ref[2]),
                             ("dK", leaves[1].grad, ref[3]), ("dV", leaves[2].grad, ref[4])):
        diff = (mine.float() - want).abs()
        raw = float(diff.max())
        # beyond half an ulp of the bf16 value (the output's own final rounding)
        ulp = torch.exp2(torch.floor(torch.log2(want.abs().clamp_min(2.0 ** -14))) - 7) / 2
        err = float((diff - ulp).max())
        print(f"config 1 {name}: max-abs {raw:.3e} (beyond bf16 rounding {err:.3e}) over "
              f"{mine.numel()} elements", flush=True)
        assert err <= TOL, f"{name} error {err}"
    del ref
    rows = stratified_tokens(w.tokens, 64, seed=4)
    pos = O.query_positions(w.batch, w.tokens, w.keys)
    ids_n = ids[:, rows].cpu().numpy()
    qn, kn, vn = _numpy(q[:, rows]), _numpy(k), _numpy(v)
    ref_o, ref_lse = O.sparse_attention(qn, kn, vn, ids_n, w.block_size, positions=pos[:, rows],
                                        chunk=8)
    _check_rows("config 1 attention rows", _numpy(out.detach()[:, rows]), lse[:, rows].cpu().numpy(),
                ref_o, ref_lse)
    # dQ of a row depends on that row alone: the oracle's closed form on the sampled rows
    dq_ref, _, _ = O.sparse_attention_backward(qn, kn, vn, ids_n, _numpy(dout[:, rows]),
                                               w.block_size, positions=pos[:, rows], chunk=8)
    err = excess_error(_numpy(leaves[0].grad[:, rows]), dq_ref, "bf16")
    print(f"config 1 dQ rows vs float64 oracle: {err:.3e}", flush=True)
    assert err <= TOL


# ---------------------------------------------------------------- config 3

@pytest.fixture(scope="module")
def cfg3(P):
    from nlogn_pisa_amd.inputs import config, make_inputs
    w = config(3)
    print(f"generating {w.name}", flush=True)
    q, k, v = make_inputs(w, "cuda")
    print("config 3 generated", flush=True)
    return w, q, k, v


def _decode_oracle(w, q, k, v, ids, b):
    """Oracle ids and attention of sequence ``b`` (its own pyramid, position N - 1)."""
    qn, kn, vn = _numpy(q[b:b + 1]), _numpy(k[b:b + 1]), _numpy(v[b:b + 1])
    levels = O.build_pyramid(kn, w.block_size, w.branching, None, "bf16")
    pos = O.query_positions(1, 1, w.keys)
    want = O.pyramid_select(qn, kn, w.method, w.block_size, w.topk, pos, w.force_first,
                            w.force_recent, levels, branching=w.branching)
    ref_o, ref_lse = O.sparse_attention(qn, kn, vn, ids[b:b + 1], w.block_size, positions=pos)
    return qn, kn, levels, pos, want, ref_o, ref_lse


def test_cfg3_decode(P, cfg3):
    """32 sequences x 131,072 keys, one query each, routing depth 3, fused selection:
    ids with a fresh pyramid and from a PyramidCache, and the decode attention."""
    w, q, k, v = cfg3
    ids, trace = _select(P, w, q, k)
    cache = P.PyramidCache.from_keys(k, w.block_size, w.branching)
    cached, ctrace = _select(P, w, q, k, pyramid=cache)
    assert torch.equal(ids, cached), "selection over a PyramidCache differs"
    out, lse = P.sparse_attention_with_lse(q, k, v, ids, block_size=w.block_size)
    ids_n, trace_n = ids.cpu().numpy(), trace.cpu().numpy()
    out_n, lse_n = _numpy(out), lse.cpu().numpy()
    exempt = 0
    for b in range(w.batch):
        qn, kn, levels, pos, want, ref_o, ref_lse = _decode_oracle(w, q, k, v, ids_n, b)
        if not np.array_equal(ids_n[b:b + 1], want):
            res = selection_parity(qn, kn, ids_n[b:b + 1], trace_n[b:b + 1], np.array([0]),
                                   w.method, w.block_size, w.topk, w.force_first, w.force_recent,
                                   w.branching, levels, pos)
            assert not res["failures"], f"sequence {b}: {res['failures']}"
            exempt += res["exempt"]
        assert (ids_n[b, 0, :, :2] >= 0).all()
        _check_rows(f"config 3 sequence {b}", out_n[b:b + 1], lse_n[b:b + 1], ref_o, ref_lse)
    print(f"config 3: {w.batch * w.key_heads} rows, {exempt} tie-exempt", flush=True)


# ---------------------------------------------------------------- config 4

@pytest.mark.parametrize("tokens", [4096, 16384, 65536, 262144])
def test_cfg4_sweep(P, tokens):
    """Block 128, branching 8, 16 / 2 heads: selection on 1024 stratified rows and
    the attention forward on 256 sampled rows at each length of the sweep."""
    from nlogn_pisa_amd.inputs import config, make_inputs
    w = config(4, tokens)
    print(f"generating {w.name}", flush=True)
    q, k, v = make_inputs(w, "cuda")
    ids, trace = _select(P, w, q, k)
    qn, kn = _numpy(q), _numpy(k)
    sample = stratified_tokens(w.tokens, min(SAMPLE, w.tokens), seed=5)
    _check_selection(w, qn, kn, ids.cpu().numpy(), trace.cpu().numpy(), sample,
                     f"config 4 T={tokens}")
    del trace
    out, lse = P.sparse_attention_with_lse(q, k, v, ids, block_size=w.block_size)
    rows = stratified_tokens(w.tokens, 256, seed=6)
    pos = O.query_positions(1, w.tokens, w.keys)
    ref_o, ref_lse = O.sparse_attention(qn[:, rows], kn, _numpy(v), ids[:, rows].cpu().numpy(),
                                        w.block_size, positions=pos[:, rows], chunk=8)
    _check_rows(f"config 4 T={tokens} attention", _numpy(out[:, rows]), lse[:, rows].cpu().numpy(),
                ref_o, ref_lse)


# ---------------------------------------------------------------- config 0

def test_cfg0_full(P):
    """Config 0 in full (fp32, all 4096 tokens): ids against the oracle, O and LSE,
    and dQ/dK/dV against the float64 closed form, at the fp32 bar of 1e-5."""
    from nlogn_pisa_amd.inputs import config, make_inputs
    w = config(0)
    q, k, v = make_inputs(w, "cuda")
    ids, trace = _select(P, w, q, k)
    qn, kn, vn = _numpy(q), _numpy(k), _numpy(v)
    positions = O.query_positions(1, w.tokens, w.keys)
    levels = O.build_pyramid(kn, w.block_size, w.branching, None, "fp32")
    res = selection_parity(qn, kn, ids.cpu().numpy(), trace.cpu().numpy(), np.arange(w.tokens),
                           w.method, w.block_size, w.topk, w.force_first, w.force_recent,
                           w.branching, levels, positions)
    print(f"config 0: {res['rows']} rows, {res['mismatched']} differ, {res['exempt']} tie-exempt")
    assert not res["failures"]
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(0)).cuda()
    leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v)]
    out, lse = P.sparse_attention_with_lse(*leaves, ids, block_size=w.block_size)
    out.backward(dout)
    ids_n = ids.cpu().numpy()
    ref_o, ref_lse = O.sparse_attention(qn, kn, vn, ids_n, w.block_size, positions=positions)
    grads = O.sparse_attention_backward(qn, kn, vn, ids_n, dout.cpu().numpy(), w.block_size,
                                        positions=positions)
    for name, mine, want in (("O", out.detach(), ref_o), ("dQ", leaves[0].grad, grads[0]),
                             ("dK", leaves[1].grad, grads[1]), ("dV", leaves[2].grad, grads[2])):
        err = float(np.abs(mine.cpu().numpy() - want).max())
        print(f"config 0 {name} max-abs {err:.3e}")
        assert err <= 1e-5, f"{name} error {err}"
    assert float(np.abs(lse.cpu().numpy() - ref_lse).max()) <= 1e-5
