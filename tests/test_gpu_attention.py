"""GPU parity of sparse attention (forward O and LSE, backward dQ/dK/dV) against
the float64 oracle on the same (upcast) inputs.

Bar (north star): max-abs error <= 1e-5 for fp32 inputs, <= 2e-2 for bf16 and
fp16, measured beyond the unavoidable final rounding of a 16-bit output (half an
ulp of the reference value, ``parity.excess_error``).
"""

import zlib

import numpy as np
import pytest
import torch

import oracle as O
from parity import excess_error, structured_qkv, to_gpu

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-5, "bf16": 2e-2, "fp16": 2e-2}


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()
    return nlogn_pisa_amd


def _indices(seed, batch, tq, kh, topk, n, block, offset=None, distinct=True, empty_rows=True):
    """Random distinct visible-or-not block ids, -1 padding, a few empty rows."""
    rng = np.random.default_rng(seed)
    blocks = -(-n // block)
    pos = O.query_positions(batch, tq, n, offset)
    idx = np.full((batch, tq, kh, topk), -1, dtype=np.int64)
    for b in range(batch):
        for t in range(tq):
            current = pos[b, t] // block
            for h in range(kh):
                pool = rng.permutation(blocks)
                pick = [current] + [x for x in pool if x != current][: topk - 1]
                idx[b, t, h, : len(pick)] = pick[:topk]
                if rng.random() < 0.1:
                    idx[b, t, h, rng.integers(0, topk)] = -1
    if empty_rows:
        idx[0, 0, 0] = -1
        idx[-1, tq // 2, kh - 1] = blocks + 5          # out of range only
    return idx


CASES = [
    # name, B, Tq, N, Hq, Hkv, D, C, K, dtype, causal, offset
    ("fp32-small", 1, 256, 256, 4, 2, 64, 16, 4, "fp32", True, None),
    ("fp32-gqa1", 2, 300, 300, 2, 2, 64, 64, 3, "fp32", True, None),
    ("bf16-cfg1ish", 2, 1024, 1024, 16, 4, 128, 64, 8, "bf16", True, None),
    ("bf16-g8", 1, 512, 512, 16, 2, 128, 128, 4, "bf16", True, None),
    ("fp16-d64", 1, 512, 512, 8, 2, 64, 32, 6, "fp16", True, None),
    ("bf16-noncausal", 1, 256, 256, 8, 2, 64, 64, 3, "bf16", False, None),
    ("bf16-decode", 3, 1, 4096, 32, 8, 128, 64, 16, "bf16", True, None),
    ("bf16-suffix", 1, 40, 900, 8, 2, 64, 64, 5, "bf16", True, 777),
    ("bf16-g16", 1, 256, 256, 16, 1, 64, 64, 4, "bf16", True, None),
    ("bf16-d32", 1, 256, 256, 8, 2, 32, 32, 4, "bf16", True, None),
    ("fp32-d16", 1, 128, 256, 4, 1, 16, 16, 6, "fp32", True, None),
    ("fp16-d16-c48", 2, 200, 200, 4, 2, 16, 48, 3, "fp16", True, None),
    ("bf16-c128", 1, 512, 640, 8, 2, 128, 128, 3, "bf16", True, None),
    # 2 x 10000 tokens x 32 heads x 128 x 2 bytes = 160 MB of q rows: three forward windows of
    # 8192 flattened (batch, token) rows under the 128 MiB budget, the second across batches
    ("bf16-windows", 2, 10000, 10000, 32, 2, 128, 64, 6, "bf16", True, None),
    # 3 x 8 x 1024 = 24576 (batch, kv head, block) groups: bucketing with global atomics
    ("bf16-wide", 3, 40, 65536, 8, 8, 16, 64, 4, "bf16", True, None),
    # register-tile backward: fp16 at head dim 128, 128-key blocks at head dim 64, G = 3
    ("fp16-d128", 1, 384, 384, 8, 2, 128, 64, 4, "fp16", True, None),
    ("bf16-d64-c128", 1, 512, 640, 8, 2, 64, 128, 3, "bf16", True, None),
    ("bf16-g3", 2, 200, 260, 6, 2, 64, 64, 3, "bf16", True, None),
    # the combine's two-pass limit of 256 (slot, head) pairs: 16 x 16 at it, 16 x 17 past it
    # (the online merge), G = 3 above takes the online merge too
    ("bf16-g16-k16", 1, 300, 1024, 16, 1, 64, 32, 16, "bf16", True, None),
    ("bf16-g16-k17", 1, 300, 1024, 16, 1, 64, 32, 17, "bf16", True, None),
    # blocks over 128 keys run as their 128-key halves; head dim 96 (forward on the general
    # kernels, backward on zero-padded 128-wide rows); 32 query heads per kv head
    ("bf16-c256", 1, 700, 1500, 8, 2, 64, 256, 4, "bf16", True, None),
    ("bf16-c1024", 1, 500, 3000, 8, 2, 64, 1024, 3, "bf16", True, None),
    ("fp32-c512-d32", 1, 300, 2100, 4, 2, 32, 512, 3, "fp32", True, None),
    ("bf16-d96", 1, 400, 400, 8, 2, 96, 64, 4, "bf16", True, None),
    ("bf16-g32", 1, 256, 512, 64, 2, 64, 64, 4, "bf16", True, None),
    ("bf16-g128", 1, 200, 400, 128, 1, 64, 64, 4, "bf16", True, None),
    # fp32 rows of 128 with 128-key blocks: the forward's tiles exceed the LDS, so the
    # blocks are attended as 64-key halves (pisa_attention_block_limit)
    ("fp32-d128-c128", 1, 300, 300, 4, 2, 128, 128, 3, "fp32", True, None),
    # head dims off the 16 grid: zero-padded to the next multiple of 16 for the forward
    # (and to 32/64/128 for the backward), the padding's columns dropped
    ("bf16-d40", 1, 300, 300, 8, 2, 40, 64, 4, "bf16", True, None),
    ("fp32-d17-decode", 2, 1, 2000, 8, 2, 17, 64, 6, "fp32", True, None),
    ("fp16-d72-suffix", 1, 50, 800, 8, 2, 72, 32, 5, "fp16", True, 600),
    ("bf16-d120-g16", 1, 256, 512, 16, 1, 120, 64, 4, "bf16", True, None),
]


def _inputs(case):
    name, batch, tq, n, qh, kh, dim, block, topk, dtype, causal, offset = case
    q, k, v = structured_qkv(zlib.crc32(name.encode()) % 97 + 3, batch, n, qh, kh, dim, dtype)
    if offset is None:
        q = q[:, n - tq:]
    else:
        q = q[:, offset:offset + tq]
    idx = _indices(len(name), batch, tq, kh, topk, n, block, offset)
    return q, k, v, idx


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_matches_oracle(P, case):
    name, batch, tq, n, qh, kh, dim, block, topk, dtype, causal, offset = case
    print(f"attention forward {name}", flush=True)
    q, k, v, idx = _inputs(case)
    out, lse = P.sparse_attention_with_lse(to_gpu(q, dtype), to_gpu(k, dtype), to_gpu(v, dtype),
                                           torch.from_numpy(idx).cuda(), block,
                                           query_offset=offset, causal=causal)
    pos = O.query_positions(batch, tq, n, offset)
    ref_o, ref_lse = O.sparse_attention(q, k, v, idx, block, positions=pos, causal=causal)
    out = out.float().cpu().numpy()
    lse = lse.cpu().numpy()
    assert excess_error(out, ref_o, dtype) <= TOL[dtype]
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(lse), ~fin)
    assert np.abs(lse[fin] - ref_lse[fin]).max() <= max(TOL[dtype], 1e-5)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_matches_oracle(P, case):
    name, batch, tq, n, qh, kh, dim, block, topk, dtype, causal, offset = case
    print(f"attention backward {name}", flush=True)
    q, k, v, idx = _inputs(case)
    dout = np.random.default_rng(5).standard_normal((batch, tq, qh, dim)).astype(np.float32)
    dout = O.round_storage(dout, dtype)
    qg, kg, vg = (to_gpu(x, dtype).requires_grad_(True) for x in (q, k, v))
    out = P.sparse_attention(qg, kg, vg, torch.from_numpy(idx).cuda(), block,
                             query_offset=offset, causal=causal)
    out.backward(to_gpu(dout, dtype))
    pos = O.query_positions(batch, tq, n, offset)
    dq, dk, dv = O.sparse_attention_backward(q, k, v, idx, dout, block, positions=pos,
                                             causal=causal)
    for name_, mine, ref in (("dq", qg.grad, dq), ("dk", kg.grad, dk), ("dv", vg.grad, dv)):
        mine = mine.float().cpu().numpy()
        err = excess_error(mine, ref, dtype)
        print(f"{name_} max-abs error {np.abs(mine - ref).max():.3e}, "
              f"beyond half an output ulp {err:.3e}")
        assert err <= TOL[dtype], f"{name_} max-abs error {err}"


@pytest.mark.parametrize("case", [CASES[2], CASES[16]], ids=[CASES[2][0], CASES[16][0]])
@pytest.mark.parametrize("shift", [20, -30])
def test_backward_scales_exactly(P, case, shift):
    """Gradients are linear in dO: scaling dO by 2^shift scales them by exactly
    2^shift (bf16 keeps fp32's exponent range).  dQ, a slot-ordered sum of
    per-request partials, must match bit for bit, which holds only if its
    partials carry the scale through their exponents (no fp16 overflow at
    2^20, none of fp16's subnormals at 2^-30).  dK and dV sum a tile's requests
    in bucketing order, which varies between runs, so they are held to a
    bf16-level bound.  Head dims 128 and 64 cover both register-tile backward
    kernels."""
    name, batch, tq, n, qh, kh, dim, block, topk, dtype, causal, offset = case
    print(f"attention backward scale 2^{shift} {name}", flush=True)
    q, k, v, idx = _inputs(case)
    dout = np.random.default_rng(7).standard_normal((batch, tq, qh, dim)).astype(np.float32)
    ids = torch.from_numpy(idx).cuda()

    def grads(scale):
        qg, kg, vg = (to_gpu(x, dtype).requires_grad_(True) for x in (q, k, v))
        out = P.sparse_attention(qg, kg, vg, ids, block, query_offset=offset, causal=causal)
        out.backward(to_gpu(dout, dtype) * scale)
        return [g.grad.float() for g in (qg, kg, vg)]

    base = grads(1.0)
    scaled = grads(2.0 ** shift)
    assert torch.equal(base[0] * 2.0 ** shift, scaled[0]), "dq is not scaled exactly"
    for name_, a, b in zip(("dk", "dv"), base[1:], scaled[1:]):
        a = a * 2.0 ** shift
        err = ((a - b).abs().max() / a.abs().max()).item()
        print(f"{name_} relative difference {err:.3e}")
        assert err <= 2 ** -7, f"{name_} relative difference {err}"


def test_selected_blocks_end_to_end(P):
    """select_blocks -> sparse_attention, as the reference's example does."""
    q, k, v = structured_qkv(11, 1, 2048, 16, 4, 128, "bf16")
    qg, kg, vg = to_gpu(q, "bf16"), to_gpu(k, "bf16"), to_gpu(v, "bf16")
    ids = P.select_blocks(qg, kg, "pisa", 64, 16, force_recent=1, branching=4)
    out, lse = P.sparse_attention_with_lse(qg, kg, vg, ids, 64)
    ref_o, ref_lse = O.sparse_attention(q, k, v, ids.cpu().numpy(), 64)
    assert excess_error(out.float().cpu().numpy(), ref_o, "bf16") <= 2e-2
    assert np.abs(lse.cpu().numpy() - ref_lse).max() <= 2e-2


@pytest.mark.parametrize("dv", [64, 32])
def test_forward_value_dim_differs(P, dv):
    """Dv != D (the general forward kernels): O [B,Tq,Hq,Dv] and LSE."""
    case = CASES[2]
    name, batch, tq, n, qh, kh, dim, block, topk, dtype, causal, offset = case
    print(f"attention forward {name} dv={dv}", flush=True)
    q, k, v, idx = _inputs(case)
    v = np.ascontiguousarray(v[..., :dv])
    out, lse = P.sparse_attention_with_lse(to_gpu(q, dtype), to_gpu(k, dtype), to_gpu(v, dtype),
                                           torch.from_numpy(idx).cuda(), block)
    ref_o, ref_lse = O.sparse_attention(q, k, v, idx, block)
    assert out.shape[-1] == dv
    assert excess_error(out.float().cpu().numpy(), ref_o, dtype) <= TOL[dtype]
    fin = np.isfinite(ref_lse)
    assert np.abs(lse.cpu().numpy()[fin] - ref_lse[fin]).max() <= TOL[dtype]


@pytest.mark.parametrize("kind", ["padding", "out-of-range"])
@pytest.mark.parametrize("tq", [1, 700])
def test_no_visible_key_anywhere(P, kind, tq):
    """Every id -1, or every id past the last block: no request reaches a tile
    (the tile walks start on an empty list), O = 0 and LSE = -inf for every row
    and every gradient is 0, as the reference's masked softmax gives
    (sparse_attn_torch.py:28-31)."""
    print(f"attention without visible keys {kind} tq={tq}", flush=True)
    n, block = 700, 64
    q, k, v = structured_qkv(31, 2, n, 8, 2, 128, "bf16")
    q = np.ascontiguousarray(q[:, n - tq:])
    fill = -1 if kind == "padding" else -(-n // block) + 2
    idx = torch.full((2, tq, 2, 8), fill, dtype=torch.int64, device="cuda")
    qg, kg, vg = (to_gpu(x, "bf16").requires_grad_(True) for x in (q, k, v))
    out, lse = P.sparse_attention_with_lse(qg.detach(), kg.detach(), vg.detach(), idx, block)
    assert torch.count_nonzero(out).item() == 0
    assert torch.isneginf(lse).all()
    out = P.sparse_attention(qg, kg, vg, idx, block)
    out.backward(torch.ones_like(out))
    for g in (qg.grad, kg.grad, vg.grad):
        assert torch.count_nonzero(g).item() == 0


def test_int32_indices_and_determinism(P):
    q, k, v, idx = _inputs(CASES[2])
    qg, kg, vg = (to_gpu(x, "bf16") for x in (q, k, v))
    a = P.sparse_attention(qg, kg, vg, torch.from_numpy(idx).cuda(), 64)
    b = P.sparse_attention(qg, kg, vg, torch.from_numpy(idx).int().cuda(), 64)
    assert torch.equal(a, b)


def _packed_indices(seed, bounds, kh, topk, block):
    """Document-local ids for a packed prefill (every document's query rows)."""
    parts = []
    for d, (s, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        parts.append(_indices(seed + d, 1, e - s, kh, topk, e - s, block, empty_rows=False))
    return np.concatenate(parts, 1)


def test_packed_documents_forward_backward(P):
    """cu_seqlens (``sparse_attn.py:29-54``): each document attends its own keys with
    document-local ids and positions; O, LSE and dQ/dK/dV equal the per-document oracle."""
    bounds = [0, 700, 1500, 1536, 2300]
    n, qh, kh, dim, block, topk, dtype = bounds[-1], 8, 2, 128, 64, 6, "bf16"
    print("attention packed documents", flush=True)
    q, k, v = structured_qkv(31, 1, n, qh, kh, dim, dtype)
    idx = _packed_indices(40, bounds, kh, topk, block)
    dout = O.round_storage(np.random.default_rng(6).standard_normal((1, n, qh, dim)).astype(np.float32), dtype)
    qg, kg, vg = (to_gpu(x, dtype).requires_grad_(True) for x in (q, k, v))
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    out, lse = P.sparse_attention_with_lse(qg, kg, vg, torch.from_numpy(idx).cuda(), block, cu_seqlens=cu)
    out.backward(to_gpu(dout, dtype))
    ref_o, ref_lse, grads = [], [], [[], [], []]
    for s, e in zip(bounds[:-1], bounds[1:]):
        sl = slice(s, e)
        o_, l_ = O.sparse_attention(q[:, sl], k[:, sl], v[:, sl], idx[:, sl], block)
        g_ = O.sparse_attention_backward(q[:, sl], k[:, sl], v[:, sl], idx[:, sl], dout[:, sl], block)
        ref_o.append(o_)
        ref_lse.append(l_)
        for j in range(3):
            grads[j].append(g_[j])
    assert excess_error(out.detach().float().cpu().numpy(), np.concatenate(ref_o, 1), dtype) <= TOL[dtype]
    mine_lse, ref_lse = lse.cpu().numpy(), np.concatenate(ref_lse, 1)
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(mine_lse), ~fin)
    assert np.abs(mine_lse[fin] - ref_lse[fin]).max() <= TOL[dtype]
    for name_, mine, ref in zip(("dq", "dk", "dv"), (qg.grad, kg.grad, vg.grad), grads):
        err = excess_error(mine.float().cpu().numpy(), np.concatenate(ref, 1), dtype)
        print(f"packed {name_} excess max-abs error {err:.3e}")
        assert err <= TOL[dtype], f"packed {name_} max-abs error {err}"


def test_packed_decode(P):
    """One decode query per document (``validation.py:72-79``): local position = document
    length - 1 unless an offset per document is given."""
    bounds = [0, 900, 2000, 4096]
    kh, qh, dim, block, topk = 2, 8, 64, 64, 5
    print("attention packed decode", flush=True)
    _, k, v = structured_qkv(32, 1, bounds[-1], qh, kh, dim, "bf16")
    q = O.round_storage(np.random.default_rng(7).standard_normal((1, 3, qh, dim)).astype(np.float32), "bf16")
    rng = np.random.default_rng(8)
    idx = np.full((1, 3, kh, topk), -1, dtype=np.int64)
    for d, (s, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        blocks = -(-(e - s) // block)
        for h in range(kh):
            pick = rng.permutation(blocks)[:topk]
            idx[0, d, h, :len(pick)] = pick
    cu = torch.tensor(bounds, dtype=torch.int64, device="cuda")
    out, lse = P.sparse_attention_with_lse(to_gpu(q, "bf16"), to_gpu(k, "bf16"), to_gpu(v, "bf16"),
                                           torch.from_numpy(idx).cuda(), block, cu_seqlens=cu)
    for d, (s, e) in enumerate(zip(bounds[:-1], bounds[1:])):
        pos = np.array([[e - s - 1]])
        ref_o, ref_lse = O.sparse_attention(q[:, d:d + 1], k[:, s:e], v[:, s:e], idx[:, d:d + 1], block,
                                            positions=pos)
        assert excess_error(out[:, d:d + 1].float().cpu().numpy(), ref_o, "bf16") <= 2e-2
        assert np.abs(lse[:, d:d + 1].cpu().numpy() - ref_lse).max() <= 2e-2


def test_packed_attention_is_one_launch_sequence(P):
    """The packed forward runs every document in one launch of each kernel (the
    documents share the launch's key blocks) - not one launch series per document,
    the per-document loop of ``sparse_attn.py:40-54`` - and equals the documents
    attended one at a time, bit for bit."""
    from nlogn_pisa_amd import _lib
    bounds = [0, 130, 700, 1500, 1536, 2300, 2301, 4096]
    n, qh, kh, dim, block, topk = bounds[-1], 8, 2, 64, 64, 6
    q, k, v = structured_qkv(33, 1, n, qh, kh, dim, "bf16")
    idx = _packed_indices(41, bounds, kh, topk, block)
    qg, kg, vg = (to_gpu(x, "bf16") for x in (q, k, v))
    ig = torch.from_numpy(idx).cuda()
    cu = torch.tensor(bounds, dtype=torch.int32, device="cuda")
    with torch.no_grad():
        _lib.profile_begin()
        out, lse = P.sparse_attention_with_lse(qg, kg, vg, ig, block, cu_seqlens=cu)
        kernels = _lib.profile_end()
        launches = {name: count for name, (count, _) in kernels.items()}
        print("packed launches:", launches)
        assert launches.get("attn_fwd", 0) + launches.get("attn_fwd_direct", 0) == 1
        assert launches["attn_combine"] == 1
        for s, e in zip(bounds[:-1], bounds[1:]):
            o, l = P.sparse_attention_with_lse(qg[:, s:e], kg[:, s:e], vg[:, s:e], ig[:, s:e],
                                               block)
            assert torch.equal(out[:, s:e], o), f"document [{s}, {e})"
            assert torch.equal(lse[:, s:e], l), f"document [{s}, {e})"


def test_strided_views_equal_contiguous(P):
    """Inputs as views, as a model hands them over: q, k, v sliced out of one fused QKV
    projection (token stride (Hq + 2 Hkv) D, used in place), and k, v sliced out of
    wider rows (head-dim slices, copied).  Selection ids and O equal those of
    contiguous copies bit for bit, dQ too (it is reproducible), dK/dV within bf16
    rounding (their float32 sums follow the tile order)."""
    print("attention strided views", flush=True)
    batch, n, qh, kh, dim, block = 2, 700, 8, 2, 64, 64
    torch.manual_seed(9)
    fused = torch.randn(batch, n, qh + 2 * kh, dim, device="cuda").to(torch.bfloat16)
    wide = torch.randn(batch, n, 2 * kh, dim + 32, device="cuda").to(torch.bfloat16)
    layouts = {
        "fused": (fused[:, :, :qh], fused[:, :, qh:qh + kh], fused[:, :, qh + kh:]),
        "wide": (fused[:, :, :qh], wide[:, :, :kh, :dim], wide[:, :, kh:, 16:16 + dim]),
    }
    dout = torch.randn(batch, n, qh, dim, device="cuda").to(torch.bfloat16)
    for name, (q, k, v) in layouts.items():
        print(f"layout {name}", flush=True)
        assert not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous())
        ids = P.select_blocks(q, k, "pisa", block, 6, force_recent=1, branching=4)
        want = P.select_blocks(q.contiguous(), k.contiguous(), "pisa", block, 6, force_recent=1,
                               branching=4)
        assert torch.equal(ids, want), name
        grads = []
        for inputs in ((q, k, v), (q.contiguous(), k.contiguous(), v.contiguous())):
            leaves = [x.detach().clone().requires_grad_(True) if x.is_contiguous() else
                      x.detach().requires_grad_(True) for x in inputs]
            out = P.sparse_attention(*leaves, ids, block)
            out.backward(dout)
            grads.append((out.detach(), *(x.grad for x in leaves)))
        (o1, dq1, dk1, dv1), (o2, dq2, dk2, dv2) = grads
        assert torch.equal(o1, o2) and torch.equal(dq1, dq2), name
        for g1, g2 in ((dk1, dk2), (dv1, dv2)):
            # one bf16 rounding apart at most: 2e-2, or one ulp (<= 2^-7 |value|) above 2.56
            bound = torch.clamp(g2.float().abs() * 2.0 ** -7, min=2e-2)
            assert ((g1.float() - g2.float()).abs() <= bound).all(), name
