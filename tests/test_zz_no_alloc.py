"""The allocation-free attention forward (``pisa_sparse_attention_fwd_noalloc``)
against the workspace entry point (``pisa_sparse_attention_fwd``), through the C ABI.

Both run the same kernels, so O and LSE must be bit-identical; the test makes two
calls in a row on each path (the second with a smaller input, so the static
scratch holds the first call's contents) for the direct (decode) and the bucketed
(prefill) schedules, and checks O against the float64 oracle as well.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from parity import excess_error, structured_qkv, to_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()
    return nlogn_pisa_amd


def _ids(seed, batch, tq, kh, topk, n, block):
    rng = np.random.default_rng(seed)
    blocks = -(-n // block)
    pos = O.query_positions(batch, tq, n)
    idx = np.full((batch, tq, kh, topk), -1, dtype=np.int64)
    for b in range(batch):
        for t in range(tq):
            cur = pos[b, t] // block
            for h in range(kh):
                pick = [cur] + [int(x) for x in rng.permutation(cur + 1) if x != cur][:topk - 1]
                idx[b, t, h, :len(pick)] = pick
    return idx


def _both(P, q, k, v, idx, block):
    """(O, LSE) of the workspace entry point and of the allocation-free one."""
    from nlogn_pisa_amd import _lib
    from nlogn_pisa_amd._common import ptr, stream_of, workspace
    from nlogn_pisa_amd.attention import _attn_desc
    lib = _lib.library()
    positions = P.query_positions(q, k).contiguous()
    desc = _attn_desc(q, k, v, idx, block, q.shape[-1] ** -0.5, True)
    results = []
    for noalloc in (False, True):
        out = torch.empty(q.shape, device=q.device, dtype=q.dtype)
        lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
        if noalloc:
            rc = lib.pisa_sparse_attention_fwd_noalloc(
                ctypes.byref(desc), ptr(q), ptr(k), ptr(v), ptr(idx), ptr(positions),
                positions.stride(0), ptr(out), ptr(lse), None, stream_of(q))
        else:
            ws = workspace(lib.pisa_attention_workspace_size(ctypes.byref(desc), 0), q.device)
            rc = lib.pisa_sparse_attention_fwd(
                ctypes.byref(desc), ptr(q), ptr(k), ptr(v), ptr(idx), ptr(positions),
                positions.stride(0), ptr(out), ptr(lse), None, ptr(ws), ws.numel(), stream_of(q))
        _lib.check(rc)
        torch.cuda.synchronize()
        results.append((out, lse))
    return results


CALLS = [
    # name, B, Tq, N, Hq, Hkv, D, C, K: a large call, then a smaller one of the same schedule
    ("decode-large", 8, 1, 32768, 32, 8, 128, 64, 32),
    ("decode-small", 2, 1, 4096, 16, 4, 128, 64, 8),
    ("prefill-large", 1, 1024, 1024, 16, 4, 128, 64, 8),
    ("prefill-small", 1, 700, 700, 8, 2, 64, 32, 6),
]


@pytest.mark.parametrize("pair", [(0, 1), (2, 3)], ids=["decode", "prefill"])
def test_noalloc_equals_workspace_entry(P, pair):
    for index in pair:
        name, batch, tq, n, qh, kh, dim, block, topk = CALLS[index]
        print(f"no-alloc attention {name}", flush=True)
        q, k, v = structured_qkv(index + 40, batch, n, qh, kh, dim, "bf16")
        q = q[:, n - tq:]
        idx = _ids(index, batch, tq, kh, topk, n, block)
        qg, kg, vg = (to_gpu(x, "bf16") for x in (q, k, v))
        ig = torch.from_numpy(idx).cuda()
        (o_ws, l_ws), (o_na, l_na) = _both(P, qg, kg, vg, ig, block)
        assert torch.equal(o_ws, o_na), f"{name}: O differs"
        assert torch.equal(l_ws, l_na), f"{name}: LSE differs"
        ref_o, _ = O.sparse_attention(q, k, v, idx, block)
        assert excess_error(o_na.float().cpu().numpy(), ref_o, "bf16") <= 2e-2


def test_noalloc_around_a_call_without_visible_keys(P):
    """The scratch keeps the previous call's buckets and tile cursors: a prefill with
    real ids, one whose ids are all padding (no request reaches a tile), then the
    first again, each bit-identical to the workspace entry point, the second
    with O = 0 and LSE = -inf."""
    name, batch, tq, n, qh, kh, dim, block, topk = CALLS[3]
    q, k, v = structured_qkv(77, batch, n, qh, kh, dim, "bf16")
    q = q[:, n - tq:]
    real = torch.from_numpy(_ids(9, batch, tq, kh, topk, n, block)).cuda()
    empty = torch.full_like(real, -1)
    qg, kg, vg = (to_gpu(x, "bf16") for x in (q, k, v))
    for step, ig in enumerate((real, empty, real)):
        print(f"no-alloc attention sequence step {step}", flush=True)
        (o_ws, l_ws), (o_na, l_na) = _both(P, qg, kg, vg, ig, block)
        assert torch.equal(o_ws, o_na) and torch.equal(l_ws, l_na), f"step {step} differs"
        if step == 1:
            assert torch.count_nonzero(o_na).item() == 0
            assert torch.isneginf(l_na).all()


def test_noalloc_rejects_oversized(P):
    """A shape whose workspace exceeds the static scratch is refused before any launch."""
    from nlogn_pisa_amd import _lib
    from nlogn_pisa_amd.attention import _attn_desc
    lib = _lib.library()
    q = torch.empty(1, 65536, 32, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(1, 65536, 8, 128, dtype=torch.bfloat16, device="cuda")
    idx = torch.empty(1, 65536, 8, 32, dtype=torch.int64, device="cuda")
    desc = _attn_desc(q, k, k, idx, 64, 128 ** -0.5, True)
    assert lib.pisa_attention_workspace_size(ctypes.byref(desc), 0) > lib.pisa_noalloc_scratch_bytes()
    rc = lib.pisa_sparse_attention_fwd_noalloc(ctypes.byref(desc), ctypes.c_void_p(q.data_ptr()),
                                               ctypes.c_void_p(k.data_ptr()),
                                               ctypes.c_void_p(k.data_ptr()),
                                               ctypes.c_void_p(idx.data_ptr()),
                                               ctypes.c_void_p(idx.data_ptr()), 65536,
                                               ctypes.c_void_p(q.data_ptr()),
                                               ctypes.c_void_p(q.data_ptr()), None, None)
    assert rc == _lib.PISA_ERR_WORKSPACE
    assert b"scratch" in lib.pisa_last_error()
