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
SETTINGS = dict(deadline=None, derandomize=True, database=None,
                suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large,
                                       HealthCheck.function_scoped_fixture])


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()   # the HIP library must load: no fallback
    return nlogn_pisa_amd


@st.composite
def selection_cases(draw):
    block = draw(st.sampled_from([16, 32, 64, 128, 256, 512]))
    # up to 400 blocks (routing three or four levels deep at b = 2), the last one ragged
    blocks = draw(st.one_of(st.integers(1, 40), st.integers(41, 400 if block <= 128 else 100)))
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
        dim=draw(st.sampled_from([16, 32, 48, 64, 96, 128, 256])),
        block=block,
        branching=draw(st.sampled_from([2, 4, 8])),
        topk=draw(st.sampled_from([k for k in (2, 4, 8, 16, 32, 64) if k >= int(ff) + fr])),
        method=draw(st.sampled_from(["pisa", "pisa2", "pisa1"])),
        ff=ff,
        fr=fr,
        dtype=draw(st.sampled_from(["fp32", "bf16", "fp16"])),
        schedule=draw(st.sampled_from(["auto", "grouped", "fused"])),
        needles=draw(st.sampled_from([0.0, 0.05])),
    )


@settings(max_examples=60, **SETTINGS)
@given(case=selection_cases())
def test_selection_random_shapes(P, case):
    c = case
    print(f"select property {c}", flush=True)
    q, k = structured_qkv(c["seed"], c["batch"], c["length"], c["group"] * c["kh"], c["kh"], c["dim"],
                          c["dtype"], offset_block=c["block"], needles=c["needles"], value=False,
                          tq=c["tq"])
    ids, trace = _run_select(P, q, k, c["dtype"], c["method"], c["block"], c["topk"], c["ff"],
                             c["fr"], None, c["schedule"], c["branching"])
    assert ids.shape == (c["batch"], q.shape[1], c["kh"], c["topk"])
    tokens = np.unique(np.linspace(0, q.shape[1] - 1, min(q.shape[1], 96)).astype(np.int64))
    _check_against(q, k, c["dtype"], c["method"], c["block"], c["topk"], c["ff"], c["fr"], None,
                   c["branching"], ids, trace, tokens=tokens)


@st.composite
def attention_cases(draw):
    block = draw(st.sampled_from([16, 32, 48, 64, 96, 128, 256]))
    length = draw(st.integers(min_value=1, max_value=12 * block))
    decode = draw(st.booleans())
    dim = draw(st.sampled_from([16, 32, 48, 64, 96, 128, 256]))
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
    )


def _random_ids(rng, batch, tq, kh, topk, blocks, duplicates):
    """Ids in [-1, blocks + 3): padding, blocks past the keys and, when asked,
    a block repeated within a row (its keys then count twice, as in the
    reference's gather)."""
    ids = rng.integers(-1, blocks + 3, size=(batch, tq, kh, topk)).astype(np.int64)
    if duplicates and topk > 1:
        ids[..., -1] = ids[..., 0]
    return ids


@settings(max_examples=60, **SETTINGS)
@given(case=attention_cases())
def test_attention_random_shapes(P, case):
    c = case
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
    pos = O.query_positions(c["batch"], c["tq"], c["length"], None)
    ref_o, ref_lse = O.sparse_attention(q, k, v, ids, c["block"], positions=pos, causal=c["causal"])
    ids_gpu = torch.from_numpy(ids).cuda()
    if not c["backward"]:
        out, lse = P.sparse_attention_with_lse(to_gpu(q, dt), to_gpu(k, dt), to_gpu(v, dt), ids_gpu,
                                               c["block"], causal=c["causal"])
        assert excess_error(out.float().cpu().numpy(), ref_o, dt) <= TOL[dt]
        lse = lse.cpu().numpy()
        fin = np.isfinite(ref_lse)
        assert np.array_equal(np.isneginf(lse), ~fin)
        if fin.any():
            assert np.abs(lse[fin] - ref_lse[fin]).max() <= max(TOL[dt], 1e-5)
        return
    dout = O.round_storage(rng.standard_normal(ref_o.shape).astype(np.float32), dt)
    qg, kg, vg = (to_gpu(x, dt).requires_grad_(True) for x in (q, k, v))
    out = P.sparse_attention(qg, kg, vg, ids_gpu, c["block"], causal=c["causal"])
    out.backward(to_gpu(dout, dt))
    assert excess_error(out.detach().float().cpu().numpy(), ref_o, dt) <= TOL[dt]
    grads = O.sparse_attention_backward(q, k, v, ids, dout, c["block"], positions=pos,
                                        causal=c["causal"])
    for name, mine, ref in zip(("dq", "dk", "dv"), (qg.grad, kg.grad, vg.grad), grads):
        err = excess_error(mine.float().cpu().numpy(), ref, dt)
        assert err <= TOL[dt], f"{name} excess error {err}"
