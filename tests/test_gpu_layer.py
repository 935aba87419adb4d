"""GPU parity of the attention layer (``pyramid_sparse_attention.py:71-222``) and its
rotary encoding (``rotary_torch.py:5-10``).

Bars: rotary within 1e-5 (fp32) or half an ulp + 1e-4 (16-bit) of the float64 oracle,
its gradient the inverse turn; the layer's prefill equals the oracle composition
(projections, rotary, selected-block attention with the layer's own ids) within 1e-4
(fp32); decode through the PyramidCache is bit-identical to decode over concatenated
keys; the layer's gradients match a float32 torch composition within 1e-4.
"""

import numpy as np
import pytest
import torch

import oracle as O
from parity import excess_error

pytestmark = pytest.mark.gpu

TORCH = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.fixture(scope="module")
def P():
    import nlogn_pisa_amd
    nlogn_pisa_amd._lib.library()
    return nlogn_pisa_amd


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
def test_rotary_matches_oracle(P, dtype):
    print(f"rotary {dtype}", flush=True)
    rng = np.random.default_rng(21)
    x = O.round_storage(rng.standard_normal((2, 37, 3, 64)).astype(np.float32), dtype)
    rope = P.RotaryEmbedding(64, 10000.0, 0.5)
    np.testing.assert_allclose(rope.theta.numpy().reshape(-1), O.rotary_frequency(64, 10000.0, 0.5),
                               rtol=1e-6)
    pos = np.stack([np.arange(37) + 5, np.arange(37) + 40000])
    xg = torch.from_numpy(x).to(TORCH[dtype]).cuda().requires_grad_(True)
    y = rope(xg, torch.from_numpy(pos).cuda())
    ref = O.rotary(x, rope.theta.numpy(), pos)
    got = y.detach().float().cpu().numpy()
    if dtype == "fp32":
        assert np.abs(got - ref).max() <= 1e-5
    else:
        assert excess_error(got, ref, dtype) <= 1e-4
    g = O.round_storage(rng.standard_normal(x.shape).astype(np.float32), dtype)
    y.backward(torch.from_numpy(g).to(TORCH[dtype]).cuda())
    ref_g = O.rotary(g, -rope.theta.numpy(), pos)
    got_g = xg.grad.float().cpu().numpy()
    if dtype == "fp32":
        assert np.abs(got_g - ref_g).max() <= 1e-5
    else:
        assert excess_error(got_g, ref_g, dtype) <= 1e-4


def test_rotary_fn_is_the_reference_operator(P):
    """``rotary_fn(x, frequency, positions, use_triton=...)`` (``lrpe/rotary.py:9-15``):
    any frequency shape and one position row per token (``[T]``) or per batch
    (``[B, T]``); equal to ``rotary`` and to the oracle."""
    rng = np.random.default_rng(22)
    x = O.round_storage(rng.standard_normal((2, 19, 4, 32)).astype(np.float32), "bf16")
    theta = O.rotary_frequency(32, 10000.0, 1.0).astype(np.float64)   # a float64 table
    xg = torch.from_numpy(x).to(torch.bfloat16).cuda()
    steps = torch.arange(19, device="cuda") + 3
    for use_triton in (True, False):
        got = P.rotary_fn(xg, torch.from_numpy(theta)[None], steps, use_triton=use_triton)
        assert torch.equal(got, P.rotary(xg, torch.from_numpy(theta).float().cuda(), steps[None]))
        ref = O.rotary(x, theta.astype(np.float32), np.broadcast_to(steps.cpu().numpy(), (2, 19)))
        assert excess_error(got.float().cpu().numpy(), ref, "bf16") <= 1e-4


def _layer(P, dtype, method="pisa", seed=0, **kw):
    torch.manual_seed(seed)
    cfg = dict(hidden_size=128, num_attention_heads=8, num_key_value_heads=2, head_dim=32,
               attention_method=method, block_size=32, topk=4, force_recent=1, branching=2,
               rope_fraction=0.5)
    cfg.update(kw)
    layer = P.PyramidSparseAttention(P.PisaLayerConfig(**cfg)).cuda().to(TORCH[dtype])
    return layer


@pytest.mark.parametrize("hd", [32, 40])   # 40: rows zero-padded by selection and attention
def test_layer_prefill_matches_oracle(P, hd):
    print(f"layer prefill fp32 head dim {hd}", flush=True)
    layer = _layer(P, "fp32", head_dim=hd)
    torch.manual_seed(1)
    x = torch.randn(1, 300, 128, device="cuda")
    out, _ = layer(x)
    c = layer.config
    with torch.no_grad():
        pos = P.token_positions(300, x.device)
        q = layer.rope(layer.q_proj(x).view(1, 300, 8, hd), pos)
        k = layer.rope(layer.k_proj(x).view(1, 300, 2, hd), pos)
        ids = P.select_blocks(q, k, method=c.attention_method, block_size=c.block_size, topk=c.topk,
                              force_recent=c.force_recent, branching=c.branching)
    w = {n: p.detach().double().cpu().numpy() for n, p in layer.named_parameters()}
    xn = x.double().cpu().numpy()
    qn = O.rotary((xn @ w["q_proj.weight"].T).reshape(1, 300, 8, hd), layer.rope.theta.cpu().numpy(),
                  np.arange(300)[None])
    kn = O.rotary((xn @ w["k_proj.weight"].T).reshape(1, 300, 2, hd), layer.rope.theta.cpu().numpy(),
                  np.arange(300)[None])
    vn = (xn @ w["v_proj.weight"].T).reshape(1, 300, 2, hd)
    o, _ = O.sparse_attention(qn, kn, vn, ids.cpu().numpy(), c.block_size)
    ref = o.reshape(1, 300, -1) @ w["o_proj.weight"].T
    assert np.abs(out.detach().double().cpu().numpy() - ref).max() <= 1e-4


@pytest.mark.parametrize("method", ["pisa", "pisa2", "pisa1"])
def test_layer_decode_cache_equals_concatenated_keys(P, method):
    """Decode with ``use_cache`` (PyramidCache, pyramid appended on the GPU) returns exactly
    what decode over the concatenated keys returns (pyramid built per call)."""
    print(f"layer decode {method}", flush=True)
    layer = _layer(P, "bf16", method, block_size=32, topk=6, force_recent=1, branching=4)
    torch.manual_seed(2)
    x = torch.randn(2, 211, 128, device="cuda").to(torch.bfloat16)
    steps = torch.randn(2, 5, 128, device="cuda").to(torch.bfloat16)
    with torch.no_grad():
        _, cache = layer(x, use_cache=True)
        for s in range(steps.shape[1]):
            plain = {"k": cache["k"].clone(), "v": cache["v"].clone()}
            step = steps[:, s:s + 1]
            out_cached, cache = layer(step, cache=cache, use_cache=True)
            out_plain, _ = layer(step, cache=plain, use_cache=False)
            assert torch.equal(out_cached, out_plain), f"decode step {s}"
            assert cache["k"].shape[1] == 211 + s + 1


def test_layer_gradients_match_torch(P):
    """Gradients w.r.t. the input and every projection weight against a float32 torch
    composition (same ids; dense masked attention; eager rotary formula)."""
    print("layer backward fp32", flush=True)
    layer = _layer(P, "fp32", topk=5)
    c = layer.config
    torch.manual_seed(3)
    x = torch.randn(1, 200, 128, device="cuda", requires_grad=True)
    g = torch.randn(1, 200, 128, device="cuda")
    out, _ = layer(x)
    out.backward(g)
    mine = [x.grad.clone()] + [p.grad.clone() for p in layer.parameters()]

    pos = torch.arange(200, device="cuda")
    with torch.no_grad():
        q0 = layer.rope(layer.q_proj(x).view(1, 200, 8, 32), pos[None])
        k0 = layer.rope(layer.k_proj(x).view(1, 200, 2, 32), pos[None])
        ids = P.select_blocks(q0, k0, method=c.attention_method, block_size=c.block_size,
                              topk=c.topk, force_recent=c.force_recent, branching=c.branching)
    tok = (ids[..., None] * c.block_size + torch.arange(c.block_size, device="cuda")).flatten(-2)
    valid = (ids[..., None] >= 0).expand(-1, -1, -1, -1, c.block_size).flatten(-2) & (tok <= pos[:, None, None])
    mask = torch.zeros(1, 200, 2, 200, device="cuda").scatter_add_(3, tok.clamp(0, 199),
                                                                  valid.float()) > 0

    def turn(t):
        ang = pos[None, :, None, None].float() * layer.rope.theta.reshape(-1)
        a, b = t.chunk(2, -1)
        return torch.cat((a * ang.cos() - b * ang.sin(), a * ang.sin() + b * ang.cos()), -1)

    x2 = x.detach().clone().requires_grad_(True)
    ws = [p.detach().clone().requires_grad_(True) for p in layer.parameters()]
    names = [n for n, _ in layer.named_parameters()]
    W = dict(zip(names, ws))
    q = turn((x2 @ W["q_proj.weight"].T).view(1, 200, 8, 32))
    k = turn((x2 @ W["k_proj.weight"].T).view(1, 200, 2, 32))
    v = (x2 @ W["v_proj.weight"].T).view(1, 200, 2, 32)
    qh = q.view(1, 200, 2, 4, 32)
    s = torch.einsum("btkgd,bnkd->btkgn", qh, k) * 32 ** -0.5
    s = s.masked_fill(~mask[:, :, :, None, :], float("-inf"))
    p = torch.softmax(s, -1)
    o = torch.einsum("btkgn,bnkd->btkgd", p, v).reshape(1, 200, -1)
    ref = o @ W["o_proj.weight"].T
    ref.backward(g)
    want = [x2.grad] + [w.grad for w in ws]
    for name, a, b in zip(["x"] + names, mine, want):
        err = (a - b).abs().max().item() / max(1.0, b.abs().max().item())
        print(f"grad {name} relative error {err:.2e}")
        assert err <= 1e-4, name


def test_layer_bsa_prefill_and_decode(P):
    """``attention_method="bsa"`` (``pisa_config.py:71-79``): prefill equals the flat BSA
    selection followed by sparse attention on the layer's own rotated q/k, and decode
    through the token cache (``key_storage``) equals decode over the concatenated keys."""
    print("layer bsa", flush=True)
    layer = _layer(P, "bf16", "bsa", block_size=32, topk=6, force_recent=2)
    c = layer.config
    torch.manual_seed(4)
    x = torch.randn(1, 300, 128, device="cuda").to(torch.bfloat16)
    with torch.no_grad():
        out, cache = layer(x, use_cache=True)
        pos = P.token_positions(300, x.device)
        q = layer.rope(layer.q_proj(x).view(1, 300, 8, 32), pos)
        k = layer.rope(layer.k_proj(x).view(1, 300, 2, 32), pos)
        v = layer.v_proj(x).view(1, 300, 2, 32)
        ids = P.bsa_fn(q, k, c.block_size, c.topk, force_first=c.force_first,
                       force_recent=c.force_recent)
        ref = layer.o_proj(P.sparse_attention(q, k, v, ids, block_size=c.block_size).flatten(2))
        assert torch.equal(out, ref)
        assert set(cache) == {"k", "v", "key_storage", "value_storage"}
        step = torch.randn(1, 1, 128, device="cuda").to(torch.bfloat16)
        plain = {"k": cache["k"].clone(), "v": cache["v"].clone()}
        out_cached, cache = layer(step, cache=cache, use_cache=True)
        out_plain, _ = layer(step, cache=plain, use_cache=False)
        assert torch.equal(out_cached, out_plain)
        assert cache["k"].shape[1] == 301
