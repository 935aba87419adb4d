"""The C ABI library without a GPU: it loads, exports every function that
``include/pisa_hip.h`` declares, its ctypes mirror has the C struct layout, and
its host-side geometry agrees with the oracle.  No kernel is launched."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import oracle as O
from nlogn_pisa_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pisa_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pisa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIBRARY_PATH):
        pytest.fail("libpisa_hip.so is not built (run python -m nlogn_pisa_amd.build)")
    return _lib.library()


def test_exports_every_declared_function(lib):
    declared = declared_functions()
    assert len(declared) >= 14
    assert set(declared) == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.pisa_abi_version() == 3


def test_ctypes_structs_match_the_c_layout(tmp_path):
    """Compile the header with gcc and compare sizeof/offsetof with the ctypes mirror."""
    structs = {"pisa_qk_desc": _lib.QkDesc, "pisa_pyramid_desc": _lib.PyramidDesc,
               "pisa_select_params": _lib.SelectParams, "pisa_attn_desc": _lib.AttnDesc,
               "pisa_kernel_time": _lib.KernelTime}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.check_output([str(exe)]).decode().split("\n") if line)
    for cname, py in structs.items():
        assert int(got[cname]) == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert int(got[f"{cname}.{field}"]) == getattr(py, field).offset, (cname, field)


def test_routing_geometry_matches_oracle(lib):
    top, width = ctypes.c_int32(), ctypes.c_int32()
    for branching in (2, 4, 8, 16):
        for topk in (1, 4, 8, 16, 32, 64):
            for blocks in list(range(1, 600)) + [1023, 1024, 1025, 2048, 4096, 16384]:
                assert lib.pisa_routing_geometry(blocks, topk, branching, ctypes.byref(top),
                                                 ctypes.byref(width)) == 0
                assert (top.value, width.value) == O.routing_geometry(blocks, topk, branching)


def test_pyramid_layout_matches_oracle_levels(lib):
    from nlogn_pisa_amd.pooling import pyramid_layout
    for keys, block, branching in ((1000, 16, 2), (4096, 64, 4), (65536, 64, 4),
                                   (262144, 128, 8), (1, 64, 2), (130, 64, 3)):
        levels = O.build_pyramid(np.zeros((1, keys, 1, 1), np.float32), block, branching)
        offsets, lengths = pyramid_layout(keys, block, branching)
        assert lengths == [x.shape[1] for x in levels]
        assert offsets == list(np.cumsum([0] + lengths[:-1]))
        _, capped = pyramid_layout(keys, block, branching, 1)
        assert capped == lengths[:2]


def test_argument_errors_surface_without_a_gpu(lib):
    qk = _lib.QkDesc()
    params = _lib.SelectParams()
    assert lib.pisa_select_workspace_size(None, None) == 0
    status = lib.pisa_select(ctypes.byref(qk), ctypes.byref(params), None, None, None, None, 0,
                             None, None, None, 0, None)
    assert status == _lib.PISA_ERR_INVALID
    assert "nonempty" in lib.pisa_last_error().decode()
    with pytest.raises(ValueError, match="nonempty"):
        _lib.check(status)
    top, width = ctypes.c_int32(), ctypes.c_int32()
    assert lib.pisa_routing_geometry(0, 8, 2, ctypes.byref(top), ctypes.byref(width)) == \
        _lib.PISA_ERR_INVALID
    desc = _lib.AttnDesc()
    assert lib.pisa_attention_workspace_size(ctypes.byref(desc), 0) == 0


def _qk(query_heads=8, key_heads=2, head_dim=64, tokens=1024):
    qk = _lib.QkDesc(batch=1, query_tokens=tokens, query_heads=query_heads, key_tokens=tokens,
                     key_heads=key_heads, head_dim=head_dim, dtype=_lib.PISA_BF16)
    qk.q_stride_token, qk.k_stride_token = query_heads * head_dim, key_heads * head_dim
    qk.q_stride_batch, qk.k_stride_batch = tokens * qk.q_stride_token, tokens * qk.k_stride_token
    return qk


@pytest.mark.parametrize("shape, params, message", [
    (dict(query_heads=129, key_heads=1), {}, "up to 128 query heads"),
    (dict(head_dim=40), {}, "multiple of 16 up to 256"),
    (dict(head_dim=272), {}, "multiple of 16 up to 256"),
    ({}, dict(block_size=1 << 17), "block_size in \\[16, 65536\\]"),
    ({}, dict(block_size=48), "power-of-two block_size"),
    ({}, dict(topk=65), "topk must be in \\[1, 64\\]"),
])
def test_selection_refuses_unsupported_shapes_without_a_gpu(lib, shape, params, message):
    """The shape checks run on the host before anything reaches the device."""
    p = _lib.SelectParams(method=2, block_size=64, branching=2, topk=8, force_first=1,
                          force_recent=2, top=1, first_width=16, schedule=0)
    for key, value in params.items():
        setattr(p, key, value)
    status = lib.pisa_select(ctypes.byref(_qk(**shape)), ctypes.byref(p), None, None, None, None,
                             0, None, None, None, 0, None)
    assert status == _lib.PISA_ERR_UNSUPPORTED
    assert re.search(message, lib.pisa_last_error().decode())


@pytest.mark.parametrize("shape, block, topk, message", [
    (dict(query_heads=129, key_heads=1), 64, 8, "at most 128 query heads"),
    ({}, 256, 8, "block_size <= 128 and topk <= 64"),
    ({}, 64, 65, "block_size <= 128 and topk <= 64"),
])
def test_bsa_refuses_unsupported_shapes_without_a_gpu(lib, shape, block, topk, message):
    fake = ctypes.c_void_p(256)   # never dereferenced: the checks return first
    status = lib.pisa_bsa_select(ctypes.byref(_qk(**shape)), block, topk, 1, 2, fake, fake, fake, 0,
                                 fake, fake, 1 << 20, None)
    assert status == _lib.PISA_ERR_UNSUPPORTED
    assert message in lib.pisa_last_error().decode()
