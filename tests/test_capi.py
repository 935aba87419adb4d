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
    assert lib.pisa_abi_version() == 2


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
