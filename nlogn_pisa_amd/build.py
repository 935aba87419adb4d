"""Build ``libpisa_hip.so`` (gfx950) in-tree with hipcc.

    python -m nlogn_pisa_amd.build          # or __graft_entry__.build()

Each ``csrc/*.hip`` file compiles to an object in ``csrc/_build`` (in
parallel), then one shared library is linked next to this file.  The build is
unconditional: it recompiles every time it is called.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(CSRC, "_build")
LIBRARY = os.path.join(HERE, "libpisa_hip.so")
ARCH = os.environ.get("PISA_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", os.path.join(HERE, "..", "include"),
]


# Per-source flags.  The attention kernels keep MFMA results in VGPRs (the
# backward's accumulators fill the VGPR file; AGPR-form products would copy
# every S/dP tile out of the accumulation registers before the VALU reads it).
SOURCE_FLAGS = {
    "pisa_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; install ROCm to build libpisa_hip.so")
    return path


def _compile(source, obj_dir, extra):
    obj = os.path.join(obj_dir, os.path.basename(source).replace(".hip", ".o"))
    cmd = [hipcc(), *FLAGS, *SOURCE_FLAGS.get(os.path.basename(source), []), *extra, "-c", source,
           "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{err}")
    return obj, err


def build(verbose=True, library=LIBRARY, extra_flags=(), obj_dir=OUT_DIR):
    """Compile every HIP source and link ``libpisa_hip.so``; returns its path.

    ``library``, ``extra_flags`` (extra hipcc options) and ``obj_dir`` build
    another copy of the library, loadable through ``PISA_HIP_LIBRARY``.
    """
    os.makedirs(obj_dir, exist_ok=True)
    sources = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        futures = [pool.submit(_compile, src, obj_dir, tuple(extra_flags)) for src in sources]
    errors = [f.exception() for f in futures if f.exception() is not None]
    if errors:
        raise RuntimeError("\n".join(str(e) for e in errors))
    results = [f.result() for f in futures]
    for obj, err in results:
        if verbose and err.strip():
            print(err, file=sys.stderr)
    tmp = library + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
           *(obj for obj, _ in results)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, library)
    if verbose:
        print(f"built {library}")
    return library


if __name__ == "__main__":
    build()
