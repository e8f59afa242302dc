"""Builds ``libkarpo_attn.so`` in-tree with hipcc for gfx950 (no JIT cache: the library travels with the tree).

``python -m karpo_decision_amd.build`` or ``build()``; objects go to ``karpo_decision_amd/_build/``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
LIBRARY = PACKAGE / "libkarpo_attn.so"
ARCH = "gfx950"

#: hipcc flags for every translation unit. Packed FP32 VALU ops are switched off (the compiler still vectorises
#: nothing into v_pk_*_f32), the kernels target gfx950 only.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", f"-I{INCLUDE}", f"-I{CSRC}",
]
SOURCES = ["attn_fwd.hip", "attn_fwd_128.hip", "attn_bwd.hip", "attn_bwd_pair.hip", "capi.cpp", "plan.cpp",
           "scratch.hip"]
# per-source flags: the head-size-128 wide / long forward tiles under the iterative-ILP machine scheduler
SOURCE_FLAGS = {"attn_fwd_128.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]}


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(found):
        raise RuntimeError("hipcc not found: the ROCm toolchain is needed to build libkarpo_attn.so")
    return found


def _compile(name: str, out: Path, verbose: bool) -> str:
    obj = out / (name + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *SOURCE_FLAGS.get(name, []), "-c", str(CSRC / name), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    done = subprocess.run(cmd, capture_output=True, text=True)
    errors = "\n".join(line for line in (done.stdout + done.stderr).splitlines()
                       if "packed-fp32-ops" not in line)  # hipcc's host pass does not know the feature
    if done.returncode != 0:
        raise RuntimeError(f"hipcc failed on {name}:\n{errors}")
    if verbose and errors.strip():
        print(errors)
    return str(obj)


def build(verbose: bool = False) -> Path:
    """Compiles every source (one hipcc process per source, side by side) and links the shared library; returns its
    path. Always rebuilds."""
    out = PACKAGE / "_build"
    out.mkdir(exist_ok=True)
    workers = max(1, min(len(SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda name: _compile(name, out, verbose), SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", str(tmp)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"linking libkarpo_attn.so failed:\n{done.stdout}{done.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
