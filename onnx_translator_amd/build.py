"""Build libtensor_ops_hip.so in-tree with hipcc for gfx950.

    python -m onnx_translator_amd.build          # or onnx_translator_amd.build.build()

Every source under csrc/ is compiled to an object in parallel, then linked
into ``onnx_translator_amd/libtensor_ops_hip.so``.  Flags:

* ``--offload-arch=gfx950``                         MI355X only, one code path;
* ``-ffp-contract=off``                             no FMA contraction: the fp64 paths
  replay the reference arithmetic operation by operation;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``  keep packed fp32 ops out of the
  generated code (hipcc's host pass warns that it does not know the feature).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtensor_ops_hip.so")
SOURCES = ["runtime.hip", "elementwise.hip", "qdq.hip", "reduce.hip", "gemm.hip", "conv.hip", "qconv.hip"]

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    noise = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if noise:
        sys.stderr.write("\n".join(noise[-40:]) + "\n")
    return obj


def build(jobs: int | None = None) -> str:
    """Compile and link; returns the library path.  Always rebuilds."""
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
