"""Build libzkie_hip.so (gfx950) from zkie_amd/csrc with hipcc, in-tree.

Each .hip translation unit compiles to an object under zkie_amd/_build/ in
parallel, then one link step produces zkie_amd/libzkie_hip.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libzkie_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("ZKIE_OFFLOAD_ARCH", "gfx950")

# The VALU issue-rate probe of bench.py --valu-peak, a library of its own.
PROBE_SRC = "valu_probe.hip"
PROBE_LIB = os.path.join(HERE, "libzkie_valu_probe.so")

SOURCES = ["runtime.hip", "ntt.hip", "merkle.hip", "fold.hip", "sumcheck.hip", "prover_data.hip",
           "noalloc.hip"]

# Packed FP32 instructions are kept out of every code object.
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _compile(src: str, force: bool = True) -> str:
    obj = os.path.join(OUT_DIR, os.path.splitext(src)[0] + ".o")
    if not force and os.path.exists(obj):
        deps = [os.path.join(CSRC, f) for f in os.listdir(CSRC)] + [os.path.join(ROOT, "include", "zkie_hip.h")]
        if all(os.path.getmtime(obj) >= os.path.getmtime(d) for d in deps if d.endswith((".hpp", ".h"))) \
                and os.path.getmtime(obj) >= os.path.getmtime(os.path.join(CSRC, src)):
            return obj
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False, force: bool = True) -> str:
    """Compile every source (force) or only those older than their sources
    and the shared headers (force=False), then link."""
    os.makedirs(OUT_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda src: _compile(src, force), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    probe_obj = _compile(PROBE_SRC, force)
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", probe_obj, "-o", PROBE_LIB + ".tmp"],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True, force="--incremental" not in sys.argv)
    sys.exit(0)
