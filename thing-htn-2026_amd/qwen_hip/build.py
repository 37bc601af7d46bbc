"""Build libqwen_hip.so (gfx950) in place with hipcc.

``python -m qwen_hip.build`` (run from ``thing-htn-2026_amd/``) or
``build_library()`` compiles every ``csrc/*.hip`` to an object (in parallel)
and links them into ``qwen_hip/libqwen_hip.so``. Packed-fp32 instructions are
disabled for all device code (``-target-feature -packed-fp32-ops``).
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "csrc")
LIB = os.path.join(HERE, "libqwen_hip.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{res.stderr[-4000:]}")


def build_library(verbose: bool = False, jobs: int | None = None) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with tempfile.TemporaryDirectory(prefix="qwen_hip_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s) + ".o") for s in srcs]
        cmds = [[hipcc, *HIPCC_FLAGS, "-I", CSRC, "-c", s, "-o", o] for s, o in zip(srcs, objs)]
        if verbose:
            for c in cmds:
                print(" ".join(c), flush=True)
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            list(pool.map(_run, cmds))
        out = LIB + ".tmp"
        link = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", out]
        if verbose:
            print(" ".join(link), flush=True)
        _run(link)
        os.replace(out, LIB)
    return LIB


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
