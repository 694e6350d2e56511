"""Build ``libwiretorch_amd.so`` (the HIP kernels and their C-ABI) for gfx950, in-tree.

    python -m wiretorch_amd.build

Flags: ``-ffp-contract=off`` keeps every float32 operation separately rounded, as the
reference's CPU step is (no fused multiply-add); packed FP32 instructions are disabled.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
LIBRARY = PACKAGE / "libwiretorch_amd.so"
SOURCES = [PACKAGE / "csrc" / "wt_kernels.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fPIC",
    "-shared",
]


def build(verbose: bool = False) -> Path:
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, *map(str, SOURCES), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errors = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{errors}")
    if verbose and errors.strip():
        print(errors, file=sys.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
