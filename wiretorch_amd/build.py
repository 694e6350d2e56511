"""Build ``libwiretorch_amd.so`` (the HIP kernels and their C-ABI) for gfx950, in-tree.

    python -m wiretorch_amd.build

Flags: ``-ffp-contract=off`` keeps every float32 operation separately rounded, as the
reference's CPU step is (no fused multiply-add); packed FP32 instructions are disabled.
"""

from __future__ import annotations

import os
import subprocess
import sys
import time
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
LIBRARY = PACKAGE / "libwiretorch_amd.so"
CSRC = PACKAGE / "csrc"
SOURCES = ([CSRC / "wt_kernels.hip", CSRC / "wt_rate.hip", CSRC / "wt_filter.hip",
            CSRC / "wt_gemm.hip"]
           + [CSRC / f"wt_run_s{s}.hip" for s in range(1, 9)])
OBJ_DIR = PACKAGE / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fPIC",
]


def _filter(stderr: str) -> str:
    noise = "is not a recognized feature for this target"
    return "\n".join(l for l in stderr.splitlines() if noise not in l)


def _stale(src: Path, obj: Path) -> bool:
    """Whether ``obj`` is older than its source or any header it may include."""
    if not obj.exists():
        return True
    headers = list(CSRC.glob("*.h")) + list((PACKAGE.parent / "include").glob("*.h"))
    return obj.stat().st_mtime < max(p.stat().st_mtime for p in [src, *headers])


def build(verbose: bool = False, jobs: int | None = None, changed_only: bool = False) -> Path:
    """Compile every source to an object (in parallel), then link the shared library.
    ``changed_only``: recompile only objects older than their sources or the headers."""
    OBJ_DIR.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 16)
    procs = []
    objects = []
    for src in SOURCES:
        obj = OBJ_DIR / (src.stem + ".o")
        objects.append(obj)
        if changed_only and not _stale(src, obj):
            continue
        cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        while len([p for p in procs if p[0].poll() is None]) >= jobs:
            procs[0][0].wait() if procs[0][0].poll() is None else None
            time.sleep(0.05)
        procs.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                       text=True), src))
    failed = []
    for proc, src in procs:
        out, err = proc.communicate()
        if proc.returncode != 0:
            failed.append(f"{src.name}:\n{_filter(err)}")
        elif verbose and _filter(err).strip():
            print(_filter(err), file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed ({proc.returncode}):\n{_filter(proc.stderr)}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True, changed_only="--changed" in sys.argv))
