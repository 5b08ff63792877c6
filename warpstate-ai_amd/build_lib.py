"""Compile ``csrc/*.hip`` for gfx950 into ``lib/libwarpstate_hip.so``.

Every translation unit is compiled on each call (in parallel), then linked into a fresh
library that atomically replaces the old one. Objects go to ``_build/``.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "lib" / "libwarpstate_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Evaluate FP32 epilogue arithmetic as written (no FMA contraction), like the
    # reference's eager path.
    "-ffp-contract=off",
    # Packed-FP32 instructions stay off in all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(source: Path) -> Path:
    obj = BUILD / (source.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        noise = "is not a recognized feature for this target"
        text = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
        raise RuntimeError(f"hipcc failed for {source.name}:\n{text}")
    return obj


def build(jobs: int | None = None) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD.mkdir(exist_ok=True)
    LIBRARY.parent.mkdir(exist_ok=True)
    jobs = jobs or min(len(sources), max(1, min(os.cpu_count() or 1, 16)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile, sources))
    staging = LIBRARY.with_name(LIBRARY.name + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(staging), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError("link failed:\n" + result.stderr)
    os.replace(staging, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(int(sys.argv[1]) if len(sys.argv) > 1 else None))
