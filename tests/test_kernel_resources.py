"""Static check of private scratch use by the kernels of the allocation-free entry point
(CPU only).

``ws_rmsnorm_backward_static`` promises to call no allocator. A kernel that spills
registers to private scratch memory makes the HIP runtime provide that memory at launch,
so every kernel the static path can launch must use none: for rows of up to 2048 columns
the vector row kernels (1, 2 and 4 segments of 512 columns) and the generic row kernel
(widths that are not a multiple of 8, unaligned views); for wider rows, up to 8192, the
block-per-row vector kernels (2 and 4 chunks of 2048 columns) and generic kernels (16 and
32 columns per thread); each in both rounding modes; and both forms of the weight
reduction. The compiler's resource remarks for ``rowops.hip``, built with the library's
flags, give each kernel's scratch bytes per lane.
"""
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE = ROOT / "warpstate-ai_amd"
sys.path.insert(0, str(PACKAGE))

import build_lib  # noqa: E402

HIPCC = shutil.which(build_lib.HIPCC) or (build_lib.HIPCC if Path(build_lib.HIPCC).exists() else None)
pytestmark = pytest.mark.skipif(HIPCC is None, reason="hipcc not available")

NAME = re.compile(r"remark: Function Name: (\S+)")
SCRATCH = re.compile(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)")


def _scratch_by_kernel(source: str, tmp_path: Path) -> dict[str, int]:
    cmd = [HIPCC, *build_lib.FLAGS, f"-I{build_lib.CSRC}", "--cuda-device-only", "-c",
           "-Rpass-analysis=kernel-resource-usage", str(build_lib.CSRC / source),
           "-o", str(tmp_path / "out.o")]
    result = subprocess.run(cmd, capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-2000:]
    out, name = {}, None
    for line in result.stderr.splitlines():
        m = NAME.search(line)
        if m:
            name = m.group(1)
            continue
        m = SCRATCH.search(line)
        if m and name is not None:
            out[name] = int(m.group(1))
            name = None
    return out


def test_static_rmsnorm_backward_kernels_use_no_private_scratch(tmp_path):
    scratch = _scratch_by_kernel("rowops.hip", tmp_path)
    # rmsnorm_bwd_kernel<SEGS, EAGER>: mangled as ...rmsnorm_bwd_kernelILi<SEGS>ELb<0|1>E...
    static_path = [k for k in scratch
                   if re.search(r"rmsnorm_bwd_kernelILi(1|2|4)ELb[01]E", k)
                   or "rmsnorm_bwd_generic_kernel" in k
                   or re.search(r"rmsnorm_bwd_wide_kernelILi(2|4)ELb[01]E", k)
                   or re.search(r"rmsnorm_bwd_wide_generic_kernelILi(16|32)ELb[01]E", k)
                   or "rms_weight_reduce_kernel" in k]
    assert len(static_path) == 18, sorted(scratch)
    assert {k: scratch[k] for k in static_path if scratch[k]} == {}
