"""Static check of the inline-assembly transposing reads in the 256 x 256 GEMM (CPU only).

With both operands M/N-contiguous, the k-loop issues its fragment reads as inline
assembly (``ds_read_b64_tr_b16``), which the compiler does not know to be LDS loads: it
inserts no wait before their results are used. Their results become usable only at the
explicit ``s_waitcnt lgkmcnt(0)`` that follows them (``tie_wait``). Until then no
instruction may read or write a destination register of a pending read, and no branch may
leave with one pending. The GPU tests check the results; this test compiles the kernels
to gfx950 assembly with the library's build flags and checks that rule on every
instantiation that uses the assembly reads, so that a compiler that moves or copies a
fragment register ahead of its wait fails here, before any GPU run.
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

TR_READ = "ds_read_b64_tr_b16"
REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")


def _regs(operands: str) -> set[int]:
    out = set()
    for lo, hi, one in REG.findall(operands):
        if one:
            out.add(int(one))
        else:
            out.update(range(int(lo), int(hi) + 1))
    return out


def _assembly(source: str, tmp_path: Path) -> str:
    target = tmp_path / (Path(source).stem + ".s")
    cmd = [HIPCC, *build_lib.FLAGS, f"-I{build_lib.CSRC}", "--cuda-device-only", "-S",
           str(build_lib.CSRC / source), "-o", str(target)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-2000:]
    return target.read_text()


def _kernels(text: str) -> dict[str, list[str]]:
    """Bodies of the unpaired gemm_fast_kernel<1, 1, false, ...> instantiations (both
    operands M/N-contiguous), the ones whose k-loop uses the assembly reads. The paired
    instantiation reads through the compiler's builtin, which the compiler waits for itself
    with counted waits that this check does not model."""
    bodies, name = {}, None
    for line in text.splitlines():
        m = re.match(r"^(_ZN2ws16gemm_fast_kernelILi1ELi1ELb0E\w*):", line)
        if m:
            name = m.group(1)
            bodies[name] = []
        elif name is not None:
            if line.strip().startswith("s_endpgm"):
                name = None
            else:
                bodies[name].append(line)
    return bodies


def _violations(body: list[str]) -> tuple[int, list[str]]:
    pending: set[int] = set()
    reads, bad = 0, []
    for raw in body:
        line = raw.split(";")[0].strip()
        if not line or line.endswith(":") or line.startswith("."):
            continue
        mnemonic, _, operands = line.partition(" ")
        if mnemonic == "s_waitcnt":
            if "lgkmcnt(0)" in operands:
                pending.clear()
            continue
        used = _regs(operands)
        if mnemonic == TR_READ:
            reads += 1
            dest = _regs(operands.split(",")[0])
            if dest & pending:
                bad.append(f"overwrites a pending read's register: {line}")
            pending |= dest
            continue
        if pending and mnemonic.startswith(("s_branch", "s_cbranch", "s_setpc", "s_swappc")):
            bad.append(f"branch with reads pending: {line}")
        if used & pending:
            bad.append(f"touches a pending read's register: {line}")
    if pending:
        bad.append("reads still pending at the end of the kernel")
    return reads, bad


@pytest.mark.parametrize("source", ["mm.hip", "fused.hip"])
def test_transposing_reads_are_waited_for_before_use(source, tmp_path):
    kernels = _kernels(_assembly(source, tmp_path))
    checked = {name: _violations(body) for name, body in kernels.items()}
    assert checked, f"no unpaired M/N-contiguous instantiation in {source}"
    for name, (reads, bad) in checked.items():
        assert reads >= 48, (name, reads)  # 24 reads per k32 step, two steps per k-tile
        assert not bad, (name, bad[:5])


def test_checker_flags_a_use_before_the_wait():
    """The rule itself, on hand-written sequences: a use of a pending read's register, a
    second read into it, or a branch while reads are pending is flagged; after the wait
    the same use is clean."""
    read = "\tds_read_b64_tr_b16 v[10:11], v200 offset:512"
    mfma = "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[8:11], v[20:23], v[0:3]"
    wait = "\ts_waitcnt lgkmcnt(0)"
    assert _violations([read, wait, mfma]) == (1, [])
    assert _violations([read, mfma, wait])[1]
    assert _violations([read, "\tds_read_b64_tr_b16 v[11:12], v201", wait])[1]
    assert _violations([read, "\ts_cbranch_scc1 .LBB0_5", wait])[1]
    assert _violations([read, "\tv_add_u32_e32 v30, v31, v32", wait]) == (1, [])
    assert _violations([read])[1]
