"""Invariants of the generated gfx950 code that the kernels rely on (CPU only).

The attention and linear kernels issue their global->LDS copies as inline
assembly that writes M0 (the LDS address of the copy).  M0 is a register the
compiler reserves, so the copies are only safe while no compiler-generated
instruction of those kernels uses M0: the first test compiles each source to gfx950
assembly (hipcc, no GPU needed) and checks that every reference to m0 sits
inside an inline-assembly block.  The second checks the buffer offsets the
short-sequence kernels rely on for their row bounds.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
CSRC = REPO / "triton-transformer-kernels_amd" / "csrc"


def _assembly(source: Path, tmp_path: Path) -> str:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is not available")
    out = tmp_path / (source.stem + ".s")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           f"-I{REPO / 'include'}", f"-I{CSRC}", str(source), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out.read_text()


@pytest.mark.parametrize("name", ["attention_fwd.hip", "linear_fwd.hip"])
def test_m0_is_only_written_by_the_inline_copies(tmp_path, name):
    text = _assembly(CSRC / name, tmp_path)
    inside = outside = 0
    in_asm = False
    for line in text.splitlines():
        stripped = line.strip()
        if stripped.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if stripped.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if stripped.startswith(";") or "m0" not in stripped.replace(",", " ").split():
            continue
        if in_asm:
            inside += 1
        else:
            outside += 1
    assert inside > 0, "expected the inline LDS-DMA copies to write m0"
    assert outside == 0, f"{outside} compiler-generated instructions use m0 in {name}"


def test_short_kernel_buffer_offsets_keep_rows_in_the_range_check(tmp_path):
    # The fp32 short-sequence kernels read rows past S as zeros (and drop
    # stores to them) through the buffer range check, which covers the VGPR
    # offset and the instruction offset but not soffset.  That holds only
    # while every soffset is a column offset inside one row: 0, an inline
    # constant, or an SGPR set from an immediate below 256 bytes (a head_dim
    # 64 row).  Any row-dependent soffset would let a row past S through.
    text = _assembly(CSRC / "attention_fwd.hip", tmp_path)
    lines = text.splitlines()
    starts = [i for i, line in enumerate(lines)
              if line.startswith("_Z") and "short_kernel" in line.split(":")[0] and ":" in line]
    assert len(starts) == 6, "expected six short-kernel instantiations"
    checked = 0
    for start in starts:
        end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
        body = [line.split(";")[0].strip() for line in lines[start:end]]
        for i, ins in enumerate(body):
            if not ins.startswith("buffer_"):
                continue
            ops = ins.replace(",", " ").split()
            soffset = ops[4]
            checked += 1
            if soffset.lstrip("-").isdigit():
                assert 0 <= int(soffset) < 256, ins
                continue
            assert soffset.startswith("s") and soffset[1:].isdigit(), ins
            # The latest write to that SGPR before this instruction.
            for j in range(i - 1, -1, -1):
                words = body[j].replace(",", " ").split()
                if len(words) >= 2 and words[0].startswith("s_") and words[1] == soffset:
                    assert words[0] in ("s_mov_b32", "s_movk_i32"), f"{ins} <- {body[j]}"
                    assert 0 <= int(words[2], 0) < 256, f"{ins} <- {body[j]}"
                    break
            else:
                raise AssertionError(f"no definition of {soffset} before {ins}")
    assert checked > 0
