"""Invariants of the generated gfx950 code that the kernels rely on (CPU only).

The attention and Linear + GELU kernels issue their global->LDS copies as
inline assembly that writes M0 (the LDS address of the copy).  M0 is a
register the compiler reserves, so the copies are only safe while no
compiler-generated instruction of those kernels uses M0: this test compiles
both sources to gfx950 assembly (hipcc, no GPU needed) and checks that every
reference to m0 sits inside an inline-assembly block.
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


@pytest.mark.parametrize("name", ["attention_fwd.hip", "linear_gelu_fwd.hip"])
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
