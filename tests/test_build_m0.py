"""The folded GEMM's global-to-LDS copies set M0 in an asm statement, which is safe only while
nothing else in those kernels uses M0 (the compiler does not know the statement changes it).
This checks the built library's own gfx950 code: in every mmqh_kernel, each instruction that
names M0 is an `s_mov_b32 m0, ...` directly followed by a `global_load_lds_dwordx4`."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "kaillm_amd" / "libkai_hip.so"
OBJDUMP = Path("/opt/rocm/llvm/bin/llvm-objdump")


@pytest.mark.skipif(not LIB.exists() or not OBJDUMP.exists(), reason="needs the built library and llvm-objdump")
def test_folded_gemm_m0_only_before_copies(tmp_path):
    lib = tmp_path / LIB.name
    shutil.copy(LIB, lib)
    # the device code objects are extracted next to the copy
    subprocess.run([str(OBJDUMP), "--offloading", str(lib)], cwd=tmp_path, check=True, capture_output=True)
    objects = sorted(tmp_path.glob(f"{LIB.name}.*gfx950"))
    assert objects, "no gfx950 code object in the library"
    kernels, writes, other = set(), 0, []
    for obj in objects:
        text = subprocess.run([str(OBJDUMP), "-d", "--no-show-raw-insn", str(obj)], check=True,
                              capture_output=True, text=True).stdout.split("\n")
        current = None
        for i, line in enumerate(text):
            m = re.match(r"^[0-9a-f]+ <(.*)>:", line)
            if m:
                current = m.group(1)
                continue
            if not current or "mmqh_kernel" not in current:
                continue
            kernels.add(current)
            if re.search(r"\bm0\b", line):
                ins = line.strip()
                if ins.startswith("s_mov_b32 m0,") and i + 1 < len(text) and "global_load_lds_dwordx4" in text[i + 1]:
                    writes += 1
                else:
                    other.append((current[:60], ins))
    assert kernels, "no mmqh_kernel in the library"
    assert writes > 0, "no global-to-LDS copy found"
    assert not other, other[:5]
