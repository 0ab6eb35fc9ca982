"""Build libkai_hip.so in-tree with hipcc for gfx950.

Every HIP translation unit is compiled for gfx950 only, with packed-FP32
instruction selection disabled (-packed-fp32-ops); the host-only quantizer is
compiled with g++. Objects go to kaillm_amd/_build/, the shared library to
kaillm_amd/libkai_hip.so, which is what kaillm_amd.native loads.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libkai_hip.so"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results straight into VGPRs: the MMQ epilogue scales every MFMA output on the
    # VALU, and the AGPR form would add a v_accvgpr_read per element
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # per-kernel register and scratch report, checked below
    "-Rpass-analysis=kernel-resource-usage",
]
CXX_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-pthread"]


def _sources():
    hip = sorted(CSRC.glob("*.hip"))
    cpp = sorted(CSRC.glob("*.cpp"))
    return hip, cpp


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is harmless
    text = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(map(str, cmd))}\n{text}")
    return text


def _check_no_scratch(text, src):
    """Every kernel must be free of register spills: the small-M GEMM returned wrong sums
    from its later waves whenever it spilled (its workgroups are 16 waves with up to 160 KiB
    of LDS), so a spill anywhere fails the build instead of shipping."""
    name = None
    for line in text.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:")[1].split("[-Rpass")[0].strip()
        elif "ScratchSize [bytes/lane]:" in line:
            size = int(line.split("ScratchSize [bytes/lane]:")[1].split("[")[0])
            if size:
                raise RuntimeError(f"{src.name}: kernel {name} spills {size} bytes per lane to scratch")


def build(jobs=None, verbose=False):
    """Compile every source and link kaillm_amd/libkai_hip.so. Returns its path."""
    hip, cpp = _sources()
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(16, os.cpu_count() or 4)
    cmds = []
    objs = []
    for src in hip:
        obj = BUILD / (src.stem + ".o")
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
        objs.append(obj)
    for src in cpp:
        obj = BUILD / (src.stem + ".cpp.o")
        cmds.append([shutil.which("g++") or "g++", *CXX_FLAGS, "-c", str(src), "-o", str(obj)])
        objs.append(obj)
    with cf.ThreadPoolExecutor(jobs) as pool:
        for src, text in zip(hip + cpp, pool.map(_run, cmds)):
            if src.suffix == ".hip":
                _check_no_scratch(text, src)
                text = "\n".join(l for l in text.splitlines() if "kernel-resource-usage" not in l and "|" not in l)
            if verbose and text:
                print(text)
    tmp = OUT.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
