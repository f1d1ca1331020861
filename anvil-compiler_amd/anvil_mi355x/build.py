"""Build libanvil_mi355x.so in-tree from csrc/*.hip for gfx950 (hipcc, no CMake).

    python -m anvil_mi355x.build           # or anvil_mi355x.build.build()

Every HIP source is compiled with packed-FP32 instruction selection off and linked into one shared library next
to this file, which the ctypes loader (anvil_mi355x.runtime) opens.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parents[1] / "include"
LIB = PKG / "libanvil_mi355x.so"
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-Wno-unused-command-line-argument", f"-I{INCLUDE}"]
# Per-source flags. attention.hip: MFMA accumulators in VGPRs. Its score tiles feed VALU requant code right after
# each MFMA, and with the accumulators in AGPRs every value would first need a v_accvgpr_read.
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources():
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every csrc/*.hip to an object and link LIB; raises RuntimeError with the compiler output."""
    objdir = PKG.parent / "_build"
    objdir.mkdir(exist_ok=True)

    def cc(src: Path):
        obj = objdir / (src.stem + ".o")
        cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
        if r.returncode:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{out}")
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(cc, sources()))
    tmp = LIB.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    shutil.rmtree(objdir, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
