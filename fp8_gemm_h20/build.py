"""Build libfp8bg.so in-tree: `python -m fp8_gemm_h20.build`.

hipcc cross-compiles for gfx950 without a GPU.  Packed-fp32 VALU forms are
disabled for all device code (-packed-fp32-ops), and MFMA instructions use the
VGPR form for their results (-amdgpu-mfma-vgpr-form).
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / "csrc" / "fp8bg.hip"
INCLUDE = ROOT / "include"
OUT = PKG / "libfp8bg.so"
ARCH = os.environ.get("FP8BG_ARCH", "gfx950")


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfp8bg.so)")


def command(out=OUT):
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            # MFMA results in VGPRs: every partial product is promoted by VALU
            # FMAs right away, so AGPR destinations only add copies
            "-mllvm", "-amdgpu-mfma-vgpr-form=1",
            f"-I{INCLUDE}", "-o", str(out), str(SRC)]


def build(verbose=False):
    tmp = OUT.with_suffix(".so.tmp")
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {OUT.name}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
