"""Build libfp8bg.so in-tree: `python -m fp8_gemm_h20.build`.

hipcc cross-compiles for gfx950 without a GPU.  Packed-fp32 VALU forms are
disabled for all device code (-packed-fp32-ops), and MFMA instructions use the
VGPR form for their results (-amdgpu-mfma-vgpr-form).

csrc/fp8bg.hip is compiled once per part of its build partition (FP8BG_PART
1..7: the C ABI and small kernels, then the ring and skinny launchers by list
half and B layout), the parts in parallel, and the objects are linked into one
library.  FP8BG_ONE_TU=1 compiles it as one translation unit instead (the
same library, one hipcc process).
"""
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / "csrc" / "fp8bg.hip"
INCLUDE = ROOT / "include"
OUT = PKG / "libfp8bg.so"
ARCH = os.environ.get("FP8BG_ARCH", "gfx950")
PARTS = tuple(range(1, 8))


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfp8bg.so)")


def flags():
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            # MFMA results in VGPRs: every partial product is promoted by VALU
            # FMAs right away, so AGPR destinations only add copies
            "-mllvm", "-amdgpu-mfma-vgpr-form=1",
            f"-I{INCLUDE}"]


def command(out=OUT):
    """One translation unit straight to the shared library."""
    return [hipcc()] + flags() + ["-shared", "-o", str(out), str(SRC)]


def part_command(part, obj):
    return [hipcc()] + flags() + [f"-DFP8BG_PART={part}", "-c", "-o", str(obj), str(SRC)]


def link_command(objs, out):
    # every launcher the table of part 1 names must be defined in some part
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(out)] + \
        [str(o) for o in objs]


def _run(cmd, what):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) {what}")


def build(verbose=False):
    tmp = OUT.with_suffix(".so.tmp")
    if os.environ.get("FP8BG_ONE_TU") == "1":
        cmd = command(tmp)
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd, f"building {OUT.name}")
    else:
        with tempfile.TemporaryDirectory(prefix="fp8bg_build_") as d:
            objs = [Path(d) / f"fp8bg_part{p}.o" for p in PARTS]
            cmds = [part_command(p, o) for p, o in zip(PARTS, objs)]
            if verbose:
                print(" ".join(cmds[0]).replace("-DFP8BG_PART=1", "-DFP8BG_PART={1..7}"), flush=True)
            jobs = max(1, min(len(PARTS), os.cpu_count() or 1))
            with ThreadPoolExecutor(jobs) as pool:
                list(pool.map(lambda pc: _run(pc[1], f"compiling part {pc[0]} of {OUT.name}"),
                              zip(PARTS, cmds)))
            link = link_command(objs, tmp)
            if verbose:
                print(" ".join(link), flush=True)
            _run(link, f"linking {OUT.name}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
