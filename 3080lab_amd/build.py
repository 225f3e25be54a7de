"""Build libqwen355.so for gfx950 with hipcc (ahead of time, in-tree).

  python 3080lab_amd/build.py          # -> 3080lab_amd/lib/libqwen355.so
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "lib" / "libqwen355.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "--offload-arch=gfx950", "-fPIC", "-shared", "-std=c++17",
         # no packed-fp32 VALU ops (v_pk_*_f32) in device code
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # MFMA results in VGPRs: no v_accvgpr_read per result before the fp32 scaling
         "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-Wno-unused-result"]


def build(verbose: bool = False) -> Path:
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-o", str(tmp), str(CSRC / "unity.hip")]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{errs}")
    if verbose and errs.strip():
        print(errs)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
