"""Build the HIP library libmamba2_ssd.so in-tree for gfx950.

Usage: python mamba-ascendc_amd/build.py   (or __graft_entry__.build()).
hipcc cross-compiles without a GPU, so this runs on CPU-only hosts too.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libmamba2_ssd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MAMBA2_SSD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed fp32 VALU ops stay off (code generation choice for this target)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results go to ordinary VGPRs: no v_accvgpr_read/write shuffles
    # between the matrix products and the fp32 epilogue math
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
]


def build(verbose: bool = False) -> str:
    src = os.path.join(CSRC, "mamba2_ssd.hip")
    tmp = OUT + ".tmp"
    cmd = [HIPCC, *FLAGS, "-o", tmp, src]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
