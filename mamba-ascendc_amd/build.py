"""Build the HIP library libmamba2_ssd.so in-tree for gfx950, and the torch
operator library libmamba2_ssd_torch.so (torch.ops.mamba_ascend.* in C++ over
the first one's C ABI).

Usage: python mamba-ascendc_amd/build.py   (or __graft_entry__.build()).
hipcc cross-compiles without a GPU, so this runs on CPU-only hosts too.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libmamba2_ssd.so")
OUT_TORCH = os.path.join(HERE, "libmamba2_ssd_torch.so")
ROCM_INCLUDE = "/opt/rocm/include"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MAMBA2_SSD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU ops stay off (code generation choice for this target)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results go to ordinary VGPRs: no v_accvgpr_read/write shuffles
    # between the matrix products and the fp32 epilogue math
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
]


# translation units (source, extra flags): the host code with the small
# kernels, the fused-forward variants (dstate 64 and dstate 128), and the
# backward variants with and without the z gate; compiled in parallel, then
# linked into one library
UNITS = [
    ("mamba2_ssd.hip", []),
    ("ssd_fwd_seg.hip", []),
    ("ssd_fwd_wide.hip", []),
    ("ssd_bwd_ws.hip", ["-DSSD_BWD_Z=0"]),
    ("ssd_bwd_ws.hip", ["-DSSD_BWD_Z=1"]),
]

_NOISE = "is not a recognized feature for this target"


def _messages(res) -> str:
    return "\n".join(l for l in (res.stdout + res.stderr).splitlines() if _NOISE not in l)


def _torch_flags():
    """Host compile and link flags of the torch operator library (this
    interpreter's torch: its headers, libraries and C++ ABI)."""
    import torch
    from torch.utils import cpp_extension

    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    libdir = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-x", "c++", "-O2", "-std=c++17", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM=1",
              "-D__HIP_PLATFORM_AMD__=1", f"-I{ROCM_INCLUDE}", *inc]
    lflags = [f"-L{libdir}", f"-Wl,-rpath,{libdir}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
              "-ltorch_hip"]
    return cflags, lflags


def build(verbose: bool = False) -> str:
    work = tempfile.mkdtemp(prefix="mamba2_ssd_build_")
    try:
        jobs, objs = [], []
        # the torch operator unit compiles beside the HIP units and links
        # against the HIP library once that exists
        tcflags, tlflags = _torch_flags()
        tobj = os.path.join(work, "torch_ops.o")
        tcmd = [HIPCC, *tcflags, "-c", "-o", tobj, os.path.join(CSRC, "torch_ops.cpp")]
        tjob = (tcmd, subprocess.Popen(tcmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
        for i, (src, extra) in enumerate(UNITS):
            obj = os.path.join(work, f"u{i}.o")
            cmd = [HIPCC, *FLAGS, *extra, "-c", "-o", obj, os.path.join(CSRC, src)]
            jobs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                               text=True)))
            objs.append(obj)
        failed = []
        for cmd, proc in jobs + [tjob]:
            out, err = proc.communicate()
            res = subprocess.CompletedProcess(cmd, proc.returncode, out, err)
            msgs = _messages(res)
            if res.returncode != 0:
                failed.append(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{msgs}")
            elif verbose and msgs.strip():
                print(msgs, file=sys.stderr)
        if failed:
            raise RuntimeError("\n\n".join(failed))
        tmp = OUT + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-fPIC", "-shared", "-o", tmp, *objs]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{' '.join(cmd)}\n{_messages(res)}")
        os.replace(tmp, OUT)
        ttmp = OUT_TORCH + ".tmp"
        cmd = [HIPCC, "-fPIC", "-shared", "-o", ttmp, tobj, f"-L{os.path.dirname(OUT)}",
               f"-l:{os.path.basename(OUT)}", "-Wl,-rpath,$ORIGIN", *tlflags]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link failed ({res.returncode}):\n{' '.join(cmd)}\n{_messages(res)}")
        os.replace(ttmp, OUT_TORCH)
    finally:
        shutil.rmtree(work, ignore_errors=True)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
