"""Loaders of the HIP library ``libmamba2_ssd.so`` (ctypes binding) and of
the torch operator library ``libmamba2_ssd_torch.so``.

Mirrors the role of the reference's runtime loader
(mamba_ascendc/python/ascend_kernel/ascend_kernel/_runtime.py:35-65), which
dlopens the operator library once at import.  Here the HIP library is the C ABI
of include/mamba2_ssd.h (the structures below are its ctypes mirror), and the
operator library registers ``torch.ops.mamba_ascend.*`` in C++ over that ABI.
There is no fallback: if either library is missing or fails to load, import
raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBRARY_NAME = "libmamba2_ssd.so"
LIBRARY_PATH = os.environ.get("MAMBA2_SSD_LIBRARY", os.path.join(_PKG_ROOT, LIBRARY_NAME))
TORCH_OPS_PATH = os.path.join(_PKG_ROOT, "libmamba2_ssd_torch.so")

ABI_VERSION = 5

DT_SOFTPLUS = 1 << 0
HAS_D = 1 << 1
D_PER_CHANNEL = 1 << 2
HAS_Z = 1 << 3
HAS_DT_BIAS = 1 << 4
HAS_INITIAL = 1 << 5
SAVED_STATES = 1 << 6
HAS_SEQ_IDX = 1 << 7
VARLEN_STATES = 1 << 8
SSU_TIED = 1 << 16
SSU_STRIDES = 1 << 17

# static device scratch of mamba2_ssd_fwd_noalloc (MAMBA2_SSD_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 40 << 20

STATUS_NAMES = {
    0: "OK",
    -1: "INVALID_ARGUMENT",
    -2: "UNSUPPORTED",
    -3: "WORKSPACE",
    -4: "LAUNCH",
}

_c_fp = ctypes.c_void_p


class Mamba2SsdShape(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("nheads", ctypes.c_int64),
        ("headdim", ctypes.c_int64),
        ("ngroups", ctypes.c_int64),
        ("dstate", ctypes.c_int64),
        ("chunk_size", ctypes.c_int64),
    ]


class Mamba2SsdFwdArgs(ctypes.Structure):
    _fields_ = [
        ("shape", Mamba2SsdShape),
        ("flags", ctypes.c_uint32),
        ("dt_limit_min", ctypes.c_float),
        ("dt_limit_max", ctypes.c_float),
        ("x", _c_fp), ("dt", _c_fp), ("A", _c_fp), ("B", _c_fp), ("C", _c_fp),
        ("D", _c_fp), ("z", _c_fp), ("dt_bias", _c_fp), ("initial_states", _c_fp),
        ("out", _c_fp),
        ("final_state", _c_fp),
        ("pre_gate", _c_fp),
        ("chunk_states", _c_fp),
        ("seq_idx", _c_fp),
        ("cu_seqlens", _c_fp),
        ("nseqs", ctypes.c_int64),
        ("varlen_states", _c_fp),
    ]


class Mamba2SsdBwdArgs(ctypes.Structure):
    _fields_ = [
        ("shape", Mamba2SsdShape),
        ("flags", ctypes.c_uint32),
        ("dt_limit_min", ctypes.c_float),
        ("dt_limit_max", ctypes.c_float),
        ("x", _c_fp), ("dt", _c_fp), ("A", _c_fp), ("B", _c_fp), ("C", _c_fp),
        ("D", _c_fp), ("z", _c_fp), ("dt_bias", _c_fp), ("initial_states", _c_fp),
        ("dout", _c_fp), ("dfinal_state", _c_fp), ("pre_gate", _c_fp), ("chunk_states", _c_fp),
        ("dx", _c_fp), ("ddt", _c_fp), ("dA", _c_fp), ("dB", _c_fp), ("dC", _c_fp),
        ("dD", _c_fp), ("dz", _c_fp), ("ddt_bias", _c_fp), ("dinitial_states", _c_fp),
        ("seq_idx", _c_fp),
    ]


class Mamba2SsuStrides(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in
                ("x_b", "x_h", "z_b", "z_h", "bc_b", "bc_g", "dt_b", "dt_h", "dt_p",
                 "A_h", "A_p", "A_n", "bias_h", "bias_p", "D_h", "D_p")]


class Mamba2SsuArgs(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64), ("nheads", ctypes.c_int64), ("headdim", ctypes.c_int64),
        ("dstate", ctypes.c_int64), ("ngroups", ctypes.c_int64),
        ("flags", ctypes.c_uint32),
        ("state", _c_fp), ("state_slots", ctypes.c_int64), ("state_slot_stride", ctypes.c_int64),
        ("state_batch_indices", _c_fp),
        ("x", _c_fp), ("dt", _c_fp), ("A", _c_fp), ("B", _c_fp), ("C", _c_fp),
        ("D", _c_fp), ("z", _c_fp), ("dt_bias", _c_fp),
        ("out", _c_fp),
        ("strides", Mamba2SsuStrides),
    ]


# Every symbol include/mamba2_ssd.h declares, with its ctypes signature.
EXPORTS = {
    "mamba2_ssd_abi_version": ([], ctypes.c_int),
    "mamba2_ssd_last_error": ([], ctypes.c_char_p),
    "mamba2_ssd_fwd_workspace_size": (
        [ctypes.POINTER(Mamba2SsdShape), ctypes.c_uint32, ctypes.POINTER(ctypes.c_size_t)],
        ctypes.c_int,
    ),
    "mamba2_ssd_fwd": (
        [ctypes.POINTER(Mamba2SsdFwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "mamba2_ssd_fwd_traced": (
        [ctypes.POINTER(Mamba2SsdFwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
         ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
         ctypes.POINTER(ctypes.c_int)],
        ctypes.c_int,
    ),
    "mamba2_ssd_fwd_noalloc": (
        [ctypes.POINTER(Mamba2SsdFwdArgs), ctypes.c_void_p],
        ctypes.c_int,
    ),
    "mamba2_ssd_bwd_m1_workspace_size": (
        [ctypes.POINTER(Mamba2SsdShape), ctypes.c_uint32, ctypes.POINTER(ctypes.c_size_t)],
        ctypes.c_int,
    ),
    "mamba2_ssd_bwd_m1": (
        [ctypes.POINTER(Mamba2SsdBwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
        ctypes.c_int,
    ),
    "mamba2_ssd_bwd_m1_traced": (
        [ctypes.POINTER(Mamba2SsdBwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
         ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
         ctypes.POINTER(ctypes.c_int)],
        ctypes.c_int,
    ),
    "mamba2_ssd_state_passing": (
        [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 5 + [ctypes.c_void_p],
        ctypes.c_int,
    ),
    "mamba2_ssd_state_passing_f16": (
        [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 5 + [ctypes.c_void_p],
        ctypes.c_int,
    ),
    "mamba2_selective_state_update": (
        [ctypes.POINTER(Mamba2SsuArgs), ctypes.c_void_p],
        ctypes.c_int,
    ),
}

_lock = threading.Lock()
_lib = None


def load_library(path: str | None = None):
    """Load (once) and return the ctypes handle of the HIP library.

    Loading does not touch the GPU, so it also works on a CPU-only host.
    Raises RuntimeError when the library is missing or its ABI differs.
    """
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIBRARY_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"HIP library {p} not found; build it with `python -c \"import __graft_entry__ as g; g.build()\"` "
                "or `python mamba-ascendc_amd/build.py`"
            )
        lib = ctypes.CDLL(p, mode=ctypes.RTLD_LOCAL)
        for name, (argtypes, restype) in EXPORTS.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        version = lib.mamba2_ssd_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{p}: ABI version {version}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


_torch_ops_loaded = False


def load_torch_ops() -> None:
    """Load (once) the torch operator library, which registers
    ``torch.ops.mamba_ascend.*`` (no GPU work).  Raises RuntimeError when it is
    missing."""
    global _torch_ops_loaded
    with _lock:
        if _torch_ops_loaded:
            return
        if not os.path.exists(TORCH_OPS_PATH):
            raise RuntimeError(
                f"torch operator library {TORCH_OPS_PATH} not found; build it with "
                "`python -c \"import __graft_entry__ as g; g.build()\"`"
            )
        import torch

        torch.ops.load_library(TORCH_OPS_PATH)
        _torch_ops_loaded = True


def last_error(lib=None) -> str:
    lib = lib or load_library()
    msg = lib.mamba2_ssd_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str, lib=None) -> None:
    """Turn a nonzero C status into RuntimeError (the TORCH_CHECK of the reference)."""
    if status != 0:
        name = STATUS_NAMES.get(status, str(status))
        raise RuntimeError(f"{what}: {name}: {last_error(lib)}")
