"""ctypes wrapper of the float64 C recurrence in ``oracle/ssd_seq.c`` (test-only).

``seq_fwd`` and ``seq_bwd`` take torch CPU tensors in the public layouts,
convert them to contiguous float64 and return float64 results.  The library
is built by ``oracle/Makefile`` (``make -C oracle``).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libssd_seq.so")
        if not os.path.exists(path):
            subprocess.run(["make", "-C", _HERE, "-s"], check=True)
        lib = ctypes.CDLL(path)
        L, I, D, P = ctypes.c_long, ctypes.c_int, ctypes.c_double, ctypes.c_void_p
        lib.ssd_seq_fwd.argtypes = [L] * 6 + [I, D, D, I] + [P] * 11
        lib.ssd_seq_fwd.restype = I
        lib.ssd_seq_bwd.argtypes = [L] * 6 + [I, D, D, I] + [P] * 20
        lib.ssd_seq_bwd.restype = I
        _LIB = lib
    return _LIB


def _d(t):
    return None if t is None else t.detach().to(torch.float64).contiguous()


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _d_mode(D):
    return 0 if D is None else (1 if D.dim() == 1 else 2)


def seq_fwd(x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False,
            dt_limit=(0.0, float("inf")), initial_states=None):
    """Float64 forward: returns (out [b,l,h,p], final [b,h,p,n])."""
    b, l, h, p = x.shape
    g, n = B.shape[2], B.shape[3]
    ins = [_d(v) for v in (x, dt, A, B, C, D, z, dt_bias, initial_states)]
    out = torch.empty(b, l, h, p, dtype=torch.float64)
    fin = torch.empty(b, h, p, n, dtype=torch.float64)
    rc = _lib().ssd_seq_fwd(b, l, h, p, g, n, int(bool(dt_softplus)), float(dt_limit[0]),
                            float(dt_limit[1]), _d_mode(D), *[_ptr(v) for v in ins],
                            _ptr(out), _ptr(fin))
    if rc != 0:
        raise RuntimeError(f"ssd_seq_fwd failed rc={rc}")
    return out, fin


def seq_bwd(x, dt, A, B, C, dout, dfinal=None, D=None, z=None, dt_bias=None,
            dt_softplus=False, dt_limit=(0.0, float("inf")), initial_states=None):
    """Float64 adjoint backward.  Returns a dict of gradients (None when absent)."""
    b, l, h, p = x.shape
    g, n = B.shape[2], B.shape[3]
    ins = [_d(v) for v in (x, dt, A, B, C, D, z, dt_bias, initial_states, dout, dfinal)]
    z64 = lambda *s: torch.zeros(*s, dtype=torch.float64)  # noqa: E731
    grads = {
        "dx": z64(b, l, h, p), "ddt": z64(b, l, h), "dA": z64(h),
        "dB": z64(b, l, g, n), "dC": z64(b, l, g, n),
        "dD": None if D is None else z64(*D.shape),
        "dz": None if z is None else z64(b, l, h, p),
        "ddt_bias": None if dt_bias is None else z64(h),
        "dinitial": None if initial_states is None else z64(b, h, p, n),
    }
    order = ["dx", "ddt", "dA", "dB", "dC", "dD", "dz", "ddt_bias", "dinitial"]
    rc = _lib().ssd_seq_bwd(b, l, h, p, g, n, int(bool(dt_softplus)), float(dt_limit[0]),
                            float(dt_limit[1]), _d_mode(D), *[_ptr(v) for v in ins],
                            *[_ptr(grads[k]) for k in order])
    if rc != 0:
        raise RuntimeError(f"ssd_seq_bwd failed rc={rc}")
    return grads
