"""Single-token decode step of the Mamba-2 SSM on MI355X.

``selective_state_update`` keeps the signature, shapes and semantics of the
reference's decode op
(mamba_triton_ascend/mamba2/ops/triton/selective_state_update.py:134-213):

* ``state`` (batch, dim, dstate) or (batch, nheads, dim, dstate) is updated in
  place; with ``state_batch_indices`` (batch,) the sequences map to state slots
  and a negative index marks padding (no update, output 0, lines 58-64);
* the tied head-dim case (A, dt and dt_bias broadcast over dim and dstate with
  stride 0, as Mamba-2's decoding passes them, lines 101-109 and 203) runs on
  the per-head values; otherwise A is per (head, dim, dstate) and dt, dt_bias
  per (head, dim);
* softplus applies to dt + dt_bias when ``dt_softplus`` (threshold 20, as the
  reference's kernel), out = S C (+ D x) (* silu z), returned in x's dtype.

The arithmetic runs in fp32 in the HIP kernel behind the C ABI entry point
``mamba2_selective_state_update`` (include/mamba2_ssd.h); ``state`` itself must
be float32 with each slot a contiguous [nheads, dim, dstate] block, since it is
updated where it lies.  The other float32 inputs go to the kernel as they are,
with their strides (broadcast views included); only other dtypes, a
non-contiguous innermost dimension of x, z, B, C, or B / C rows off 16-byte
alignment are copied first.  There is no CPU path.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _runtime as rt


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float32)


def _rows(t: torch.Tensor) -> torch.Tensor:
    """float32 with a contiguous innermost dimension."""
    t = t.to(torch.float32)
    return t if t.stride(-1) == 1 else t.contiguous()


def _aligned_rows(t: torch.Tensor) -> bool:
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(st % 4 == 0 for st in t.stride()[:-1]))


def selective_state_update(state: torch.Tensor, x: torch.Tensor, dt: torch.Tensor,
                           A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                           D: Optional[torch.Tensor] = None, z: Optional[torch.Tensor] = None,
                           dt_bias: Optional[torch.Tensor] = None, dt_softplus: bool = False,
                           state_batch_indices: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One decode step (see the module docstring); returns out (batch, [nheads,] dim)."""
    call = prepare_state_update(state, x, dt, A, B, C, D=D, z=z, dt_bias=dt_bias,
                                dt_softplus=dt_softplus, state_batch_indices=state_batch_indices)
    return call()


def prepare_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False,
                         state_batch_indices=None):
    """Validate and lay out the arguments of one decode step once; the
    returned callable enqueues the step on the current stream and returns
    ``out`` (calling it again repeats the step on the same tensors)."""
    has_heads = state.dim() > 3
    if state.dim() == 3:
        state = state.unsqueeze(1)
    if x.dim() == 2:
        x = x.unsqueeze(1)
    if dt.dim() == 2:
        dt = dt.unsqueeze(1)
    if A.dim() == 2:
        A = A.unsqueeze(0)
    if B.dim() == 2:
        B = B.unsqueeze(1)
    if C.dim() == 2:
        C = C.unsqueeze(1)
    if D is not None and D.dim() == 1:
        D = D.unsqueeze(0)
    if z is not None and z.dim() == 2:
        z = z.unsqueeze(1)
    if dt_bias is not None and dt_bias.dim() == 1:
        dt_bias = dt_bias.unsqueeze(0)
    _, nheads, dim, dstate = state.shape
    batch = x.shape[0]
    if x.shape != (batch, nheads, dim):
        raise ValueError(f"selective_state_update: x must be {(batch, nheads, dim)}, got {tuple(x.shape)}")
    if dt.shape != x.shape:
        raise ValueError("selective_state_update: dt must have x's shape")
    if A.shape != (nheads, dim, dstate):
        raise ValueError(f"selective_state_update: A must be {(nheads, dim, dstate)}")
    ngroups = B.shape[1]
    if nheads % ngroups:
        raise ValueError("selective_state_update: nheads must be divisible by ngroups")
    if B.shape != (batch, ngroups, dstate) or C.shape != B.shape:
        raise ValueError(f"selective_state_update: B and C must be {(batch, ngroups, dstate)}")
    if D is not None and D.shape != (nheads, dim):
        raise ValueError(f"selective_state_update: D must be {(nheads, dim)}")
    if z is not None and z.shape != x.shape:
        raise ValueError("selective_state_update: z must have x's shape")
    if dt_bias is not None and dt_bias.shape != (nheads, dim):
        raise ValueError(f"selective_state_update: dt_bias must be {(nheads, dim)}")
    if state_batch_indices is not None and state_batch_indices.shape != (batch,):
        raise ValueError(f"selective_state_update: state_batch_indices must be {(batch,)}")

    tensors = [state, x, dt, A, B, C] + [t for t in (D, z, dt_bias, state_batch_indices) if t is not None]
    if any(t.device.type != "cuda" for t in tensors):
        raise RuntimeError("selective_state_update: every tensor must be on the ROCm GPU")
    if state.dtype != torch.float32:
        raise RuntimeError("selective_state_update: state must be float32 (it is updated in place)")
    if state.stride(3) != 1 or state.stride(2) != dstate or state.stride(1) != dim * dstate:
        raise RuntimeError("selective_state_update: each state slot must be a contiguous "
                           "[nheads, dim, dstate] block")

    tied = (A.stride(-1) == 0 and A.stride(-2) == 0 and dt.stride(-1) == 0
            and (dt_bias is None or dt_bias.stride(-1) == 0))
    flags = rt.SSU_STRIDES | (rt.DT_SOFTPLUS if dt_softplus else 0) | (rt.SSU_TIED if tied else 0)
    dt_k, A_k = _f32(dt), _f32(A)
    bias_k = None if dt_bias is None else _f32(dt_bias)
    if not tied and A_k.stride(-1) == 1 and (A_k.data_ptr() % 16 or A_k.stride(0) % 4 or A_k.stride(1) % 4):
        A_k = A_k.clone(memory_format=torch.contiguous_format)  # 16-byte rows for the kernel
    x_k = _rows(x)
    z_k = None if z is None else _rows(z)
    B_k, C_k = _f32(B), _f32(C)
    if not (_aligned_rows(B_k) and _aligned_rows(C_k) and B_k.stride() == C_k.stride()):
        B_k, C_k = B_k.contiguous(), C_k.contiguous()
    # D broadcast over dim (Mamba-2's repeat "h -> h p") is read per head
    d_per_channel = D is not None and D.stride(-1) != 0
    D_k = None if D is None else _f32(D)
    idx = None if state_batch_indices is None else state_batch_indices.to(torch.int32).contiguous()
    if D_k is not None:
        flags |= rt.HAS_D | (rt.D_PER_CHANNEL if d_per_channel else 0)
    if z_k is not None:
        flags |= rt.HAS_Z
    if bias_k is not None:
        flags |= rt.HAS_DT_BIAS
    out = torch.empty(batch, nheads, dim, device=x.device, dtype=torch.float32)

    st = rt.Mamba2SsuStrides()
    st.x_b, st.x_h = x_k.stride(0), x_k.stride(1)
    if z_k is not None:
        st.z_b, st.z_h = z_k.stride(0), z_k.stride(1)
    st.bc_b, st.bc_g = B_k.stride(0), B_k.stride(1)
    st.dt_b, st.dt_h, st.dt_p = dt_k.stride(0), dt_k.stride(1), dt_k.stride(2)
    st.A_h, st.A_p, st.A_n = A_k.stride(0), A_k.stride(1), A_k.stride(2)
    if bias_k is not None:
        st.bias_h, st.bias_p = bias_k.stride(0), bias_k.stride(1)
    if D_k is not None:
        st.D_h, st.D_p = D_k.stride(0), D_k.stride(1)

    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    args = rt.Mamba2SsuArgs(batch, nheads, dim, dstate, ngroups, flags,
                            P(state), state.shape[0], state.stride(0), P(idx),
                            P(x_k), P(dt_k), P(A_k), P(B_k), P(C_k), P(D_k), P(z_k), P(bias_k), P(out),
                            st)
    lib = rt.load_library()

    def launch() -> torch.Tensor:
        stream = ctypes.c_void_p(torch.cuda.current_stream(out.device).cuda_stream)
        with torch.cuda.device(out.device):
            rt.check(lib.mamba2_selective_state_update(ctypes.byref(args), stream),
                     "mamba2_selective_state_update", lib)
        res = out.to(x.dtype)
        return res if has_heads else res.squeeze(1)

    # the tensors args points at live as long as the callable
    launch.tensors = (state, x_k, dt_k, A_k, B_k, C_k, D_k, z_k, bias_k, idx, out)
    return launch
