"""PyTorch-facing Mamba-2 SSD API on MI355X.

Public surface mirrors mamba_ascendc/python/ascend_kernel/ascend_kernel/mamba2.py:

* ``mamba2_ssd_fwd`` / ``mamba_chunk_scan_combined`` (mamba2.py:1923-2020): same
  signature, same return convention (``out`` or ``(out, final_state)``), same
  autograd contract (gradients for x, dt, A, B, C, D, z, dt_bias and
  initial_states in forward-argument order, mamba2.py:1824-1838), same error
  types (RuntimeError for bad tensors, NotImplementedError for an unsupported
  training spec, mamba2.py:1978-1982).
* ``torch.ops.mamba_ascend.mamba2_ssd_fwd`` / ``mamba2_ssd_bwd_m1`` /
  ``mamba2_ssd_state_passing``: op schemas of mamba_ascendc/csrc/register.cpp
  (forward 175-179, state passing 89-90), registered in C++ by the operator
  library (csrc/torch_ops.cpp) on the CUDA key (ROCm tensors are
  ``device.type == "cuda"``), CPU (rejected) and Meta.

The public calls go through those C++ operators, which validate, allocate
outputs and workspace from torch's caching allocator and enqueue the HIP
library's kernels on the current stream; packed-sequence calls (seq_idx,
cu_seqlens) use the ctypes binding of the same C ABI below.  A nonzero status
becomes RuntimeError.  There is no CPU path: CPU tensors are rejected.
"""

from __future__ import annotations

import contextlib
import contextvars
import ctypes
import dataclasses
import math
import threading
from typing import Iterator, Optional, Tuple, Union

import torch

from . import _runtime as rt



# ----------------------------------------------------------------------------- validation

def _check_tensor(op: str, name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{op}: {name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{op}: {name} must be a ROCm GPU tensor (got device {t.device})")
    if t.dtype != torch.float32:
        raise RuntimeError(f"{op}: {name} must be float32 (got {t.dtype})")
    if not t.is_contiguous():
        raise RuntimeError(f"{op}: {name} must be contiguous")


def _validate_fwd(op, x, dt, A, B, C, chunk_size, D, z, dt_bias, initial_states,
                  dt_limit_min, dt_limit_max):
    """Checks of the reference host wrapper
    (mamba_ascendc/csrc/ops/mamba2_ssd_fwd/op_host/mamba2_ssd_fwd.cpp:15-113)."""
    for name, t in (("x", x), ("dt", dt), ("A", A), ("B", B), ("C", C)):
        _check_tensor(op, name, t)
    for name, t in (("D", D), ("z", z), ("dt_bias", dt_bias), ("initial_states", initial_states)):
        if t is not None:
            _check_tensor(op, name, t)
    if x.dim() != 4:
        raise RuntimeError(f"{op}: x must have shape [B,L,H,P]")
    if dt.dim() != 3:
        raise RuntimeError(f"{op}: dt must have shape [B,L,H]")
    if A.dim() != 1:
        raise RuntimeError(f"{op}: A must have shape [H]")
    if B.dim() != 4 or C.dim() != 4:
        raise RuntimeError(f"{op}: B and C must have shape [B,L,G,N]")
    batch, seqlen, nheads, headdim = x.shape
    ngroups, dstate = B.shape[2], B.shape[3]
    if min(batch, seqlen, nheads, headdim) <= 0:
        raise RuntimeError(f"{op}: zero-sized dimensions are not supported")
    if dstate <= 0 or ngroups <= 0:
        raise RuntimeError(f"{op}: dstate and ngroups must be positive")
    if tuple(dt.shape) != (batch, seqlen, nheads):
        raise RuntimeError(f"{op}: dt shape must equal [B,L,H]")
    if A.shape[0] != nheads:
        raise RuntimeError(f"{op}: A shape must equal [H]")
    if B.shape != C.shape:
        raise RuntimeError(f"{op}: B and C shapes must match")
    if B.shape[0] != batch or B.shape[1] != seqlen:
        raise RuntimeError(f"{op}: B/C batch and sequence dimensions must match x")
    if nheads % ngroups:
        raise RuntimeError(f"{op}: nheads must be divisible by ngroups")
    if int(chunk_size) <= 0:
        raise RuntimeError(f"{op}: chunk_size must be positive")
    if not float(dt_limit_min) <= float(dt_limit_max):
        raise RuntimeError(f"{op}: dt_limit_min must not exceed dt_limit_max")
    if D is not None:
        if not ((D.dim() == 1 and D.shape[0] == nheads)
                or (D.dim() == 2 and tuple(D.shape) == (nheads, headdim))):
            raise RuntimeError(f"{op}: D must have shape [H] or [H,P]")
    if z is not None and z.shape != x.shape:
        raise RuntimeError(f"{op}: z shape must match x")
    if dt_bias is not None and tuple(dt_bias.shape) != (nheads,):
        raise RuntimeError(f"{op}: dt_bias shape must equal [H]")
    if initial_states is not None and tuple(initial_states.shape) != (batch, nheads, headdim, dstate):
        raise RuntimeError(f"{op}: initial_states must have shape [B,H,P,N]")
    devices = {t.device for t in (x, dt, A, B, C, D, z, dt_bias, initial_states) if t is not None}
    if len(devices) != 1:
        raise RuntimeError(f"{op}: all tensors must be on the same device")


def _packed_shape_ok(x, B) -> bool:
    return x.shape[-1] % 64 == 0 and B.shape[-1] in (64, 128)


def _check_seq_idx(x, seq_idx, chunk_size, B) -> Optional[torch.Tensor]:
    """seq_idx [B, L] of any integer dtype on x's device -> int32 contiguous."""
    if seq_idx is None:
        return None
    if not isinstance(seq_idx, torch.Tensor) or seq_idx.dtype.is_floating_point or seq_idx.is_complex():
        raise RuntimeError("mamba2_ssd_fwd: seq_idx must be an integer tensor")
    if tuple(seq_idx.shape) != tuple(x.shape[:2]):
        raise RuntimeError(f"mamba2_ssd_fwd: seq_idx must have shape {tuple(x.shape[:2])}")
    if seq_idx.device != x.device:
        raise RuntimeError("mamba2_ssd_fwd: seq_idx must be on x's device")
    if not _packed_shape_ok(x, B):
        raise NotImplementedError("mamba2_ssd_fwd: seq_idx needs a headdim that is a multiple of 64 "
                                  "with dstate 64 or 128")
    return seq_idx.to(torch.int32).contiguous()


def _check_cu_seqlens(x, cu_seqlens, chunk_size, B) -> torch.Tensor:
    """cu_seqlens [nseq + 1] of any integer dtype on x's device -> int32 contiguous."""
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dtype.is_floating_point:
        raise RuntimeError("mamba2_ssd_fwd: cu_seqlens must be an integer tensor")
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise RuntimeError("mamba2_ssd_fwd: cu_seqlens must be 1-D with at least 2 entries")
    if cu_seqlens.device != x.device:
        raise RuntimeError("mamba2_ssd_fwd: cu_seqlens must be on x's device")
    if x.shape[0] != 1:
        raise RuntimeError("mamba2_ssd_fwd: varlen states need batch 1")
    if x.shape[-1] != 64 or B.shape[-1] not in (64, 128) or int(chunk_size) % 64:
        raise NotImplementedError("mamba2_ssd_fwd: varlen states need headdim 64, dstate 64 or "
                                  "128 and a chunk_size that is a multiple of 64")
    return cu_seqlens.to(torch.int32).contiguous()


def _flags(D, z, dt_bias, initial_states, dt_softplus) -> int:
    f = 0
    if dt_softplus:
        f |= rt.DT_SOFTPLUS
    if D is not None:
        f |= rt.HAS_D
        if D.dim() == 2:
            f |= rt.D_PER_CHANNEL
    if z is not None:
        f |= rt.HAS_Z
    if dt_bias is not None:
        f |= rt.HAS_DT_BIAS
    if initial_states is not None:
        f |= rt.HAS_INITIAL
    return f


def _shape(x, B, chunk_size) -> rt.Mamba2SsdShape:
    b, l, h, p = x.shape
    return rt.Mamba2SsdShape(b, l, h, p, B.shape[2], B.shape[3], int(chunk_size))


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _limit(v: float) -> float:
    # the schema default 3.402823466e+38 (FLT_MAX) and +inf both mean "no upper clamp"
    v = float(v)
    return math.inf if v >= 3.4e38 else v


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


# ----------------------------------------------------------------------------- raw calls

def _nchunks(x) -> int:
    return (x.shape[1] + 63) // 64


def _fwd_raw(x, dt, A, B, C, D, z, dt_bias, initial_states, chunk_size, dt_softplus,
             dt_limit_min, dt_limit_max, want_final=True, want_pre_gate=False,
             want_states=False, seq_idx=None, cu_seqlens=None):
    """Returns (out, final_state or None, pre_gate or None, chunk_states or None,
    varlen_states or None); pre_gate (y + D x before the z gate) is produced
    only when z is given and it is asked for; chunk_states [B, H, ceil(L/64),
    P, N] (the state entering each 64-token chunk, for the backward) only when
    asked for; varlen_states [nseq, H, P, N] when ``cu_seqlens`` (int32,
    validated) is given.  ``seq_idx`` is an int32 [B, L] tensor or None."""
    lib = rt.load_library()
    shape = _shape(x, B, chunk_size)
    flags = _flags(D, z, dt_bias, initial_states, dt_softplus)
    if want_states:
        flags |= rt.SAVED_STATES
    if seq_idx is not None:
        flags |= rt.HAS_SEQ_IDX
    if cu_seqlens is not None:
        flags |= rt.VARLEN_STATES
    nbytes = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(shape), flags, ctypes.byref(nbytes)),
             "mamba2_ssd_fwd_workspace_size", lib)
    out = torch.empty_like(x)
    b, _, h, p = x.shape
    final = torch.empty(b, h, p, B.shape[3], device=x.device, dtype=torch.float32) if want_final else None
    pre_gate = torch.empty_like(x) if (want_pre_gate and z is not None) else None
    states = (torch.empty(b, h, _nchunks(x), p, B.shape[3], device=x.device, dtype=torch.float32)
              if want_states else None)
    nseqs = 0 if cu_seqlens is None else cu_seqlens.numel() - 1
    varlen = (torch.empty(nseqs, h, p, B.shape[3], device=x.device, dtype=torch.float32)
              if cu_seqlens is not None else None)
    ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=x.device)
    args = rt.Mamba2SsdFwdArgs(
        shape, flags, float(dt_limit_min), _limit(dt_limit_max),
        _ptr(x), _ptr(dt), _ptr(A), _ptr(B), _ptr(C),
        _ptr(D), _ptr(z), _ptr(dt_bias), _ptr(initial_states),
        _ptr(out), _ptr(final), _ptr(pre_gate), _ptr(states),
        _ptr(seq_idx), _ptr(cu_seqlens), nseqs, _ptr(varlen),
    )
    with torch.cuda.device(x.device):
        rt.check(lib.mamba2_ssd_fwd(ctypes.byref(args), _ptr(ws), ws.numel(), _stream(x.device)),
                 "mamba2_ssd_fwd", lib)
    return out, final, pre_gate, states, varlen


def _bwd_raw(x, dt, A, B, C, dout, dfinal_state, D, z, dt_bias, initial_states, chunk_size,
             dt_softplus, dt_limit_min, dt_limit_max, pre_gate=None, chunk_states=None,
             seq_idx=None):
    lib = rt.load_library()
    shape = _shape(x, B, chunk_size)
    flags = _flags(D, z, dt_bias, initial_states, dt_softplus)
    if chunk_states is not None:
        flags |= rt.SAVED_STATES
    if seq_idx is not None:
        flags |= rt.HAS_SEQ_IDX
    nbytes = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_bwd_m1_workspace_size(ctypes.byref(shape), flags, ctypes.byref(nbytes)),
             "mamba2_ssd_bwd_m1_workspace_size", lib)
    dx = torch.empty_like(x)
    ddt = torch.empty_like(dt)
    dA = torch.empty_like(A)
    dB = torch.empty_like(B)
    dC = torch.empty_like(C)
    dD = torch.empty_like(D) if D is not None else None
    dz = torch.empty_like(z) if z is not None else None
    ddt_bias = torch.empty_like(dt_bias) if dt_bias is not None else None
    dinit = torch.empty_like(initial_states) if initial_states is not None else None
    ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=x.device)
    args = rt.Mamba2SsdBwdArgs(
        shape, flags, float(dt_limit_min), _limit(dt_limit_max),
        _ptr(x), _ptr(dt), _ptr(A), _ptr(B), _ptr(C),
        _ptr(D), _ptr(z), _ptr(dt_bias), _ptr(initial_states),
        _ptr(dout), _ptr(dfinal_state), _ptr(pre_gate), _ptr(chunk_states),
        _ptr(dx), _ptr(ddt), _ptr(dA), _ptr(dB), _ptr(dC),
        _ptr(dD), _ptr(dz), _ptr(ddt_bias), _ptr(dinit), _ptr(seq_idx),
    )
    with torch.cuda.device(x.device):
        rt.check(lib.mamba2_ssd_bwd_m1(ctypes.byref(args), _ptr(ws), ws.numel(), _stream(x.device)),
                 "mamba2_ssd_bwd_m1", lib)
    return dx, ddt, dA, dB, dC, dD, dz, ddt_bias, dinit


# ----------------------------------------------------------------------------- torch ops

def register_ops() -> None:
    """Make ``torch.ops.mamba_ascend.*`` available: load (once) the C++
    operator library, which registers the reference's ``mamba2_ssd_fwd`` and
    ``mamba2_ssd_state_passing`` schemas (mamba_ascendc/csrc/register.cpp:
    175-179, 89-90), this build's ``mamba2_ssd_bwd_m1`` and the internal
    ``mamba2_ssd_fwd_ex`` (the forward with the training outputs) on the CUDA,
    CPU (rejected by the device check) and Meta keys."""
    rt.load_torch_ops()


# ----------------------------------------------------------------------------- training policy

@dataclasses.dataclass(frozen=True)
class TrainingPolicy:
    """What the training forward keeps for the M1 backward.

    ``save_chunk_states``: keep the state entering every 64-token chunk
    (B*H*ceil(L/64)*P*N fp32, 2 GiB at [8,4096,256,64,64]) from the forward to
    the backward (True, the default: the training forward writes them in the
    same pass, about +0.3 ms at that size), or let the backward recompute them
    with one extra streaming pass over x, dt and B (False: that memory is not
    held between the passes).  This is the reference's save/recompute switch for
    ``states_start`` (mamba_ascendc/python/ascend_kernel/ascend_kernel/mamba2.py:
    1682-1697, ``MAMBA_ASCENDC_SAVE_STATES_START``), as an object instead of an
    environment variable.  The gradients do not depend on the choice.
    """

    save_chunk_states: bool = True


_policy_lock = threading.Lock()
_policy = TrainingPolicy()  # the process-wide default
# the policy of an enclosing training_policy() block in this thread / context
_scoped_policy: contextvars.ContextVar = contextvars.ContextVar("mamba2_training_policy", default=None)


def get_training_policy() -> TrainingPolicy:
    """The policy new training calls in this context use: that of the
    innermost enclosing ``training_policy()`` block, else the process-wide
    default."""
    scoped = _scoped_policy.get()
    return _policy if scoped is None else scoped


def set_training_policy(policy: TrainingPolicy) -> TrainingPolicy:
    """Make ``policy`` the process-wide default for new training calls (calls
    inside a ``training_policy()`` block keep that block's policy); returns the
    old default."""
    global _policy
    if not isinstance(policy, TrainingPolicy):
        raise TypeError("set_training_policy expects a TrainingPolicy")
    with _policy_lock:
        old, _policy = _policy, policy
    return old


@contextlib.contextmanager
def training_policy(**fields) -> Iterator[TrainingPolicy]:
    """``with training_policy(save_chunk_states=False): ...`` -- the current
    policy with the given fields changed, for the calls inside the block.  The
    block's policy is held in a context variable: other threads (and asyncio
    tasks) keep theirs, and overlapping blocks in different threads cannot
    leave each other's policy behind."""
    new = dataclasses.replace(get_training_policy(), **fields)
    token = _scoped_policy.set(new)
    try:
        yield new
    finally:
        _scoped_policy.reset(token)


# ----------------------------------------------------------------------------- autograd

def _requires_grad(*values) -> bool:
    return torch.is_grad_enabled() and any(
        isinstance(v, torch.Tensor) and v.requires_grad for v in values
    )


def _can_use_native_bwd_m1(x, dt, A, B, C, chunk_size, D, z, dt_bias, initial_states) -> bool:
    """Training spec served by the M1 backward (mamba2.py:742-803): fp32
    contiguous GPU tensors with headdim == dstate == 64.  Unlike the reference,
    any chunk_size and any seqlen are accepted: the kernels run fixed 64-token
    execution chunks and the result does not depend on the logical chunk."""
    tensors = [t for t in (x, dt, A, B, C, D, z, dt_bias, initial_states) if t is not None]
    if any(t.device.type != "cuda" or t.dtype != torch.float32 or not t.is_contiguous()
           for t in tensors):
        return False
    if x.dim() != 4 or B.dim() != 4:
        return False
    return x.shape[-1] == 64 and B.shape[-1] == 64 and int(chunk_size) > 0


class _Mamba2SsdAutogradM1(torch.autograd.Function):
    """Autograd contract of mamba2.py:1661-1838: saves the inputs (and
    pre_gate with z), and the chunk-start states unless the training policy
    says to recompute them, recomputes the other forward intermediates in
    backward, returns 13 gradients (plus None for the packed-sequence arguments
    ``seq_idx`` / ``cu_seqlens``, the Triton port's extension,
    ssd_combined.py:612-637, and for ``save_states``).  The third output, the
    varlen states, is not differentiable (that port's backward rejects it)."""

    @staticmethod
    def forward(ctx, x, dt, A, B, C, chunk_size, D, z, dt_bias, dt_softplus,
                dt_limit_min, dt_limit_max, initial_states, seq_idx=None, cu_seqlens=None,
                save_states=True):
        if seq_idx is not None or cu_seqlens is not None:
            _validate_fwd("mamba2_ssd_fwd", x, dt, A, B, C, chunk_size, D, z, dt_bias,
                          initial_states, dt_limit_min, dt_limit_max)
        # (without them the C++ operator validates)
        # the pre-gate output y + D x is saved when z is present (dz needs it),
        # as the reference's Train forward does (mamba2.py:1682-1770), and the
        # chunk-start states when the policy keeps them (the reference's
        # training forward returns states_start for its backward,
        # mamba2.py:228,322,408-418); varlen states are read from them
        if seq_idx is None and cu_seqlens is None:
            out, final_state, pre_gate, states = torch.ops.mamba_ascend.mamba2_ssd_fwd_ex(
                x, dt, A, B, C, D, z, dt_bias, initial_states, int(chunk_size), bool(dt_softplus),
                float(dt_limit_min), float(dt_limit_max), True, z is not None, bool(save_states))
            pre_gate = pre_gate if z is not None else None
            states = states if save_states else None
            varlen = None
        else:
            out, final_state, pre_gate, states, varlen = _fwd_raw(
                x, dt, A, B, C, D, z, dt_bias, initial_states, int(chunk_size), bool(dt_softplus),
                float(dt_limit_min), float(dt_limit_max), want_final=True,
                want_pre_gate=z is not None, want_states=bool(save_states), seq_idx=seq_idx,
                cu_seqlens=cu_seqlens)
        empty = x.new_empty(0)
        ctx.save_for_backward(
            x, dt, A, B, C,
            D if D is not None else empty,
            z if z is not None else empty,
            dt_bias if dt_bias is not None else empty,
            initial_states if initial_states is not None else empty,
            pre_gate if pre_gate is not None else empty,
            states if states is not None else empty,
            seq_idx if seq_idx is not None else empty,
        )
        ctx.has = (D is not None, z is not None, dt_bias is not None, initial_states is not None,
                   seq_idx is not None, states is not None)
        ctx.chunk_size = int(chunk_size)
        ctx.dt_softplus = bool(dt_softplus)
        ctx.dt_limit = (float(dt_limit_min), float(dt_limit_max))
        if varlen is None:
            varlen = empty
        ctx.mark_non_differentiable(varlen)
        return out, final_state, varlen

    @staticmethod
    def backward(ctx, dout, dfinal_state, _dvarlen):
        x, dt, A, B, C, D, z, dt_bias, initial_states, pre_gate, states, seq_idx = ctx.saved_tensors
        has_D, has_z, has_bias, has_init, has_seq, has_states = ctx.has
        if dout is None:
            dout = torch.zeros_like(x)
        grads = torch.ops.mamba_ascend.mamba2_ssd_bwd_m1(
            x, dt, A, B, C, dout.contiguous(),
            None if dfinal_state is None else dfinal_state.contiguous(),
            D if has_D else None, z if has_z else None, dt_bias if has_bias else None,
            initial_states if has_init else None, pre_gate if has_z else None,
            states if has_states else None,
            ctx.chunk_size, ctx.dt_softplus, ctx.dt_limit[0], ctx.dt_limit[1],
            seq_idx if has_seq else None)
        dx, ddt, dA, dB, dC, dD, dz, ddt_bias, dinit = grads
        return (dx, ddt, dA, dB, dC, None,
                dD if has_D else None, dz if has_z else None, ddt_bias if has_bias else None,
                None, None, None, dinit if has_init else None, None, None, None)


# ----------------------------------------------------------------------------- public API

def mamba2_ssd_fwd(
    x: torch.Tensor,
    dt: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    chunk_size: int,
    D: Optional[torch.Tensor] = None,
    z: Optional[torch.Tensor] = None,
    dt_bias: Optional[torch.Tensor] = None,
    dt_softplus: bool = False,
    dt_limit: Tuple[float, float] = (0.0, float("inf")),
    initial_states: Optional[torch.Tensor] = None,
    return_final_state: bool = False,
    *,
    seq_idx: Optional[torch.Tensor] = None,
    cu_seqlens: Optional[torch.Tensor] = None,
    return_varlen_states: bool = False,
    return_final_states: Optional[bool] = None,
    save_chunk_states: Optional[bool] = None,
) -> Union[torch.Tensor, Tuple[torch.Tensor, ...]]:
    """Mamba-2 SSD forward (chunked selective scan) on MI355X.

    Shapes: x [B,L,H,P], dt [B,L,H], A [H], B/C [B,L,G,N], D [H] or [H,P],
    z [B,L,H,P], dt_bias [H], initial_states [B,H,P,N]; all fp32 contiguous
    ROCm tensors.  Returns ``out`` [B,L,H,P], plus ``final_state`` [B,H,P,N]
    when ``return_final_state``.  When any input requires grad the call goes
    through the M1 autograd function.

    Keyword-only, from the reference's Triton port
    (mamba_triton_ascend/mamba2/ops/triton/ssd_combined.py:612-659):
    ``seq_idx`` [B,L] integer sequence id per token (packed sequences);
    ``cu_seqlens`` [nseq + 1] with ``return_varlen_states`` (batch 1) appends
    the state at the end of every sequence [nseq,H,P,N], giving ``(out,
    varlen_states)`` or ``(out, final_state, varlen_states)``;
    ``return_final_states`` is that port's name for ``return_final_state``.
    Both need headdim 64 with dstate 64 or 128 (gradients: dstate 64); varlen
    states also a chunk_size that is a multiple of 64 and are not
    differentiable.

    ``save_chunk_states`` (keyword-only, training calls): keep the chunk-start
    states for the backward (True) or recompute them there (False); None takes
    the current ``TrainingPolicy`` (``set_training_policy`` /
    ``training_policy``).
    """
    register_ops()
    if return_final_states is not None:
        return_final_state = bool(return_final_states)
    lo, hi = float(dt_limit[0]), float(dt_limit[1])
    if return_varlen_states and cu_seqlens is None:
        raise ValueError("mamba2_ssd_fwd: return_varlen_states needs cu_seqlens")
    seq32 = _check_seq_idx(x, seq_idx, chunk_size, B)
    cu32 = _check_cu_seqlens(x, cu_seqlens, chunk_size, B) if return_varlen_states else None
    if _requires_grad(x, dt, A, B, C, D, z, dt_bias, initial_states):
        if not _can_use_native_bwd_m1(x, dt, A, B, C, chunk_size, D, z, dt_bias, initial_states):
            raise NotImplementedError(
                "mamba2_ssd_fwd backward requires contiguous FP32 GPU tensors with "
                "headdim == dstate == 64"
            )
        save = get_training_policy().save_chunk_states if save_chunk_states is None else bool(save_chunk_states)
        out, final_state, varlen = _Mamba2SsdAutogradM1.apply(
            x, dt, A, B, C, chunk_size, D, z, dt_bias, dt_softplus, lo, hi, initial_states,
            seq32, cu32, save)
        if cu32 is not None:
            return (out, final_state, varlen) if return_final_state else (out, varlen)
    elif seq32 is None and cu32 is None:
        # the C++ operator validates, allocates and launches (a few us of host work)
        out, final_state, _, _ = torch.ops.mamba_ascend.mamba2_ssd_fwd_ex(
            x, dt, A, B, C, D, z, dt_bias, initial_states, int(chunk_size), bool(dt_softplus), lo, hi,
            bool(return_final_state), False, False)
    else:
        _validate_fwd("mamba2_ssd_fwd", x, dt, A, B, C, chunk_size, D, z, dt_bias,
                      initial_states, lo, hi)
        out, final_state, _, _, varlen = _fwd_raw(
            x, dt, A, B, C, D, z, dt_bias, initial_states, chunk_size, dt_softplus, lo, hi,
            want_final=return_final_state, seq_idx=seq32, cu_seqlens=cu32)
        if cu32 is not None:
            return (out, final_state, varlen) if return_final_state else (out, varlen)
    if return_final_state:
        return out, final_state
    return out


mamba_chunk_scan_combined = mamba2_ssd_fwd
