"""CPU-side checks of the C ABI and the host logic (no GPU work).

* the library loads and exports every function include/mamba2_ssd.h declares;
* argument validation returns the documented status codes before any HIP call
  (the host checks of mamba_ascendc/csrc/ops/mamba2_ssd_fwd/op_host/mamba2_ssd_fwd.cpp:15-113);
* the Python API raises the reference's error types (RuntimeError for bad
  tensors, NotImplementedError for an unsupported training spec,
  mamba2.py:1978-1982) and the Meta implementation infers shapes.
"""

import ctypes
import math
import os
import re
import subprocess

import pytest
import torch

from ascend_kernel import _runtime as rt
from ascend_kernel import mamba2 as api

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mamba2_ssd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mamba2_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    assert "mamba2_ssd_fwd" in names and "mamba2_ssd_bwd_m1" in names
    assert set(names) == set(rt.EXPORTS), (names, sorted(rt.EXPORTS))


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", rt.LIBRARY_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mamba2_\w+)", out))
    for name in _declared_functions():
        assert name in exported, name
    lib = rt.load_library()
    assert lib.mamba2_ssd_abi_version() == rt.ABI_VERSION


def _shape(**kw):
    d = dict(batch=2, seqlen=128, nheads=4, headdim=64, ngroups=2, dstate=64, chunk_size=64)
    d.update(kw)
    return rt.Mamba2SsdShape(**d)


@pytest.mark.parametrize(
    "kw,flags,code",
    [
        (dict(), 0, 0),
        (dict(nheads=3), 0, -1),
        (dict(batch=0), 0, -1),
        (dict(chunk_size=0), 0, -1),
        (dict(dstate=-1), 0, -1),
        (dict(), rt.D_PER_CHANNEL, -1),
        (dict(), 1 << 12, -1),
        (dict(batch=70000), 0, -2),
        # 64 token rows of H*P (or G*N) floats must stay within 32-bit byte offsets
        (dict(nheads=65535, ngroups=65535, headdim=128), 0, 0),
        (dict(nheads=65535, ngroups=65535, headdim=192), 0, -2),
        (dict(nheads=65535, ngroups=65535, dstate=192), 0, -2),
    ],
)
def test_workspace_size_validation(kw, flags, code):
    lib = rt.load_library()
    nbytes = ctypes.c_size_t(123)
    rc = lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(_shape(**kw)), flags, ctypes.byref(nbytes))
    assert rc == code, rt.last_error(lib)
    if code:
        assert rt.last_error(lib)
    rc = lib.mamba2_ssd_bwd_m1_workspace_size(ctypes.byref(_shape(**kw)), flags, ctypes.byref(nbytes))
    assert rc == code


def test_workspace_size_formula():
    """Forward plan: P = 64 with N = 64 or 128 runs the fused segment-serial
    kernel, which needs no workspace when there are >= 256 (b, h, state-half)
    streams (C3) or the sequence is short, and a per-segment state buffer
    otherwise, for N = 128 too.
    The backward needs states (unless the forward's
    are passed in), per-chunk partials, and dstates only where the state
    gradients are not carried in the reverse fused chunk kernel (other than
    1, 2 or 4 heads per group); with fewer than 256 (b, g) streams the fused
    kernel's runs take a carry buffer [B, H, runs, P, N] instead."""
    lib = rt.load_library()
    nbytes = ctypes.c_size_t(0)

    def ws(fn, **kw):
        assert fn(ctypes.byref(_shape(**kw)), 0, ctypes.byref(nbytes)) == 0
        return nbytes.value

    fwd = lib.mamba2_ssd_fwd_workspace_size
    assert ws(fwd, batch=8, seqlen=4096, nheads=256, ngroups=64) == 0
    # 64 streams, 32 chunks -> 4 segments of 8 chunks, whose entering states
    # each segment folds from the state-only contributions of the segments
    # before it (short segments: pre-segments of the same 8 chunks): the 3
    # before the last segment, [B,H,3,P,N] + [B,H,3]
    got = ws(fwd, batch=4, seqlen=2048, nheads=16, ngroups=4)
    assert 4 * 16 * 3 * 64 * 64 * 4 + 4 * 16 * 3 * 4 <= got <= 4 * 16 * 3 * (64 * 64 + 1) * 4 + 2 * 256
    # N = 128: 64 (b, h) x 2 workgroups = 128 streams -> 2 segments of 16
    # chunks, 2 pre-segments before the last; nothing else with 4 heads per
    # group (each workgroup writes its channels of out itself)
    got = ws(fwd, batch=4, seqlen=2048, nheads=16, ngroups=4, dstate=128)
    seg = 4 * 16 * 2 * 64 * 128 * 4
    assert seg <= got <= seg + 2 * 256 + 4 * 16 * 2 * 4
    # with 8 heads per group C . B^T of every (b, g, chunk) [B,G,K,64,64]
    # (256 streams here: no segments)
    assert ws(fwd, batch=4, seqlen=2048, nheads=32, ngroups=4, dstate=128) == 4 * 4 * 32 * 64 * 64 * 4
    # many segments (2 streams, 64 chunks -> 32 segments of 2): no fold, all
    # 64 pre-segments of 1 chunk and the segment recurrence over them
    got = ws(fwd, batch=1, seqlen=4096, nheads=2, ngroups=1)
    assert 2 * 64 * 64 * 64 * 4 <= got <= 2 * 64 * (64 * 64 + 1) * 4 + 2 * 256
    # a short sequence is not cut (the cut would save fewer than 6 chunk
    # steps); dstate 128 with 8 heads per group keeps C . B^T of its 2 chunks
    assert ws(fwd, batch=1, seqlen=128, nheads=2, ngroups=1, dstate=128) == 0
    assert ws(fwd, batch=1, seqlen=128, nheads=8, ngroups=1, dstate=128) == 2 * 64 * 64 * 4
    assert ws(fwd, batch=1, seqlen=384, nheads=2, ngroups=1) == 0   # 6 chunks: saves 5
    assert ws(fwd, batch=1, seqlen=512, nheads=2, ngroups=1) > 0    # 8 chunks: saves 7
    # headdim 32, dstate 128 (zero-padded into the fused kernels): x and out
    # padded to [B,L,H,64], the final state to [B,H,64,128], then the fused
    # plan of the padded shape (here one segment: nothing more)
    got = ws(fwd, batch=8, seqlen=4096, nheads=64, ngroups=64, headdim=32, dstate=128)
    blh = 8 * 4096 * 64
    assert got == 2 * blh * 64 * 4 + 8 * 64 * 64 * 128 * 4
    # dstate 32: B and C padded to [B,L,G,64], the final state to [B,H,64,64]
    got = ws(fwd, batch=8, seqlen=4096, nheads=256, ngroups=64, dstate=32)
    assert got == 2 * 8 * 4096 * 64 * 64 * 4 + 8 * 256 * 64 * 64 * 4
    # one segment per stream: no segment buffers (dstate 128: C . B^T only)
    assert ws(fwd, batch=8, seqlen=4096, nheads=64, ngroups=8, dstate=128) == 8 * 8 * 64 * 64 * 64 * 4
    assert ws(fwd, batch=8, seqlen=4096, nheads=64, ngroups=8) == 0
    assert ws(fwd, seqlen=0) == 0
    # varlen states without saved states: the chunk states join the workspace
    one = _shape(batch=1, seqlen=4096, nheads=256, ngroups=64)
    assert fwd(ctypes.byref(one), rt.VARLEN_STATES, ctypes.byref(nbytes)) == 0
    with_states = nbytes.value
    assert fwd(ctypes.byref(one), rt.VARLEN_STATES | rt.SAVED_STATES, ctypes.byref(nbytes)) == 0
    assert with_states - nbytes.value == 256 * 64 * 64 * 64 * 4
    bwd = lib.mamba2_ssd_bwd_m1_workspace_size
    k = 4096 // 64
    state_buf = 8 * 256 * k * 64 * 64 * 4
    # C3: 512 (b, g) streams, 4 heads per group -> reverse fused, no dstates
    full = ws(bwd, batch=8, seqlen=4096, nheads=256, ngroups=64)
    assert state_buf <= full < 2 * state_buf
    # with the forward's chunk states passed in, the recompute buffer goes away
    assert bwd(ctypes.byref(_shape(batch=8, seqlen=4096, nheads=256, ngroups=64)), rt.SAVED_STATES,
               ctypes.byref(nbytes)) == 0
    assert full - nbytes.value == state_buf
    assert nbytes.value < state_buf // 8  # partials only
    # 8 heads per group: split path with a dstates buffer
    split = ws(bwd, batch=8, seqlen=4096, nheads=256, ngroups=32)
    assert split >= 2 * state_buf
    # 16 (b, g) streams of 32 chunks -> 16 runs of 2 chunks each: states
    # [B,H,K,P,N] + the recompute's pre-segment states [B,H,3,P,N] (segments
    # of 8 chunks, pre-segments as long) + run carries [B,H,16,P,N] +
    # partials, no dstates
    k = 2048 // 64
    states = 4 * 16 * k * 64 * 64 * 4
    segs = 4 * 16 * 3 * 64 * 64 * 4
    carries = 4 * 16 * 16 * 64 * 64 * 4
    got = ws(bwd, batch=4, seqlen=2048, nheads=16, ngroups=4)
    assert states + segs + carries <= got < states + segs + carries + states // 8
    # one run per stream when there are 256 (b, g) streams (no carries)
    assert ws(bwd, batch=4, seqlen=2048, nheads=256, ngroups=64) < 4 * 256 * k * 64 * 64 * 4 * 5 // 4


def test_fwd_rejects_null_and_flag_mismatch_without_gpu():
    lib = rt.load_library()
    args = rt.Mamba2SsdFwdArgs()
    args.shape = _shape()
    args.dt_limit_max = math.inf
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1
    assert "non-NULL" in rt.last_error(lib)
    fake = ctypes.c_void_p(0x1000)
    for name in ("x", "dt", "A", "B", "C", "out"):
        setattr(args, name, fake)
    args.flags = rt.HAS_D  # flag without pointer
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1
    assert "HAS_D" in rt.last_error(lib)
    args.flags = 0
    args.dt_limit_min, args.dt_limit_max = 1.0, 0.5
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1
    args.dt_limit_min, args.dt_limit_max = 0.0, math.inf
    args.flags = rt.SAVED_STATES  # flag without the chunk_states pointer
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1
    assert "SAVED_STATES" in rt.last_error(lib)
    args.chunk_states = fake
    args.shape = _shape(dstate=32)  # chunk states are saved by the fused kernel only
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -2
    args.shape, args.flags, args.chunk_states = _shape(), 0, None
    # packed sequences: flag and pointer must agree; fused shapes only
    args.flags = rt.HAS_SEQ_IDX
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1
    assert "seq_idx" in rt.last_error(lib)
    args.seq_idx = fake
    args.shape = _shape(headdim=32)
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -2
    args.shape, args.flags, args.seq_idx = _shape(), 0, None
    # varlen states: batch 1, nseqs >= 1, chunk_size a multiple of 64
    args.flags = rt.VARLEN_STATES
    args.cu_seqlens = fake
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1  # no varlen_states
    args.varlen_states, args.nseqs = fake, 3
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1  # batch 2
    assert "batch 1" in rt.last_error(lib)
    args.shape = _shape(batch=1, chunk_size=96)
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -2
    args.shape, args.nseqs = _shape(batch=1), 0
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -1
    args.flags, args.cu_seqlens, args.varlen_states = 0, None, None
    # a segmented shape (few streams, long sequence) without its workspace
    args.shape = _shape(batch=1, seqlen=4096)
    assert lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, None) == -3
    assert lib.mamba2_ssd_fwd(None, None, 0, None) == -1


def test_forward_issues_kernels_only():
    """The forward (also the empty-sequence path, whose states a fill kernel
    writes) enqueues no memset or memcpy, so a caller may capture it in a
    graph: no library source calls them and the built library does not link
    them."""
    csrc = os.path.join(ROOT, "mamba-ascendc_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h")):
            code = re.sub(r"//.*", "", open(os.path.join(csrc, name)).read())
            assert not re.search(r"\bhipMem(set|cpy)\w*\s*\(", code), name
    out = subprocess.run(["nm", "-D", "--undefined-only", rt.LIBRARY_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert not re.search(r"\bhipMem(set|cpy)", out), out


def test_state_passing_rejects_bad_arguments():
    lib = rt.load_library()
    fake = ctypes.c_void_p(0x1000)
    assert lib.mamba2_ssd_state_passing(None, fake, None, fake, None, 1, 1, 1, 64, 64, None) == -1
    assert lib.mamba2_ssd_state_passing(fake, fake, None, fake, None, 1, 1, 0, 64, 64, None) == -1
    assert lib.mamba2_ssd_state_passing(fake, fake, None, fake, None, 1, 1, 1, 3, 3, None) == -2
    # limits of the kernel's 32-bit offsets: 16 chunks of P*N floats, and the
    # log decays of K + 32 chunks, must stay below 2^31 bytes
    biggest_pn = 0x7FFFFFFF // (4 * 16)
    assert lib.mamba2_ssd_state_passing(fake, fake, None, fake, None, 1, 1, 1, biggest_pn + 1, 1,
                                        None) == -2
    assert "headdim*dstate" in rt.last_error(lib)
    assert lib.mamba2_ssd_state_passing(fake, fake, None, fake, None, 1, 1, 0x7FFFFFFF // 4 - 31,
                                        64, 64, None) == -2
    assert lib.mamba2_ssd_state_passing(fake, fake, None, fake, None, 256, 256, 1, 64, 64,
                                        None) == -2
    # the fp16 form: the same checks, and its fp32 output may not overlap the fp16 input
    f16 = lib.mamba2_ssd_state_passing_f16
    assert f16(None, fake, None, fake, None, 1, 1, 1, 64, 64, None) == -1
    assert f16(fake, fake, None, fake, None, 1, 1, 1, 3, 3, None) == -2
    assert f16(fake, fake, None, fake, None, 1, 1, 2, 64, 64, None) == -1
    assert "overlap" in rt.last_error(lib)


def test_decode_step_rejects_bad_arguments():
    """mamba2_selective_state_update validates before any GPU work."""
    lib = rt.load_library()
    fake = ctypes.c_void_p(0x1000)

    def args(**kw):
        a = rt.Mamba2SsuArgs(2, 4, 64, 128, 2, rt.SSU_TIED, fake, 2, 4 * 64 * 128, None,
                             fake, fake, fake, fake, fake, None, None, None, fake)
        for k, v in kw.items():
            setattr(a, k, v)
        return a

    assert lib.mamba2_selective_state_update(None, None) == -1
    assert lib.mamba2_selective_state_update(ctypes.byref(args(x=None)), None) == -1
    assert "non-NULL" in rt.last_error(lib)
    assert lib.mamba2_selective_state_update(ctypes.byref(args(ngroups=3)), None) == -1
    assert lib.mamba2_selective_state_update(ctypes.byref(args(flags=rt.SSU_TIED | rt.HAS_D)), None) == -1
    assert "HAS_D" in rt.last_error(lib)
    assert lib.mamba2_selective_state_update(ctypes.byref(args(flags=1 << 20)), None) == -1
    assert lib.mamba2_selective_state_update(ctypes.byref(args(dstate=130)), None) == -2
    assert lib.mamba2_selective_state_update(ctypes.byref(args(dstate=512)), None) == -2
    # slot stride smaller than a slot, too few slots for the batch
    assert lib.mamba2_selective_state_update(ctypes.byref(args(state_slot_stride=100)), None) == -1
    assert lib.mamba2_selective_state_update(ctypes.byref(args(state_slots=1)), None) == -1
    # misaligned state
    assert lib.mamba2_selective_state_update(ctypes.byref(args(state=ctypes.c_void_p(0x1004))), None) == -1
    # explicit strides: B / C rows must stay 16-byte aligned
    bad = args(flags=rt.SSU_TIED | rt.SSU_STRIDES)
    bad.strides.bc_b, bad.strides.bc_g = 6, 128
    assert lib.mamba2_selective_state_update(ctypes.byref(bad), None) == -1
    assert "multiples of 4" in rt.last_error(lib)
    # an untied A read by rows of four needs head / dim strides that keep them aligned
    bad = args(flags=rt.SSU_STRIDES)
    bad.strides.bc_b, bad.strides.bc_g = 256, 128
    bad.strides.A_h, bad.strides.A_p, bad.strides.A_n = 64 * 130, 130, 1
    assert lib.mamba2_selective_state_update(ctypes.byref(bad), None) == -1


def test_decode_step_python_shape_errors():
    """The Python entry point checks shapes (the reference's asserts) before
    touching the GPU."""
    from ascend_kernel import selective_state_update

    b, h, p, n = 2, 4, 8, 16
    state, x = torch.zeros(b, h, p, n), torch.zeros(b, h, p)
    dt, A = torch.zeros(b, h, p), torch.zeros(h, p, n)
    B = C = torch.zeros(b, 2, n)
    with pytest.raises(ValueError, match="x must be"):
        selective_state_update(state, torch.zeros(b, h, p + 1), dt, A, B, C)
    with pytest.raises(ValueError, match="divisible"):
        selective_state_update(state, x, dt, A, torch.zeros(b, 3, n), torch.zeros(b, 3, n))
    with pytest.raises(ValueError, match="D must be"):
        selective_state_update(state, x, dt, A, B, C, D=torch.zeros(h, p + 1))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        selective_state_update(state, x, dt, A, B, C)


def test_ssdcore_rejects_unknown_backend_and_cpu():
    from ascend_kernel import SsdCore

    with pytest.raises(ValueError):
        SsdCore(backend="tpu")
    x, dt, A, B, C = _cpu_inputs()
    with pytest.raises(RuntimeError, match="ROCm"):
        SsdCore()(x, dt, A, B, C, 64, D=None, z=None, dt_bias=None)


def _cpu_inputs():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 64, 2, 64, generator=g)
    dt = torch.rand(1, 64, 2, generator=g)
    A = -torch.rand(2, generator=g)
    B = torch.randn(1, 64, 1, 64, generator=g)
    C = torch.randn(1, 64, 1, 64, generator=g)
    return x, dt, A, B, C


def test_public_api_rejects_cpu_tensors():
    x, dt, A, B, C = _cpu_inputs()
    with pytest.raises(RuntimeError, match="ROCm GPU tensor"):
        api.mamba2_ssd_fwd(x, dt, A, B, C, 64)


def test_public_api_training_spec_error():
    x, dt, A, B, C = _cpu_inputs()
    x.requires_grad_(True)
    with pytest.raises(NotImplementedError):
        api.mamba2_ssd_fwd(x, dt, A, B, C, 64, dt_softplus=True)


def test_public_api_packed_sequence_errors():
    x, dt, A, B, C = _cpu_inputs()
    b, l = x.shape[:2]
    with pytest.raises(RuntimeError, match="seq_idx must have shape"):
        api.mamba2_ssd_fwd(x, dt, A, B, C, 64, seq_idx=torch.zeros(b, l + 1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="integer"):
        api.mamba2_ssd_fwd(x, dt, A, B, C, 64, seq_idx=torch.zeros(b, l))
    with pytest.raises(ValueError, match="cu_seqlens"):
        api.mamba2_ssd_fwd(x, dt, A, B, C, 64, return_varlen_states=True)
    two = [torch.cat([t, t]) if t.dim() > 1 else t for t in (x, dt, A, B, C)]
    with pytest.raises(RuntimeError, match="batch 1"):
        api.mamba2_ssd_fwd(*two, 64, cu_seqlens=torch.tensor([0, l]), return_varlen_states=True)
    with pytest.raises(NotImplementedError, match="multiple of 64"):
        api.mamba2_ssd_fwd(x, dt, A, B, C, 96, cu_seqlens=torch.tensor([0, l]),
                           return_varlen_states=True)
    with pytest.raises(NotImplementedError, match="dstate"):
        api.mamba2_ssd_fwd(x[..., :32].contiguous(), dt, A, B, C, 64,
                           seq_idx=torch.zeros(b, l, dtype=torch.int32))


def test_operator_library_schemas():
    """torch.ops.mamba_ascend.* come from the C++ operator library with the
    reference's schemas for the forward and the state-passing op
    (mamba_ascendc/csrc/register.cpp:175-179, 89-90), this build's backward,
    and the internal forward with the training outputs."""
    api.register_ops()
    want = {
        "mamba2_ssd_fwd": "mamba2_ssd_fwd(Tensor x, Tensor dt, Tensor A, Tensor B, Tensor C, Tensor? D=None, "
                          "Tensor? z=None, Tensor? dt_bias=None, Tensor? initial_states=None, int chunk_size=256, "
                          "bool dt_softplus=False, float dt_limit_min=0.0, float dt_limit_max=3.402823466e+38) "
                          "-> (Tensor, Tensor)",
        "mamba2_ssd_state_passing": "mamba2_ssd_state_passing(Tensor chunk_states, Tensor dA_cumsum, "
                                    "Tensor? initial_states=None) -> (Tensor, Tensor)",
    }
    for name, schema in want.items():
        got = getattr(torch.ops.mamba_ascend, name).default._schema
        assert got == torch._C.parse_schema("mamba_ascend::" + schema), str(got)
    bwd = str(torch.ops.mamba_ascend.mamba2_ssd_bwd_m1.default._schema)
    assert bwd.endswith("Tensor? seq_idx=None) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, "
                        "Tensor, Tensor)")
    ex = str(torch.ops.mamba_ascend.mamba2_ssd_fwd_ex.default._schema)
    assert "bool want_final, bool want_pre_gate, bool want_states" in ex
    # the operators' device check runs first for CPU tensors
    x, dt, A, B, C = _cpu_inputs()
    with pytest.raises(RuntimeError, match="x must be a ROCm GPU tensor"):
        torch.ops.mamba_ascend.mamba2_ssd_fwd(x, dt, A, B, C)
    with pytest.raises(RuntimeError, match="chunk_states must be a ROCm GPU tensor"):
        torch.ops.mamba_ascend.mamba2_ssd_state_passing(torch.zeros(1, 1, 2, 4, 4), torch.zeros(1, 1, 2, 8))


def test_meta_shape_inference():
    api.register_ops()
    x = torch.empty(2, 100, 8, 64, device="meta")
    dt = torch.empty(2, 100, 8, device="meta")
    A = torch.empty(8, device="meta")
    B = torch.empty(2, 100, 2, 128, device="meta")
    out, final = torch.ops.mamba_ascend.mamba2_ssd_fwd(x, dt, A, B, B, None, None, None, None, 64)
    assert out.shape == x.shape and final.shape == (2, 8, 64, 128)
    grads = torch.ops.mamba_ascend.mamba2_ssd_bwd_m1(x, dt, A, B, B, x, None, None, None, None, None)
    assert [tuple(g.shape) for g in grads[:5]] == [tuple(x.shape), tuple(dt.shape), (8,), tuple(B.shape), tuple(B.shape)]
    states, fin = torch.ops.mamba_ascend.mamba2_ssd_state_passing(
        torch.empty(2, 8, 4, 64, 64, device="meta"), torch.empty(2, 8, 4, 64, device="meta"), None)
    assert states.shape == (2, 8, 4, 64, 64) and fin.shape == (2, 8, 64, 64)
    # fp16 chunk states give fp32 states (the reference op's output dtype)
    states, fin = torch.ops.mamba_ascend.mamba2_ssd_state_passing(
        torch.empty(2, 8, 4, 64, 64, device="meta", dtype=torch.float16), torch.empty(2, 8, 4, 64, device="meta"),
        None)
    assert states.dtype == torch.float32 and fin.dtype == torch.float32


@pytest.mark.parametrize(
    "mutate,match",
    [
        (lambda t: {**t, "dt": t["dt"][..., :1].contiguous()}, "dt shape"),
        (lambda t: {**t, "A": t["A"][:1].contiguous()}, "A shape"),
        (lambda t: {**t, "C": t["C"][:, :, :, :32].contiguous()}, "B and C shapes"),
        (lambda t: {**t, "x": t["x"].transpose(1, 2)}, "contiguous"),
        (lambda t: {**t, "x": t["x"].double()}, "float32"),
    ],
)
def test_validation_messages(mutate, match, monkeypatch):
    """Shape/dtype/layout checks, with the device check bypassed (no GPU here)."""
    x, dt, A, B, C = _cpu_inputs()
    t = mutate(dict(x=x, dt=dt, A=A, B=B, C=C))

    def check(op, name, ten):
        if ten.dtype != torch.float32:
            raise RuntimeError(f"{op}: {name} must be float32 (got {ten.dtype})")
        if not ten.is_contiguous():
            raise RuntimeError(f"{op}: {name} must be contiguous")

    monkeypatch.setattr(api, "_check_tensor", check)
    with pytest.raises(RuntimeError, match=match):
        api._validate_fwd("mamba2_ssd_fwd", t["x"], t["dt"], t["A"], t["B"], t["C"], 64,
                          None, None, None, None, 0.0, math.inf)


def test_header_constants_match_the_python_side():
    """Flag bits, ABI version and status codes of include/mamba2_ssd.h are the
    values the ctypes layer passes and decodes."""
    text = open(HEADER).read()
    flags = re.findall(r"#define (MAMBA2_\w+) \(1u << (\d+)\)", text)
    assert len(flags) >= 11
    for name, bit in flags:
        short = name.replace("MAMBA2_SSD_", "").replace("MAMBA2_", "")
        assert getattr(rt, short) == 1 << int(bit), name
    assert rt.ABI_VERSION == int(re.search(r"#define MAMBA2_SSD_ABI_VERSION (\d+)", text).group(1))
    codes = re.findall(r"#define MAMBA2_SSD_(OK|ERR_\w+) \(?(-?\d+)\)?", text)
    assert len(codes) == len(rt.STATUS_NAMES)
    for name, value in codes:
        assert rt.STATUS_NAMES[int(value)] == name.replace("ERR_", ""), name


def test_struct_layouts_match_ctypes(tmp_path):
    """sizeof and every member offset of the header's argument structs, as a C
    compiler lays them out, equal the ctypes declarations."""
    import shutil

    if shutil.which("gcc") is None:
        pytest.skip("needs gcc")
    classes = [rt.Mamba2SsdShape, rt.Mamba2SsdFwdArgs, rt.Mamba2SsdBwdArgs, rt.Mamba2SsuStrides,
               rt.Mamba2SsuArgs]
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "mamba2_ssd.h"', "int main(void) {"]
    for cls in classes:
        n = cls.__name__
        lines.append(f'  printf("{n} %zu\\n", sizeof({n}));')
        for field in cls._fields_:
            lines.append(f'  printf("{n}.{field[0]} %zu\\n", offsetof({n}, {field[0]}));')
    lines += ["  return 0;", "}"]
    src, exe = tmp_path / "layout.c", tmp_path / "layout"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["gcc", "-std=c11", "-I", os.path.dirname(HEADER), "-o", str(exe), str(src)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines())
    for cls in classes:
        n = cls.__name__
        assert int(got[n]) == ctypes.sizeof(cls), n
        for field in cls._fields_:
            assert int(got[f"{n}.{field[0]}"]) == getattr(cls, field[0]).offset, (n, field[0])


def test_noalloc_forward_limits_without_gpu():
    """mamba2_ssd_fwd_noalloc: its scratch size is the header's, and a forward
    whose scratch would exceed it is rejected with the workspace status before
    any GPU work (here: varlen states without saved states, whose chunk states
    of a 2^20-token sequence need 2 GiB)."""
    text = open(HEADER).read()
    m = re.search(r"#define MAMBA2_SSD_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == rt.NOALLOC_SCRATCH_BYTES
    lib = rt.load_library()
    assert lib.mamba2_ssd_fwd_noalloc(None, None) == -1
    fake = ctypes.c_void_p(0x1000)
    shape = _shape(batch=1, seqlen=1 << 20, nheads=8, ngroups=1)
    need = ctypes.c_size_t(0)
    assert lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(shape), rt.VARLEN_STATES, ctypes.byref(need)) == 0
    assert need.value > rt.NOALLOC_SCRATCH_BYTES
    args = rt.Mamba2SsdFwdArgs(shape, rt.VARLEN_STATES, 0.0, math.inf, fake, fake, fake, fake, fake,
                               None, None, None, None, fake, None, None, None, None, fake, 2, fake)
    assert lib.mamba2_ssd_fwd_noalloc(ctypes.byref(args), None) == -3
    assert "mamba2_ssd_fwd_noalloc" in rt.last_error(lib)


def test_training_policy_object():
    """TrainingPolicy: the default keeps the chunk states; set_training_policy
    swaps the default and returns the old one; training_policy(...) changes it
    for a block only; the public forward takes a per-call override."""
    import inspect

    import ascend_kernel

    assert ascend_kernel.get_training_policy() == ascend_kernel.TrainingPolicy(save_chunk_states=True)
    with ascend_kernel.training_policy(save_chunk_states=False) as pol:
        assert pol.save_chunk_states is False
        assert ascend_kernel.get_training_policy() is pol
    assert ascend_kernel.get_training_policy().save_chunk_states is True
    old = ascend_kernel.set_training_policy(ascend_kernel.TrainingPolicy(save_chunk_states=False))
    try:
        assert ascend_kernel.get_training_policy().save_chunk_states is False
    finally:
        ascend_kernel.set_training_policy(old)
    with pytest.raises(TypeError):
        ascend_kernel.set_training_policy(False)
    with pytest.raises(TypeError):
        with ascend_kernel.training_policy(no_such_field=True):
            pass
    # a block affects its own thread only, and overlapping blocks in two
    # threads each restore their own state
    import threading

    inside, release, seen = threading.Event(), threading.Event(), {}

    def other():
        with ascend_kernel.training_policy(save_chunk_states=False):
            inside.set()
            release.wait(10)
            seen["other_in_block"] = ascend_kernel.get_training_policy().save_chunk_states
        seen["other_after"] = ascend_kernel.get_training_policy().save_chunk_states

    th = threading.Thread(target=other)
    th.start()
    assert inside.wait(10)
    seen["main_during"] = ascend_kernel.get_training_policy().save_chunk_states
    with ascend_kernel.training_policy(save_chunk_states=True):
        release.set()
        th.join(10)
    assert seen == {"other_in_block": False, "other_after": True, "main_during": True}
    assert ascend_kernel.get_training_policy().save_chunk_states is True
    sig = inspect.signature(ascend_kernel.mamba2_ssd_fwd)
    assert sig.parameters["save_chunk_states"].kind is inspect.Parameter.KEYWORD_ONLY
