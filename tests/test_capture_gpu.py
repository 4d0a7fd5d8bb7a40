"""The forward under HIP graph capture, and its empty-sequence path.

The forward enqueues kernels only (no memset or memcpy nodes, no allocation):
the empty sequence (seqlen 0, allowed by the C ABI) writes its final state
(the initial state, or zero) and its varlen states (zero) with a fill kernel.
A captured forward is replayed several times, with the program's own eager
work and synchronisations between the replays and the outputs reset to NaN
before each, and every replay must equal the eager call bit for bit.
"""

import ctypes
import math
import sys

import pytest
import torch

from oracle.ssd_reference import make_inputs

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _flags(rt, dev):
    f = rt.DT_SOFTPLUS
    if "D" in dev:
        f |= rt.HAS_D | (rt.D_PER_CHANNEL if dev["D"].dim() == 2 else 0)
    f |= (rt.HAS_Z if "z" in dev else 0) | (rt.HAS_DT_BIAS if "dt_bias" in dev else 0)
    return f | (rt.HAS_INITIAL if "initial_states" in dev else 0)


def _args(rt, shape, dev, flags, out, fin, cu=None, nseqs=0, varlen=None):
    b, l, h, p, n, chunk, g = shape
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return rt.Mamba2SsdFwdArgs(rt.Mamba2SsdShape(b, l, h, p, g, n, chunk), flags, 0.0, math.inf,
                               P(dev["x"]), P(dev["dt"]), P(dev["A"]), P(dev["B"]), P(dev["C"]),
                               P(dev.get("D")), P(dev.get("z")), P(dev.get("dt_bias")),
                               P(dev.get("initial_states")), P(out), P(fin), None, None, None, P(cu), nseqs,
                               P(varlen))


def _stand_ins():
    """Tensors whose pointers the empty-sequence call takes but never reads
    (the ABI wants them non-NULL)."""
    one = torch.zeros(16, device="cuda")
    return {"x": one, "dt": one, "A": one, "B": one, "C": one}


@pytest.mark.parametrize("noalloc", [False, True], ids=["workspace", "noalloc"])
def test_empty_sequence_writes_the_states_by_kernel(noalloc):
    """seqlen 0: the final state is the initial state (or zero) and every
    varlen state is zero; outputs start as NaN, so each element must be
    written."""
    _need_gpu()
    from ascend_kernel import _runtime as rt

    lib = rt.load_library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    shape = [2, 0, 4, 64, 64, 64, 2]
    b, _l, h, p, n, _c, _g = shape

    def run(args):
        if noalloc:
            return lib.mamba2_ssd_fwd_noalloc(ctypes.byref(args), stream)
        return lib.mamba2_ssd_fwd(ctypes.byref(args), None, 0, stream)

    dev = _stand_ins()
    out = torch.zeros(16, device="cuda")
    init = torch.randn(b, h, p, n, device="cuda")
    for with_init in (True, False):
        _say(f"empty sequence, initial state {with_init}, noalloc {noalloc}")
        d = dict(dev, initial_states=init) if with_init else dev
        fin = torch.full((b, h, p, n), math.nan, device="cuda")
        rt.check(run(_args(rt, shape, d, _flags(rt, d), out, fin)), "fwd L=0", lib)
        torch.cuda.synchronize()
        assert torch.equal(fin, init if with_init else torch.zeros_like(fin))
    # varlen states of an empty batch-1 problem: all zero
    shape1 = [1, 0, 4, 64, 64, 64, 2]
    fin = torch.full((1, h, p, n), math.nan, device="cuda")
    var = torch.full((3, h, p, n), math.nan, device="cuda")
    cu = torch.zeros(4, dtype=torch.int32, device="cuda")
    args = _args(rt, shape1, dev, rt.DT_SOFTPLUS | rt.VARLEN_STATES, out, fin, cu=cu, nseqs=3, varlen=var)
    rt.check(run(args), "fwd L=0 varlen", lib)
    torch.cuda.synchronize()
    assert torch.equal(var, torch.zeros_like(var)) and torch.equal(fin, torch.zeros_like(fin))


CAPTURED = [
    # [B, L, H, P, N, chunk, G], features
    ([2, 0, 4, 64, 64, 64, 2], ("init",)),            # empty sequence: the fill kernel
    ([2, 1024, 4, 64, 64, 64, 2], ("D", "init")),     # segments folded from pre-segments
    ([1, 600, 2, 64, 128, 128, 1], ("z", "init")),    # dstate 128, segments
    ([1, 300, 8, 64, 128, 64, 1], ("D",)),            # dstate 128, C . B^T precomputed
]


@pytest.mark.parametrize("shape,feats", CAPTURED, ids=[str(c[0]) for c in CAPTURED])
@pytest.mark.parametrize("noalloc", [False, True], ids=["workspace", "noalloc"])
def test_captured_forward_replays_match_eager(shape, feats, noalloc):
    _need_gpu()
    import ascend_kernel
    from ascend_kernel import _runtime as rt

    lib = rt.load_library()
    b, l, h, p, n, chunk, g = shape
    _say(f"capture {shape} {feats} noalloc {noalloc}")
    if l == 0:
        dev = _stand_ins()
        dev["initial_states"] = torch.randn(b, h, p, n, device="cuda")
        out = torch.zeros(16, device="cuda")
    else:
        dev = {k: v.cuda() for k, v in make_inputs(shape, seed=41, features=feats).items()}
        out = torch.full_like(dev["x"], math.nan)
    fin = torch.full((b, h, p, n), math.nan, device="cuda")
    flags = _flags(rt, dev)
    args = _args(rt, shape, dev, flags, out, fin)
    nb = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(args.shape), flags, ctypes.byref(nb)), "ws", lib)
    ws = torch.empty(max(1, nb.value), dtype=torch.uint8, device="cuda")

    def call(stream):
        st = ctypes.c_void_p(stream.cuda_stream)
        if noalloc:
            return lib.mamba2_ssd_fwd_noalloc(ctypes.byref(args), st)
        return lib.mamba2_ssd_fwd(ctypes.byref(args), ctypes.c_void_p(ws.data_ptr()), ws.numel(), st)

    # eager call (also the noalloc entry's one-time scratch lookup, outside capture)
    rt.check(call(torch.cuda.current_stream()), "eager", lib)
    torch.cuda.synchronize()
    want_out, want_fin = out.clone(), fin.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = call(torch.cuda.current_stream())
    rt.check(rc, "captured", lib)
    # other eager work between the replays: the same forward on other inputs
    other = {k: v.cuda() for k, v in make_inputs([1, 256, 2, 64, 64, 64, 1], seed=42).items()}
    for rep in range(3):
        if l > 0:  # (the empty sequence has no token outputs: `out` is a stand-in)
            out.fill_(math.nan)
        fin.fill_(math.nan)
        y, _ = ascend_kernel.mamba2_ssd_fwd(other["x"], other["dt"], other["A"], other["B"], other["C"], 64,
                                            dt_softplus=True, return_final_state=True)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_out) and torch.equal(fin, want_fin), rep
        assert bool(torch.isfinite(y).all())
    _say("  3 replays identical to the eager call")
