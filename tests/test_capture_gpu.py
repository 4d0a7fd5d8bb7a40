"""The forward and the M1 backward under HIP graph capture, and the forward's empty-sequence path.

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


CAPTURED_BWD = [
    # [B, L, H, P, N, chunk, G], features, keep the forward's chunk states
    ([4, 130, 256, 64, 64, 64, 64], ("D", "bias", "init"), False),  # group-major state recompute
    ([4, 130, 256, 64, 64, 64, 64], ("D", "bias", "init"), True),   # saved chunk states
    ([2, 700, 8, 64, 64, 64, 2], ("z", "init"), False),             # runs: pre-pass + recurrence over runs
]


@pytest.mark.parametrize("shape,feats,saved", CAPTURED_BWD,
                         ids=[f"{c[0]}-{'saved' if c[2] else 'recompute'}" for c in CAPTURED_BWD])
def test_captured_backward_replays_match_eager(shape, feats, saved):
    """The M1 backward enqueues kernels only as well (state recompute, run
    pre-pass, recurrence over runs, the fused chunk kernel, the fixed-order
    finalize), so a captured call replays bit for bit."""
    _need_gpu()
    from ascend_kernel import _runtime as rt
    from ascend_kernel import mamba2 as m

    lib = rt.load_library()
    b, l, h, p, n, chunk, g = shape
    _say(f"capture bwd {shape} {feats} saved {saved}")
    dev = {k: v.cuda() for k, v in make_inputs(shape, seed=43, features=feats).items()}
    gen = torch.Generator().manual_seed(9)
    dout = torch.randn(b, l, h, p, generator=gen).cuda()
    dfin = torch.randn(b, h, p, n, generator=gen).cuda()
    D, z, bias, init = dev.get("D"), dev.get("z"), dev.get("dt_bias"), dev.get("initial_states")
    _, _, pre_gate, states, _ = m._fwd_raw(dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], D, z, bias, init,
                                           chunk, True, 0.0, math.inf, want_pre_gate=z is not None,
                                           want_states=saved)
    flags = m._flags(D, z, bias, init, True) | (rt.SAVED_STATES if saved else 0)
    shp = m._shape(dev["x"], dev["B"], chunk)
    nb = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_bwd_m1_workspace_size(ctypes.byref(shp), flags, ctypes.byref(nb)), "ws", lib)
    ws = torch.empty(max(1, nb.value), dtype=torch.uint8, device="cuda")
    grads = {"dx": torch.empty_like(dev["x"]), "ddt": torch.empty_like(dev["dt"]),
             "dA": torch.empty_like(dev["A"]), "dB": torch.empty_like(dev["B"]), "dC": torch.empty_like(dev["C"]),
             "dD": torch.empty_like(D) if D is not None else None,
             "dz": torch.empty_like(z) if z is not None else None,
             "ddt_bias": torch.empty_like(bias) if bias is not None else None,
             "dinit": torch.empty_like(init) if init is not None else None}
    P = m._ptr
    args = rt.Mamba2SsdBwdArgs(
        shp, flags, 0.0, m._limit(math.inf),
        P(dev["x"]), P(dev["dt"]), P(dev["A"]), P(dev["B"]), P(dev["C"]), P(D), P(z), P(bias), P(init),
        P(dout), P(dfin), P(pre_gate), P(states),
        P(grads["dx"]), P(grads["ddt"]), P(grads["dA"]), P(grads["dB"]), P(grads["dC"]),
        P(grads["dD"]), P(grads["dz"]), P(grads["ddt_bias"]), P(grads["dinit"]), None)

    def call(stream):
        return lib.mamba2_ssd_bwd_m1(ctypes.byref(args), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                     ctypes.c_void_p(stream.cuda_stream))

    rt.check(call(torch.cuda.current_stream()), "eager", lib)
    torch.cuda.synchronize()
    want = {k: v.clone() for k, v in grads.items() if v is not None}
    assert all(bool(torch.isfinite(v).all()) for v in want.values())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = call(torch.cuda.current_stream())
    rt.check(rc, "captured", lib)
    import ascend_kernel
    other = {k: v.cuda() for k, v in make_inputs([1, 256, 2, 64, 64, 64, 1], seed=44).items()}
    for rep in range(3):
        for v in grads.values():
            if v is not None:
                v.fill_(math.nan)
        y, _ = ascend_kernel.mamba2_ssd_fwd(other["x"], other["dt"], other["A"], other["B"], other["C"], 64,
                                            dt_softplus=True, return_final_state=True)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, v in want.items():
            assert torch.equal(grads[k], v), (rep, k)
        assert bool(torch.isfinite(y).all())
    _say("  3 replays identical to the eager call")
