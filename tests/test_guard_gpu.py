"""Out-of-bounds guard: every output and the workspace of the C ABI calls sit
inside larger buffers whose margins hold a sentinel bit pattern; after the call
the margins must be unchanged.  The cases cover the paths whose stores rely on
in-kernel guards or clamps: ragged sequence ends (partial last chunk), dstate
128 (state halves and their workspace), segmented streams (segment states in
the workspace), packed sequences and varlen states, the training forward's
pre_gate and chunk states, and the backward's outputs and workspace.
"""

import ctypes
import math
import sys

import pytest
import torch

from oracle.ssd_reference import make_inputs

pytestmark = pytest.mark.gpu

GUARD = 4096           # floats of margin on each side (16 KiB)
SENTINEL = 0x7FBADBAD  # a NaN payload no kernel writes


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class Guarded:
    """A float32 (or byte) region of `shape` inside a buffer with sentinel margins."""

    def __init__(self, shape, dtype=torch.float32):
        n = math.prod(shape)
        self.dtype = dtype
        if dtype == torch.uint8:
            n4 = (n + 3) // 4
            self.buf = torch.full((GUARD + n4 + GUARD,), SENTINEL, dtype=torch.int32, device="cuda")
            self.n4 = n4
            self.view = self.buf[GUARD:GUARD + n4].view(torch.uint8)[:n]
        else:
            self.buf = torch.full((GUARD + n + GUARD,), SENTINEL, dtype=torch.int32, device="cuda")
            self.n4 = n
            self.view = self.buf[GUARD:GUARD + n].view(torch.float32).view(shape)

    def ptr(self):
        return ctypes.c_void_p(self.view.data_ptr())

    def intact(self):
        lo = self.buf[:GUARD]
        hi = self.buf[GUARD + self.n4:]
        return bool((lo == SENTINEL).all()) and bool((hi == SENTINEL).all())


def _flags(rt, feats, softplus=True):
    f = rt.DT_SOFTPLUS if softplus else 0
    if "D" in feats:
        f |= rt.HAS_D
    if "D2" in feats:
        f |= rt.HAS_D | rt.D_PER_CHANNEL
    if "z" in feats:
        f |= rt.HAS_Z
    if "bias" in feats:
        f |= rt.HAS_DT_BIAS
    if "init" in feats:
        f |= rt.HAS_INITIAL
    return f


FWD = [
    # shape [B, L, H, P, N, chunk, G], features, extra
    ([2, 600, 4, 64, 64, 64, 2], ("D", "z"), ""),                 # ragged end, segmented
    ([1, 800, 2, 64, 128, 128, 1], ("D2", "z", "init"), ""),      # dstate 128, ragged, segments
    ([2, 130, 256, 64, 64, 64, 64], ("bias",), ""),               # many streams, one segment
    ([1, 300, 4, 128, 64, 64, 2], ("D", "init"), ""),             # headdim 128 (head split)
    ([2, 150, 4, 64, 64, 64, 2], ("z", "bias", "init"), "save"),  # training forward
    ([1, 270, 4, 64, 128, 64, 1], ("D",), "packed"),              # packed sequences, dstate 128
    ([1, 250, 4, 64, 64, 64, 2], ("init",), "varlen"),            # varlen states
    ([2, 70, 3, 32, 16, 16, 1], ("D", "z"), ""),                  # zero-padded (P 32, N 16)
    ([1, 200, 2, 80, 96, 64, 1], ("D2", "z", "init"), ""),        # zero-padded (P 80, N 96)
    ([1, 40, 2, 20, 200, 8, 1], ("D",), ""),                      # generic path (N 200)
]


@pytest.mark.parametrize("shape,feats,extra", FWD, ids=[f"{c[0]}-{'+'.join(c[1])}-{c[2]}" for c in FWD])
def test_forward_writes_stay_in_bounds(shape, feats, extra):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from ascend_kernel import _runtime as rt

    lib = rt.load_library()
    b, l, h, p, n, chunk, g = shape
    _say(f"guard forward {shape} {feats} {extra}")
    inp = {k: v.cuda() for k, v in make_inputs(shape, seed=17, features=feats).items()}
    flags = _flags(rt, feats)
    k = (l + 63) // 64
    outs = {"out": Guarded((b, l, h, p)), "final": Guarded((b, h, p, n))}
    if "z" in feats:
        outs["pre_gate"] = Guarded((b, l, h, p))
    if extra == "save":
        flags |= rt.SAVED_STATES
        outs["states"] = Guarded((b, h, k, p, n))
    seq = cu = None
    nseqs = 0
    if extra == "packed":
        flags |= rt.HAS_SEQ_IDX
        seq = torch.cat([torch.zeros(90), torch.ones(100), 2 * torch.ones(80)]).to(torch.int32)[None].cuda()
    if extra == "varlen":
        flags |= rt.VARLEN_STATES
        cu = torch.tensor([0, 100, 180, 250], dtype=torch.int32, device="cuda")
        nseqs = 3
        outs["varlen"] = Guarded((nseqs, h, p, n))
    shp = rt.Mamba2SsdShape(b, l, h, p, g, n, chunk)
    nb = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(shp), flags, ctypes.byref(nb)), "ws", lib)
    ws = Guarded((max(1, nb.value),), torch.uint8)
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    args = rt.Mamba2SsdFwdArgs(shp, flags, 0.0, math.inf, P(inp["x"]), P(inp["dt"]), P(inp["A"]),
                               P(inp["B"]), P(inp["C"]), P(inp.get("D")), P(inp.get("z")),
                               P(inp.get("dt_bias")), P(inp.get("initial_states")), outs["out"].ptr(),
                               outs["final"].ptr(), outs["pre_gate"].ptr() if "pre_gate" in outs else None,
                               outs["states"].ptr() if "states" in outs else None, P(seq), P(cu), nseqs,
                               outs["varlen"].ptr() if "varlen" in outs else None)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rt.check(lib.mamba2_ssd_fwd(ctypes.byref(args), ws.ptr(), nb.value, stream), "fwd", lib)
    torch.cuda.synchronize()
    for name, gb in list(outs.items()) + [("workspace", ws)]:
        assert gb.intact(), f"{name}: a store landed outside its buffer"
        if name != "workspace":
            assert bool(torch.isfinite(gb.view).all()), f"{name}: not every element written"


BWD = [
    ([2, 200, 4, 64, 64, 64, 2], ("D2", "z", "bias", "init"), True),    # reverse runs of 1 chunk, ragged
    ([1, 700, 8, 64, 64, 64, 2], ("D",), False),                        # reverse runs, segmented recompute
    ([4, 2200, 8, 64, 64, 64, 4], ("D", "z", "init"), False),           # runs of 3 chunks, last of 2
    ([2, 300, 16, 64, 64, 64, 2], ("z", "init"), True),                 # split path (8 heads per group)
    ([4, 150, 256, 64, 64, 64, 64], ("z", "init"), True),               # fused reverse, R = 4
    ([2, 100, 512, 64, 64, 64, 128], ("D", "bias"), False),             # fused reverse, R = 4
    ([2, 100, 256, 64, 64, 64, 32], ("z", "init"), True),               # reverse dstate pass (R = 8)
]


@pytest.mark.parametrize("shape,feats,saved", BWD, ids=[f"{c[0]}-{'+'.join(c[1])}-{c[2]}" for c in BWD])
def test_backward_writes_stay_in_bounds(shape, feats, saved):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from ascend_kernel import _runtime as rt
    from ascend_kernel import mamba2 as api

    lib = rt.load_library()
    b, l, h, p, n, chunk, g = shape
    _say(f"guard backward {shape} {feats} saved={saved}")
    inp = {k: v.cuda() for k, v in make_inputs(shape, seed=19, features=feats).items()}
    out, fin, pre_gate, states, _ = api._fwd_raw(
        inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp.get("D"), inp.get("z"), inp.get("dt_bias"),
        inp.get("initial_states"), chunk, True, 0.0, math.inf, want_pre_gate=True, want_states=saved)
    flags = _flags(rt, feats) | (rt.SAVED_STATES if saved else 0)
    dout, dfin = torch.randn_like(out), torch.randn_like(fin)
    grads = {"dx": Guarded((b, l, h, p)), "ddt": Guarded((b, l, h)), "dA": Guarded((h,)),
             "dB": Guarded((b, l, g, n)), "dC": Guarded((b, l, g, n))}
    if "D" in feats:
        grads["dD"] = Guarded((h,))
    if "D2" in feats:
        grads["dD"] = Guarded((h, p))
    if "z" in feats:
        grads["dz"] = Guarded((b, l, h, p))
    if "bias" in feats:
        grads["ddt_bias"] = Guarded((h,))
    if "init" in feats:
        grads["dinit"] = Guarded((b, h, p, n))
    shp = rt.Mamba2SsdShape(b, l, h, p, g, n, chunk)
    nb = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_bwd_m1_workspace_size(ctypes.byref(shp), flags, ctypes.byref(nb)), "ws", lib)
    ws = Guarded((max(1, nb.value),), torch.uint8)
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    G = lambda k: grads[k].ptr() if k in grads else None  # noqa: E731
    args = rt.Mamba2SsdBwdArgs(shp, flags, 0.0, math.inf, P(inp["x"]), P(inp["dt"]), P(inp["A"]),
                               P(inp["B"]), P(inp["C"]), P(inp.get("D")), P(inp.get("z")),
                               P(inp.get("dt_bias")), P(inp.get("initial_states")), P(dout), P(dfin),
                               P(pre_gate), P(states), G("dx"), G("ddt"), G("dA"), G("dB"), G("dC"),
                               G("dD"), G("dz"), G("ddt_bias"), G("dinit"))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rt.check(lib.mamba2_ssd_bwd_m1(ctypes.byref(args), ws.ptr(), nb.value, stream), "bwd", lib)
    torch.cuda.synchronize()
    for name, gb in list(grads.items()) + [("workspace", ws)]:
        assert gb.intact(), f"{name}: a store landed outside its buffer"
        if name != "workspace":
            assert bool(torch.isfinite(gb.view).all()), f"{name}: not every element written"
