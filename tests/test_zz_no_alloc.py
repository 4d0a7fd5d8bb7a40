"""mamba2_ssd_fwd_noalloc (the allocation-free forward) against mamba2_ssd_fwd.

Both entry points run the same kernels on the same plan; the allocation-free one
takes its scratch (segment contributions and log decays of long sequences with
few streams, the C . B^T products of dstate 128 with many heads per group, the
padded copies of headdims off multiples of 64) from the library's static device
array instead of a workspace, so the results must be bit-identical.  The calls come in a row on one GPU, each
smaller than the one before, so a call that read scratch contents left by the
previous one would show.  Output buffers start as NaN: every element must be
written.
"""

import ctypes
import math
import sys

import pytest
import torch

from oracle.ssd_reference import make_inputs, parity_metrics, ssd_chunk_scan_ref

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _args(rt, shape, dev, flags, limit, out, fin):
    b, l, h, p, n, chunk, g = shape
    shp = rt.Mamba2SsdShape(b, l, h, p, g, n, chunk)
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return rt.Mamba2SsdFwdArgs(shp, flags, limit[0], limit[1], P(dev["x"]), P(dev["dt"]), P(dev["A"]),
                               P(dev["B"]), P(dev["C"]), P(dev.get("D")), P(dev.get("z")),
                               P(dev.get("dt_bias")), P(dev.get("initial_states")), P(out), P(fin))


CALLS = [
    # shape [B, L, H, P, N, chunk, G], features: 16 (b, h) streams of 32
    # chunks -> 16 segments of 2 chunks, 32 state-only pre-segments and the
    # segment recurrence over them (too many to fold)
    ([2, 2048, 8, 64, 64, 64, 2], ("D2", "z", "bias", "init")),
    # smaller: 4 streams -> 13 segments of one chunk folding up to 12
    # pre-segments, a ragged last chunk
    ([1, 800, 4, 64, 64, 64, 1], ("D",)),
    # smaller still, dstate 128: 4 streams of 10 chunks -> 10 segments
    ([1, 600, 2, 64, 128, 128, 1], ("z", "init")),
    # dstate 128 with 8 heads per group: C . B^T of each chunk in the scratch
    ([1, 300, 8, 64, 128, 64, 1], ("D",)),
    # headdim 32, dstate 48: zero-padded copies in the scratch
    ([1, 200, 2, 32, 48, 64, 1], ("D2", "z", "init")),
]


def test_noalloc_forward_matches_workspace_forward():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from ascend_kernel import _runtime as rt

    lib = rt.load_library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, (shape, feats) in enumerate(CALLS):
        _say(f"call {i}: {shape} {feats}")
        b, l, h, p, n, chunk, g = shape
        inp = make_inputs(shape, seed=31 + i, features=feats)
        dev = {k: v.cuda() for k, v in inp.items()}
        flags = rt.DT_SOFTPLUS
        if "D" in dev:
            flags |= rt.HAS_D | (rt.D_PER_CHANNEL if dev["D"].dim() == 2 else 0)
        flags |= (rt.HAS_Z if "z" in dev else 0) | (rt.HAS_DT_BIAS if "dt_bias" in dev else 0)
        flags |= rt.HAS_INITIAL if "initial_states" in dev else 0
        limit = (0.0, math.inf)
        nb = ctypes.c_size_t(0)
        shp = rt.Mamba2SsdShape(b, l, h, p, g, n, chunk)
        rt.check(lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(shp), flags, ctypes.byref(nb)), "ws", lib)
        assert 0 < nb.value <= rt.NOALLOC_SCRATCH_BYTES, nb.value  # the scratch is in use
        outs = []
        for noalloc in (False, True):
            out = torch.full_like(dev["x"], math.nan)
            fin = torch.full((b, h, p, n), math.nan, device="cuda")
            args = _args(rt, shape, dev, flags, limit, out, fin)
            if noalloc:
                rc = lib.mamba2_ssd_fwd_noalloc(ctypes.byref(args), stream)
            else:
                ws = torch.empty(nb.value, dtype=torch.uint8, device="cuda")
                rc = lib.mamba2_ssd_fwd(ctypes.byref(args), ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                        stream)
            rt.check(rc, "noalloc" if noalloc else "fwd", lib)
            torch.cuda.synchronize()
            outs.append((out.cpu(), fin.cpu()))
        (o_ws, f_ws), (o_na, f_na) = outs
        assert bool(torch.isfinite(o_na).all()) and bool(torch.isfinite(f_na).all())
        assert torch.equal(o_na, o_ws) and torch.equal(f_na, f_ws), i
        ref, ref_fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], chunk,
                                          D=inp.get("D"), z=inp.get("z"), dt_bias=inp.get("dt_bias"),
                                          dt_softplus=True, initial_states=inp.get("initial_states"),
                                          return_final_state=True)
        ma, rl = parity_metrics(o_na, ref)
        fma, frl = parity_metrics(f_na, ref_fin)
        _say(f"  identical to the workspace forward; vs oracle out maxabs {ma:.3e} rel {rl:.3e} | "
             f"final maxabs {fma:.3e} rel {frl:.3e}")
        assert ma <= 2e-2 and rl <= 5e-3 and fma <= 2e-2 and frl <= 5e-3
