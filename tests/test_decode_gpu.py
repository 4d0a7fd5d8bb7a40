"""GPU parity of the decode step ``selective_state_update`` (HIP kernel k_ssu).

Checked against the oracle's ``selective_state_update_ref`` in float64 on the
same inputs (output and the updated state slots), over the tied and untied
forms, the optional D / z / dt_bias, padding slots of a state pool, 3-D
inputs, dstate 16..256 and a head dim that is not a multiple of the rows a
workgroup covers; and as a whole: a sequence decoded token by token equals
the chunked forward on it (every output and the final state).
"""

import math
import sys

import pytest
import torch

from oracle.ssd_reference import parity_metrics, selective_state_update_ref

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


CASES = [
    # batch, nheads, dim, dstate, ngroups, tied, features, softplus, slots (None: one per sequence)
    (3, 8, 64, 128, 2, True, ("D", "z", "bias"), True, None),
    (2, 4, 48, 64, 1, False, ("bias",), False, None),
    (2, 2, 50, 16, 1, True, ("D",), True, None),
    (4, 2, 64, 256, 2, True, ("z",), True, [3, -1, 0, 4]),
    (5, 3, 32, 32, 3, False, ("D", "z", "bias"), True, [1, 0, -2, 2, 4]),
]


@pytest.mark.parametrize("b,h,p,n,g,tied,features,softplus,slots", CASES,
                         ids=[f"b{c[0]}h{c[1]}p{c[2]}n{c[3]}g{c[4]}-{'tied' if c[5] else 'untied'}"
                              f"-{'+'.join(c[6])}" + ("-slots" if c[8] else "") for c in CASES])
def test_decode_step_parity(b, h, p, n, g, tied, features, softplus, slots):
    _need_gpu()
    from ascend_kernel import selective_state_update

    _say(f"decode step b={b} h={h} p={p} n={n} g={g} tied={tied} {features} slots={slots}")
    gen = torch.Generator().manual_seed(7 + n)
    r = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    nslots = b if slots is None else 5
    state = r(nslots, h, p, n)
    x, Bm, Cm = r(b, h, p), r(b, g, n), r(b, g, n)
    if tied:
        dt_h, A_h = torch.rand(b, h, generator=gen), -torch.rand(h, generator=gen)
        bias_h = r(h) * 0.1
        dt, A = dt_h[..., None].expand(b, h, p), A_h[:, None, None].expand(h, p, n)
        bias = bias_h[:, None].expand(h, p)
    else:
        dt, A, bias = torch.rand(b, h, p, generator=gen), -torch.rand(h, p, n, generator=gen), r(h, p) * 0.1
    D = r(h, p) if "D" in features else None
    z = r(b, h, p) if "z" in features else None
    bias = bias if "bias" in features else None
    idx = None if slots is None else torch.tensor(slots, dtype=torch.int32)

    ref_state = state.double()
    want = selective_state_update_ref(
        ref_state, x.double(), dt.double(), A.double(), Bm.double(), Cm.double(),
        D=None if D is None else D.double(), z=None if z is None else z.double(),
        dt_bias=None if bias is None else bias.double(), dt_softplus=softplus,
        state_batch_indices=idx)

    dev = lambda t: None if t is None else t.cuda()  # noqa: E731
    gstate = state.cuda()
    got = selective_state_update(gstate, dev(x), dev(dt), dev(A), dev(Bm), dev(Cm), D=dev(D), z=dev(z),
                                 dt_bias=dev(bias), dt_softplus=softplus,
                                 state_batch_indices=dev(idx))
    torch.cuda.synchronize()
    ma, rl = parity_metrics(got.cpu(), want)
    sa, sl = parity_metrics(gstate.cpu(), ref_state)
    _say(f"  out maxabs {ma:.3e} relL2 {rl:.3e}; state maxabs {sa:.3e} relL2 {sl:.3e}")
    assert got.shape == (b, h, p)
    assert rl <= 1e-5 and sl <= 1e-5, (rl, sl)
    if slots is not None:
        # padding rows are exact zeros and untouched slots keep their bits
        for bi, sidx in enumerate(slots):
            if sidx < 0:
                assert torch.equal(got[bi].cpu(), torch.zeros(h, p))
        used = {s for s in slots if s >= 0}
        for sidx in range(nslots):
            if sidx not in used:
                assert torch.equal(gstate[sidx].cpu(), state[sidx])


def test_decode_step_without_heads():
    """3-D form (batch, dim, dstate): one head, shapes squeezed back."""
    _need_gpu()
    from ascend_kernel import selective_state_update

    gen = torch.Generator().manual_seed(11)
    b, p, n = 3, 64, 64
    state = torch.randn(b, p, n, generator=gen)
    x, dt = torch.randn(b, p, generator=gen), torch.rand(b, p, generator=gen)
    A = -torch.rand(p, n, generator=gen)
    Bm, Cm = torch.randn(b, n, generator=gen), torch.randn(b, n, generator=gen)
    D = torch.randn(p, generator=gen)
    ref_state = state.double().unsqueeze(1).clone()
    want = selective_state_update_ref(ref_state, x.double()[:, None], dt.double()[:, None],
                                      A.double()[None], Bm.double()[:, None], Cm.double()[:, None],
                                      D=D.double()[None], dt_softplus=True)[:, 0]
    gstate = state.cuda()
    got = selective_state_update(gstate, x.cuda(), dt.cuda(), A.cuda(), Bm.cuda(), Cm.cuda(), D=D.cuda(),
                                 dt_softplus=True)
    torch.cuda.synchronize()
    assert got.shape == (b, p)
    _, rl = parity_metrics(got.cpu(), want)
    _, sl = parity_metrics(gstate.cpu(), ref_state[:, 0])
    assert rl <= 1e-5 and sl <= 1e-5, (rl, sl)


def test_decode_loop_equals_chunked_forward():
    """Decoding a sequence token by token from an initial state gives the
    chunked forward's outputs and final state."""
    _need_gpu()
    import ascend_kernel

    b, l, h, p, n, g = 2, 40, 4, 64, 128, 2
    gen = torch.Generator().manual_seed(12)
    x = torch.randn(b, l, h, p, generator=gen).cuda()
    dt = torch.rand(b, l, h, generator=gen).cuda()
    A = -torch.rand(h, generator=gen).cuda()
    Bm = torch.randn(b, l, g, n, generator=gen).cuda()
    Cm = torch.randn(b, l, g, n, generator=gen).cuda()
    D = torch.randn(h, generator=gen).cuda()
    z = torch.randn(b, l, h, p, generator=gen).cuda()
    bias = (torch.randn(h, generator=gen) * 0.1).cuda()
    S0 = torch.randn(b, h, p, n, generator=gen).cuda()
    want, want_final = ascend_kernel.mamba2_ssd_fwd(x, dt, A, Bm, Cm, 64, D=D, z=z, dt_bias=bias,
                                                    dt_softplus=True, initial_states=S0,
                                                    return_final_state=True)
    state = S0.clone()
    outs = []
    for t in range(l):
        outs.append(ascend_kernel.selective_state_update(
            state, x[:, t], dt[:, t, :, None].expand(b, h, p), A[:, None, None].expand(h, p, n),
            Bm[:, t], Cm[:, t], D=D[:, None].expand(h, p), z=z[:, t],
            dt_bias=bias[:, None].expand(h, p), dt_softplus=True))
    got = torch.stack(outs, dim=1)
    torch.cuda.synchronize()
    ma, rl = parity_metrics(got.cpu(), want.cpu())
    sa, sl = parity_metrics(state.cpu(), want_final.cpu())
    _say(f"decode loop vs chunked forward: out relL2 {rl:.3e}, final relL2 {sl:.3e}")
    assert rl <= 5e-5 and sl <= 5e-5, (rl, sl)


def test_decode_strided_views_match_contiguous():
    """Serving-style inputs: x, B, C views into one projection output (batch
    stride = its width), z a slice of another, dt / A / D / dt_bias broadcast
    with stride 0.  The kernel reads them in place; the result equals the call
    on contiguous copies and the oracle."""
    _need_gpu()
    from ascend_kernel import selective_state_update

    b, h, p, n, g = 6, 8, 64, 128, 2
    gen = torch.Generator().manual_seed(21)
    width = h * p + 2 * g * n + 12                       # an extra 12 columns (e.g. dt)
    xbc = torch.randn(b, width, generator=gen).cuda()
    zx = torch.randn(b, 2 * h * p, generator=gen).cuda()
    x = xbc[:, : h * p].view(b, h, p)
    Bm = xbc[:, h * p: h * p + g * n].view(b, g, n)
    Cm = xbc[:, h * p + g * n: h * p + 2 * g * n].view(b, g, n)
    z = zx[:, h * p:].view(b, h, p)
    dt_h = torch.rand(b, h, generator=gen).cuda()
    A_h = -torch.rand(h, generator=gen).cuda()
    D_h = torch.randn(h, generator=gen).cuda()
    bias_h = (torch.randn(h, generator=gen) * 0.1).cuda()
    dt = dt_h[..., None].expand(b, h, p)
    A = A_h[:, None, None].expand(h, p, n)
    D = D_h[:, None].expand(h, p)
    bias = bias_h[:, None].expand(h, p)
    state0 = torch.randn(b, h, p, n, generator=gen).cuda()
    assert x.stride(0) == width and Bm.stride(0) == width and dt.stride(-1) == 0

    s1, s2 = state0.clone(), state0.clone()
    got = selective_state_update(s1, x, dt, A, Bm, Cm, D=D, z=z, dt_bias=bias, dt_softplus=True)
    want = selective_state_update(s2, x.contiguous(), dt.contiguous(), A.contiguous(), Bm.contiguous(),
                                  Cm.contiguous(), D=D.contiguous(), z=z.contiguous(),
                                  dt_bias=bias.contiguous(), dt_softplus=True)
    torch.cuda.synchronize()
    assert torch.allclose(got, want, rtol=1e-6, atol=1e-6)
    assert torch.allclose(s1, s2, rtol=1e-6, atol=1e-6)
    ref_state = state0.double().cpu()
    ref = selective_state_update_ref(ref_state, x.double().cpu(), dt.double().cpu(), A.double().cpu(),
                                     Bm.double().cpu(), Cm.double().cpu(), D=D.double().cpu(),
                                     z=z.double().cpu(), dt_bias=bias.double().cpu(), dt_softplus=True)
    _, rl = parity_metrics(got.cpu(), ref)
    _, sl = parity_metrics(s1.cpu(), ref_state)
    assert rl <= 1e-5 and sl <= 1e-5, (rl, sl)


def test_decode_c_abi_default_layout():
    """The C ABI without MAMBA2_SSU_STRIDES reads every input in the
    contiguous layout of its shape (tied form: dt [B, H], A [H], D [H])."""
    _need_gpu()
    import ctypes

    from ascend_kernel import _runtime as rt
    from ascend_kernel import selective_state_update

    b, h, p, n, g = 3, 4, 64, 64, 2
    gen = torch.Generator().manual_seed(22)
    r = lambda *s: torch.randn(*s, generator=gen).cuda()  # noqa: E731
    x, Bm, Cm, z = r(b, h, p), r(b, g, n), r(b, g, n), r(b, h, p)
    dt_h, A_h, D_h = torch.rand(b, h, generator=gen).cuda(), -torch.rand(h, generator=gen).cuda(), r(h)
    state0 = r(b, h, p, n)
    s1, s2 = state0.clone(), state0.clone()
    out = torch.empty(b, h, p, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    flags = rt.SSU_TIED | rt.DT_SOFTPLUS | rt.HAS_D | rt.HAS_Z
    args = rt.Mamba2SsuArgs(b, h, p, n, g, flags, P(s1), b, h * p * n, None,
                            P(x), P(dt_h), P(A_h), P(Bm), P(Cm), P(D_h), P(z), None, P(out))
    lib = rt.load_library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rt.check(lib.mamba2_selective_state_update(ctypes.byref(args), stream), "ssu", lib)
    want = selective_state_update(s2, x, dt_h[..., None].expand(b, h, p), A_h[:, None, None].expand(h, p, n),
                                  Bm, Cm, D=D_h[:, None].expand(h, p), z=z, dt_softplus=True)
    torch.cuda.synchronize()
    assert torch.allclose(out, want, rtol=1e-6, atol=1e-6)
    assert torch.allclose(s1, s2, rtol=1e-6, atol=1e-6)
