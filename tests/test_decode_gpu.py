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
