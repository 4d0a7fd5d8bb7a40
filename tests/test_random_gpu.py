"""Seeded randomized GPU parity sweep of the public API against the oracle.

Each case draws a shape (batch, ragged seqlen, groups and heads per group,
headdim 64 or 128, dstate 64 or 128, logical chunk 32 to 256), a subset of the
features (D per head or per channel, z, dt_bias, initial states, softplus or a
dt_limit clamp) and, for some cases, packed-sequence ids (non-decreasing or
interleaved with padding ids).  The forward (output and final state) is
compared with the float64 oracle; where headdim = dstate = 64 the gradients of
every input through autograd are compared too.  Bounds: relative L2 <= 1e-4
(forward) and <= 2e-4 (gradients) against float64, well inside the contract.

The long cases (400 to 2600 tokens over at most 16 heads) have fewer (b, h)
streams than the GPU has CUs, so they take the segmented forward (state-only
pre-pass folded into each segment's entering state) and the run-split reverse
backward (run pre-pass, recurrence over runs) with the same random features.
"""

import sys

import pytest
import torch

from oracle.ssd_reference import make_inputs, parity_metrics, ssd_chunk_scan_ref

pytestmark = pytest.mark.gpu

NCASES = 24


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _draw(seed, long=False):
    g = torch.Generator().manual_seed((7000 if long else 1000) + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]  # noqa: E731
    b = pick([1, 2]) if long else pick([1, 2, 3])
    l = int(torch.randint(400, 2600, (1,), generator=g)) if long else int(torch.randint(1, 300, (1,), generator=g))
    groups, r = (pick([1, 2]), pick([1, 2, 4])) if long else (pick([1, 2, 4]), pick([1, 2, 4, 8]))
    p, n = pick([64, 64, 128]), pick([64, 64, 128])
    chunk = pick([32, 64, 128, 256])
    feats = tuple(f for f in ("D", "D2", "z", "bias", "init") if bool(torch.rand(1, generator=g) < 0.4))
    if "D" in feats and "D2" in feats:
        feats = tuple(f for f in feats if f != "D")
    softplus = bool(torch.rand(1, generator=g) < 0.7)
    limit = (0.0, float("inf")) if bool(torch.rand(1, generator=g) < 0.6) else (0.05, 0.9)
    seq = pick([None, None, "packed"]) if long else pick([None, None, "packed", "mixed"])
    return [b, l, groups * r, p, n, chunk, groups], feats, softplus, limit, seq


NLONG = 8
CASES = [_draw(i) for i in range(NCASES)] + [_draw(i, long=True) for i in range(NLONG)]


def _ids(kind, b, l, seed):
    g = torch.Generator().manual_seed(2000 + seed)
    if kind == "packed":
        rows = []
        for _ in range(b):
            cuts = sorted(torch.randint(0, l, (3,), generator=g).tolist())
            row = torch.zeros(l, dtype=torch.int32)
            for c in cuts:
                row[c:] += 1
            rows.append(row)
        return torch.stack(rows)
    return torch.randint(-1, 3, (b, l), generator=g, dtype=torch.int32)


@pytest.mark.parametrize("case", range(NCASES + NLONG),
                         ids=[f"{c[0]}-{'+'.join(c[1]) or 'plain'}-{c[4] or 'noseq'}" for c in CASES])
def test_random_case(case):
    _need_gpu()
    import ascend_kernel

    shape, feats, softplus, limit, seq = CASES[case]
    b, l, h, p, n, chunk, groups = shape
    if seq == "mixed":
        chunk = 64  # interleaved ids are defined per 64-token execution chunk
    print(f"random case {case}: {shape} {feats} softplus={softplus} limit={limit} seq={seq}", flush=True)
    sys.stdout.flush()
    inp = make_inputs([b, l, h, p, n, chunk, groups], seed=3000 + case, features=feats)
    ids = None if seq is None else _ids(seq, b, l, case)
    train = p == 64 and n == 64
    gen = torch.Generator().manual_seed(4000 + case)
    gy, gf = torch.randn(b, l, h, p, generator=gen), torch.randn(b, h, p, n, generator=gen)

    def run(on_gpu):
        conv = (lambda t: t.cuda()) if on_gpu else (lambda t: t.double())
        leaves = {k: conv(v).clone().requires_grad_(train) for k, v in inp.items()}
        args = (leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], chunk)
        kw = dict(D=leaves.get("D"), z=leaves.get("z"), dt_bias=leaves.get("dt_bias"),
                  dt_softplus=softplus, dt_limit=limit, initial_states=leaves.get("initial_states"),
                  return_final_state=True)
        if on_gpu:
            out, fin = ascend_kernel.mamba2_ssd_fwd(*args, seq_idx=None if ids is None else ids.cuda(), **kw)
        else:
            out, fin = ssd_chunk_scan_ref(*args, seq_idx=ids, compute_dtype=torch.float64, **kw)
        grads = {}
        if train:
            ((out * conv(gy)).sum() + (fin * conv(gf)).sum()).backward()
            grads = {k: v.grad.detach().cpu() for k, v in leaves.items()}
        if on_gpu:
            torch.cuda.synchronize()
        return out.detach().cpu(), fin.detach().cpu(), grads

    got_y, got_f, got_g = run(True)
    want_y, want_f, want_g = run(False)
    for name, a, e, bound in [("out", got_y, want_y, 1e-4), ("final", got_f, want_f, 1e-4)] + \
            [(f"d{k}", got_g[k], want_g[k], 2e-4) for k in got_g]:
        ma, rl = parity_metrics(a, e)
        print(f"  {name:<16} maxabs {ma:.3e} relL2 {rl:.3e}", flush=True)
        assert torch.isfinite(a).all(), name
        assert rl <= bound, (name, rl)
