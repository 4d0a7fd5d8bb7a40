"""Pins for the CPU oracle (oracle/ssd_reference.py and oracle/ssd_seq.c).

The first group mirrors the reference's CPU oracle tests
(tests/mamba2/test_reference.py:13-319); the rest pin the restatement against
an independent float64 C recurrence, closed forms, partition invariance and
finite differences, so that a dropped term, a wrong sign or a shifted index in
either oracle fails at least one test.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle.ssd_reference import (
    discretize,
    make_inputs,
    segsum,
    ssd_chunk_scan_ref,
    ssd_chunked_core,
    ssd_sequential_ref,
    selective_state_update_ref,
)
from oracle.ssd_seq import seq_bwd, seq_fwd

F64 = torch.float64


def _inputs(b, l, h, p, n, g, seed=0, dtype=F64, features=()):
    inp = make_inputs([b, l, h, p, n, 8, g], seed, dtype=dtype, features=features)
    inp["dt"] = 0.1 + 0.9 * inp["dt"]
    return inp


# --------------------------------------------------------------------------- segsum

def test_segsum_known_answer():
    s = segsum(torch.tensor([1.0, 2.0, 3.0], dtype=F64))
    inf = float("-inf")
    expected = torch.tensor([[0.0, inf, inf], [2.0, 0.0, inf], [5.0, 3.0, 0.0]], dtype=F64)
    assert torch.equal(s, expected)
    L = torch.exp(s)
    assert L[0, 1] == 0 and L[0, 2] == 0 and L[1, 2] == 0
    assert math.isclose(L[2, 0].item(), math.exp(5.0))


def test_segsum_matches_double_loop():
    v = torch.randn(2, 3, 9, dtype=F64)
    s = segsum(v)
    for i in range(9):
        for j in range(9):
            if i < j:
                assert torch.isinf(s[..., i, j]).all() and (s[..., i, j] < 0).all()
            else:
                ref = v[..., j + 1 : i + 1].sum(-1)
                assert torch.allclose(s[..., i, j], ref, atol=1e-12)


# --------------------------------------------------------------------------- forward pins

def test_core_vs_sequential_fp32():
    """_ssd_core-style chunked math equals the token recurrence (fp32, 1e-3)."""
    b, l, h, p, n, T = 1, 32, 2, 4, 8, 8
    A = torch.full((h,), math.log(0.5))
    q = 0.1 + 0.1 * torch.rand(b, l, h)
    x = torch.randn(b, l, h, p)
    Bh = torch.randn(b, l, h, n)
    Ch = torch.randn(b, l, h, n)
    y, final = ssd_chunked_core(x * q[..., None], q * A, Bh, Ch, T)
    S = torch.zeros(b, h, p, n)
    for t in range(l):
        S = torch.exp(q[:, t] * A)[..., None, None] * S + (x[:, t] * q[:, t, :, None])[..., None] * Bh[:, t, :, None, :]
        yt = (S * Ch[:, t, :, None, :]).sum(-1)
        assert (y[:, t] - yt).abs().max() < 1e-3
    assert (final - S).abs().max() < 1e-3


@pytest.mark.parametrize(
    "features,g,softplus,limit",
    [
        ((), 1, True, (0.0, float("inf"))),
        ((), 2, False, (0.0, float("inf"))),
        (("D", "z", "bias"), 2, True, (0.0, float("inf"))),
        (("D2", "init"), 1, True, (0.0, float("inf"))),
        (("D2", "z", "bias", "init"), 2, True, (0.4, 0.9)),
        (("bias",), 4, False, (-0.2, 0.3)),
    ],
)
def test_chunked_vs_c_fp64(features, g, softplus, limit):
    """Torch restatement (fp64) == independent C float64 recurrence."""
    inp = _inputs(2, 37, 4, 8, 6, g, seed=3, features=features)
    kw = dict(
        D=inp.get("D"), z=inp.get("z"), dt_bias=inp.get("dt_bias"),
        dt_softplus=softplus, dt_limit=limit, initial_states=inp.get("initial_states"),
    )
    y, fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], 8,
                                return_final_state=True, compute_dtype=F64, **kw)
    yc, fc = seq_fwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], **kw)
    assert torch.allclose(y, yc, atol=1e-10, rtol=1e-10)
    assert torch.allclose(fin, fc, atol=1e-10, rtol=1e-10)
    ys, fs = ssd_sequential_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                                return_final_state=True, **kw)
    assert torch.allclose(ys, yc, atol=1e-10, rtol=1e-10)
    assert torch.allclose(fs, fc, atol=1e-10, rtol=1e-10)


def test_partition_invariance():
    inp = _inputs(1, 48, 2, 4, 8, 1, seed=5, features=("init",))
    outs = [
        ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], T,
                           dt_softplus=True, initial_states=inp["initial_states"],
                           return_final_state=True, compute_dtype=F64)
        for T in (1, 3, 8, 16, 48, 64)
    ]
    for y, f in outs[1:]:
        assert torch.allclose(y, outs[0][0], atol=1e-10)
        assert torch.allclose(f, outs[0][1], atol=1e-10)


def test_closed_form_B_zero():
    """B == 0 and no initial state: the SSD term vanishes, y = D x silu(z)."""
    inp = _inputs(2, 20, 4, 8, 6, 2, seed=7, features=("D2", "z"))
    y = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], torch.zeros_like(inp["B"]), inp["C"], 8,
                           D=inp["D"], z=inp["z"], dt_softplus=True, compute_dtype=F64)
    ref = inp["x"] * inp["D"][None, None] * F.silu(inp["z"])
    assert torch.allclose(y, ref, atol=1e-12)


def test_closed_form_A_zero():
    """A == 0: y_t = sum_{s<=t} (C_t . B_s) q_s x_s (pure causal prefix sum)."""
    inp = _inputs(1, 24, 2, 4, 5, 1, seed=9)
    A = torch.zeros(2, dtype=F64)
    y, fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], A, inp["B"], inp["C"], 8,
                                dt_softplus=True, return_final_state=True, compute_dtype=F64)
    q = F.softplus(inp["dt"])
    xdt = inp["x"] * q[..., None]
    CB = torch.einsum("bln,bsn->bls", inp["C"][:, :, 0], inp["B"][:, :, 0])
    mask = torch.ones(24, 24, dtype=torch.bool).tril()
    ref = torch.einsum("bls,bshp->blhp", CB * mask, xdt)
    assert torch.allclose(y, ref, atol=1e-10)
    ref_fin = torch.einsum("bshp,bsn->bhpn", xdt, inp["B"][:, :, 0])
    assert torch.allclose(fin, ref_fin, atol=1e-10)


def test_closed_form_single_token():
    """L == 1 with initial state: y = exp(Aq) init.C + q x (B.C)."""
    inp = _inputs(2, 1, 2, 4, 5, 1, seed=11, features=("init",))
    y, fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], 4,
                                dt_softplus=True, initial_states=inp["initial_states"],
                                return_final_state=True, compute_dtype=F64)
    q = F.softplus(inp["dt"])[:, 0]  # [b, h]
    decay = torch.exp(q * inp["A"])
    bc = (inp["B"][:, 0, 0] * inp["C"][:, 0, 0]).sum(-1)  # [b]
    init_c = torch.einsum("bhpn,bn->bhp", inp["initial_states"], inp["C"][:, 0, 0])
    ref = decay[..., None] * init_c + q[..., None] * inp["x"][:, 0] * bc[:, None, None]
    assert torch.allclose(y[:, 0], ref, atol=1e-12)
    ref_fin = decay[..., None, None] * inp["initial_states"] + (q[..., None] * inp["x"][:, 0])[..., None] * inp["B"][:, 0, 0][:, None, None, :]
    assert torch.allclose(fin, ref_fin, atol=1e-12)


def test_clamp_applies_without_softplus():
    dt = torch.tensor([[[-1.0, 0.5, 3.0]]], dtype=F64)
    q = discretize(dt, None, False, (0.0, 1.0))
    assert q.tolist() == [[[0.0, 0.5, 1.0]]]
    q2 = discretize(dt, torch.tensor([0.0, 0.0, -2.5], dtype=F64), True, (0.0, float("inf")))
    assert torch.allclose(q2, F.softplus(torch.tensor([[[-1.0, 0.5, 0.5]]], dtype=F64)))


def test_padding_tail_and_final_state():
    """L not a multiple of the chunk: output trimmed, final state = state after L."""
    inp = _inputs(2, 30, 2, 4, 8, 1, seed=13)
    y, fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], 7,
                                dt_softplus=True, return_final_state=True, compute_dtype=F64)
    yc, fc = seq_fwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], dt_softplus=True)
    assert y.shape == (2, 30, 2, 4)
    assert torch.allclose(y, yc, atol=1e-10) and torch.allclose(fin, fc, atol=1e-10)


def test_dtype_preservation_and_fp32_final():
    inp = _inputs(1, 16, 2, 4, 8, 1, seed=1, dtype=torch.bfloat16)
    out, fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"].float(), inp["B"], inp["C"], 8,
                                  dt_softplus=True, return_final_state=True)
    assert out.dtype == torch.bfloat16 and fin.dtype == torch.float32
    assert fin.shape == (1, 2, 4, 8)


def test_shape_errors():
    inp = _inputs(1, 8, 3, 4, 4, 2, seed=1)
    with pytest.raises(ValueError):
        ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], 4)


# --------------------------------------------------------------------------- backward pins

def _loss_grads_torch(inp, features, softplus, limit, T=8):
    leaves = {k: v.clone().requires_grad_(True) for k, v in inp.items()}
    y, fin = ssd_chunk_scan_ref(
        leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], T,
        D=leaves.get("D"), z=leaves.get("z"), dt_bias=leaves.get("dt_bias"),
        dt_softplus=softplus, dt_limit=limit, initial_states=leaves.get("initial_states"),
        return_final_state=True, compute_dtype=F64,
    )
    gy = torch.linspace(-1, 1, y.numel(), dtype=F64).reshape(y.shape)
    gf = torch.linspace(0.5, -0.5, fin.numel(), dtype=F64).reshape(fin.shape)
    (y * gy).sum().backward(inputs=list(leaves.values()), retain_graph=True)
    (fin * gf).sum().backward(inputs=list(leaves.values()))
    return {k: v.grad for k, v in leaves.items()}, gy, gf


@pytest.mark.parametrize(
    "features,g,softplus,limit",
    [
        ((), 2, True, (0.0, float("inf"))),
        (("D", "z", "bias", "init"), 2, True, (0.0, float("inf"))),
        (("D2", "bias"), 1, True, (0.5, 0.9)),
        (("z",), 4, False, (-0.2, 0.3)),
    ],
)
def test_backward_autograd_vs_c_adjoint(features, g, softplus, limit):
    inp = _inputs(2, 21, 4, 4, 5, g, seed=17, features=features)
    tg, gy, gf = _loss_grads_torch(inp, features, softplus, limit)
    cg = seq_bwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], gy, gf,
                 D=inp.get("D"), z=inp.get("z"), dt_bias=inp.get("dt_bias"),
                 dt_softplus=softplus, dt_limit=limit,
                 initial_states=inp.get("initial_states"))
    names = {"x": "dx", "dt": "ddt", "A": "dA", "B": "dB", "C": "dC", "D": "dD",
             "z": "dz", "dt_bias": "ddt_bias", "initial_states": "dinitial"}
    for k, g_t in tg.items():
        assert torch.allclose(g_t, cg[names[k]], atol=1e-9, rtol=1e-9), k


def test_c_adjoint_finite_differences():
    """Directional derivative of the C forward equals <grad, direction> (fp64)."""
    feats = ("D2", "z", "bias", "init")
    inp = _inputs(1, 9, 2, 3, 4, 1, seed=19, features=feats)
    kw = dict(dt_softplus=True, dt_limit=(0.0, float("inf")))
    gy = torch.randn(1, 9, 2, 3, dtype=F64)
    gf = torch.randn(1, 2, 3, 4, dtype=F64)
    cg = seq_bwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], gy, gf, D=inp["D"], z=inp["z"],
                 dt_bias=inp["dt_bias"], initial_states=inp["initial_states"], **kw)
    names = {"x": "dx", "dt": "ddt", "A": "dA", "B": "dB", "C": "dC", "D": "dD",
             "z": "dz", "dt_bias": "ddt_bias", "initial_states": "dinitial"}
    gen = torch.Generator().manual_seed(23)
    dirs = {k: torch.randn(v.shape, generator=gen, dtype=F64) for k, v in inp.items()}

    def f(eps):
        pert = {k: v + eps * dirs[k] for k, v in inp.items()}
        y, fin = seq_fwd(pert["x"], pert["dt"], pert["A"], pert["B"], pert["C"], D=pert["D"],
                         z=pert["z"], dt_bias=pert["dt_bias"],
                         initial_states=pert["initial_states"], **kw)
        return (y * gy).sum() + (fin * gf).sum()

    eps = 1e-6
    fd = (f(eps) - f(-eps)) / (2 * eps)
    an = sum((cg[names[k]] * dirs[k]).sum() for k in inp)
    assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (fd.item(), an.item())


def test_planted_index_shift_is_caught():
    """A plausible oracle mistake (decaying the entering state by exp(cs_{t-1})
    instead of exp(cs_t)) must fail the sequential comparison."""
    inp = _inputs(1, 16, 2, 4, 4, 1, seed=29, features=("init",))
    q = F.softplus(inp["dt"])
    xdt = inp["x"] * q[..., None]
    dA = q * inp["A"]
    Bh = inp["B"].expand(-1, -1, 2, -1)
    Ch = inp["C"].expand(-1, -1, 2, -1)
    y_good, _ = ssd_chunked_core(xdt, dA, Bh, Ch, 8, inp["initial_states"])
    # planted: shift dA by one position inside each chunk
    dA_bad = dA.clone()
    dA_bad[:, 1:] = dA[:, :-1]
    y_bad, _ = ssd_chunked_core(xdt, dA_bad, Bh, Ch, 8, inp["initial_states"])
    yc, _ = seq_fwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], dt_softplus=True,
                    initial_states=inp["initial_states"])
    assert torch.allclose(y_good, yc, atol=1e-10)
    assert not torch.allclose(y_bad, yc, atol=1e-3)


def test_autograd_finite_reference_style():
    """Reference-style smoke (tests/mamba2/test_reference.py:299-319)."""
    inp = _inputs(1, 16, 2, 4, 8, 1, seed=31, dtype=torch.float32)
    leaves = {k: v.clone().requires_grad_(True) for k, v in inp.items()}
    out = ssd_chunk_scan_ref(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], 8,
                             dt_softplus=True)
    out.sum().backward()
    for k, v in leaves.items():
        assert v.grad is not None and torch.isfinite(v.grad).all(), k


# ----------------------------------------------------------------------------- decode step

def test_decode_steps_equal_sequential_recurrence():
    """L tied decode steps from an initial state reproduce the token-by-token
    recurrence (output of every token and the final state)."""
    b, l, h, p, n, g = 2, 5, 4, 3, 8, 2
    gen = torch.Generator().manual_seed(31)
    x = torch.randn(b, l, h, p, generator=gen, dtype=torch.float64)
    dt = torch.rand(b, l, h, generator=gen, dtype=torch.float64)
    A = -torch.rand(h, generator=gen, dtype=torch.float64)
    B = torch.randn(b, l, g, n, generator=gen, dtype=torch.float64)
    C = torch.randn(b, l, g, n, generator=gen, dtype=torch.float64)
    D = torch.randn(h, generator=gen, dtype=torch.float64)
    z = torch.randn(b, l, h, p, generator=gen, dtype=torch.float64)
    bias = torch.randn(h, generator=gen, dtype=torch.float64) * 0.1
    S0 = torch.randn(b, h, p, n, generator=gen, dtype=torch.float64)
    want, want_final = ssd_sequential_ref(x, dt, A, B, C, D=D, z=z, dt_bias=bias, dt_softplus=True,
                                          initial_states=S0.clone(), return_final_state=True)
    state = S0.clone()
    A3 = A[:, None, None].expand(h, p, n)
    for t in range(l):
        out = selective_state_update_ref(state, x[:, t], dt[:, t, :, None].expand(b, h, p), A3,
                                         B[:, t], C[:, t], D=D[:, None].expand(h, p), z=z[:, t],
                                         dt_bias=bias[:, None].expand(h, p), dt_softplus=True)
        torch.testing.assert_close(out, want[:, t], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(state, want_final, rtol=1e-12, atol=1e-12)


def test_decode_untied_matches_element_loop():
    """Per-(head, dim) dt and per-element A against a direct loop over every
    state element."""
    b, h, p, n, g = 2, 2, 3, 4, 1
    gen = torch.Generator().manual_seed(32)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)  # noqa: E731
    x, dt, A, B, C, D, z = r(b, h, p), r(b, h, p), -r(h, p, n).abs(), r(b, g, n), r(b, g, n), r(h, p), r(b, h, p)
    bias = r(h, p)
    S0 = r(b, h, p, n)
    state = S0.clone()
    out = selective_state_update_ref(state, x, dt, A, B, C, D=D, z=z, dt_bias=bias, dt_softplus=True)
    for bi in range(b):
        for hi in range(h):
            for pi in range(p):
                u = float(dt[bi, hi, pi] + bias[hi, pi])
                q = u if u > 20 else math.log1p(math.exp(u))
                acc = 0.0
                for ni in range(n):
                    s = math.exp(q * float(A[hi, pi, ni])) * float(S0[bi, hi, pi, ni]) + \
                        q * float(x[bi, hi, pi]) * float(B[bi, 0, ni])
                    assert abs(s - float(state[bi, hi, pi, ni])) < 1e-12
                    acc += s * float(C[bi, 0, ni])
                acc += float(D[hi, pi]) * float(x[bi, hi, pi])
                zz = float(z[bi, hi, pi])
                acc *= zz / (1.0 + math.exp(-zz))
                assert abs(acc - float(out[bi, hi, pi])) < 1e-10


def test_decode_padding_slots():
    """A negative slot leaves the state alone and outputs zeros; the other
    sequences update their own slots."""
    b, h, p, n = 3, 2, 2, 4
    gen = torch.Generator().manual_seed(33)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)  # noqa: E731
    state = r(4, h, p, n)
    before = state.clone()
    idx = torch.tensor([2, -1, 0])
    out = selective_state_update_ref(state, r(b, h, p), torch.rand(b, h, p, dtype=torch.float64),
                                     -torch.rand(h, p, n, dtype=torch.float64), r(b, 1, n), r(b, 1, n),
                                     state_batch_indices=idx)
    assert torch.equal(out[1], torch.zeros(h, p, dtype=torch.float64))
    assert torch.equal(state[1], before[1]) and torch.equal(state[3], before[3])
    assert not torch.equal(state[2], before[2]) and not torch.equal(state[0], before[0])


# ----------------------------------------------------------------------------- packed sequences

def _ids_from_lengths(lengths, first=0):
    return torch.cat([torch.full((n,), first + i, dtype=torch.int64) for i, n in enumerate(lengths)])


@pytest.mark.parametrize("chunk", [8, 16, 32])
def test_seq_idx_all_equal_is_unmasked(chunk):
    inp = _inputs(2, 40, 4, 3, 5, 2, seed=41, features=("D", "init"))
    ids = torch.zeros(2, 40, dtype=torch.int64)
    y0, f0 = ssd_chunk_scan_ref(**inp, chunk_size=chunk, dt_softplus=True, return_final_state=True,
                                compute_dtype=F64)
    y1, f1 = ssd_chunk_scan_ref(**inp, chunk_size=chunk, dt_softplus=True, return_final_state=True,
                                compute_dtype=F64, seq_idx=ids)
    torch.testing.assert_close(y1, y0, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(f1, f0, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("chunk", [8, 16, 32])
def test_seq_idx_packed_equals_separate_runs(chunk):
    """Non-decreasing ids: every token's output equals that of its sequence
    run alone (the first sequence, id 0, from the initial state), and the
    final state is the last sequence's; boundaries inside chunks, on chunk
    edges, a one-token sequence and one spanning several chunks."""
    lengths = [5, 11, 1, 16, 3, 21, 7]
    L = sum(lengths)
    inp = _inputs(1, L, 4, 3, 5, 2, seed=42, features=("D2", "z", "bias", "init"))
    ids = _ids_from_lengths(lengths)[None]
    y, fin = ssd_chunk_scan_ref(**inp, chunk_size=chunk, dt_softplus=True, return_final_state=True,
                                compute_dtype=F64, seq_idx=ids)
    t0 = 0
    for i, n in enumerate(lengths):
        part = {k: (v[:, t0:t0 + n] if k in ("x", "dt", "B", "C", "z") else v) for k, v in inp.items()}
        part["initial_states"] = inp["initial_states"] if i == 0 else None
        want, want_fin = ssd_sequential_ref(**part, dt_softplus=True, return_final_state=True)
        torch.testing.assert_close(y[:, t0:t0 + n], want, rtol=1e-10, atol=1e-10)
        t0 += n
    torch.testing.assert_close(fin, want_fin, rtol=1e-10, atol=1e-10)


def test_seq_idx_first_sequence_not_zero_drops_initial_state():
    lengths = [9, 12]
    inp = _inputs(1, 21, 2, 3, 4, 1, seed=43, features=("init",))
    ids = _ids_from_lengths(lengths, first=3)[None]
    y, fin = ssd_chunk_scan_ref(**inp, chunk_size=8, dt_softplus=True, return_final_state=True,
                                compute_dtype=F64, seq_idx=ids)
    part = {k: (v[:, :9] if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}
    part["initial_states"] = None
    torch.testing.assert_close(y[:, :9], ssd_sequential_ref(**part, dt_softplus=True),
                               rtol=1e-10, atol=1e-10)


def test_seq_idx_interleaved_in_one_chunk():
    """Ids interleaved inside one chunk: the tokens of id X see the other
    tokens of id X (decayed through every token in between) and nothing else,
    which is the sequential recurrence over the chunk with the x of the other
    ids zeroed."""
    L = 16
    inp = _inputs(1, L, 2, 3, 4, 1, seed=44)
    ids = torch.tensor([[0, 0, 1, 1, 1, 0, 0, 2, 2, 1, 0, 0, 2, 1, 1, 0]])
    y = ssd_chunk_scan_ref(**inp, chunk_size=L, dt_softplus=True, compute_dtype=F64, seq_idx=ids)
    for v in (0, 1, 2):
        sel = ids[0] == v
        part = dict(inp)
        part["x"] = inp["x"] * sel[None, :, None, None].to(F64)
        want = ssd_sequential_ref(**part, dt_softplus=True)
        torch.testing.assert_close(y[:, sel], want[:, sel], rtol=1e-10, atol=1e-10)


def test_seq_idx_negative_ids_are_padding():
    """All-negative ids: no chunk enters the state and the initial state is
    dropped, so the final state is zero and every chunk runs on its own."""
    T, L = 8, 24
    inp = _inputs(1, L, 2, 3, 4, 1, seed=45, features=("init",))
    ids = torch.full((1, L), -1)
    y, fin = ssd_chunk_scan_ref(**inp, chunk_size=T, dt_softplus=True, return_final_state=True,
                                compute_dtype=F64, seq_idx=ids)
    assert torch.equal(fin, torch.zeros_like(fin))
    for c in range(L // T):
        part = {k: (v[:, c * T:(c + 1) * T] if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}
        part["initial_states"] = None
        torch.testing.assert_close(y[:, c * T:(c + 1) * T], ssd_sequential_ref(**part, dt_softplus=True),
                                   rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("chunk", [8, 16])
def test_varlen_states_equal_separate_final_states(chunk):
    """chunk_state_varlen: the state at the end of every packed sequence is
    that sequence's final state run alone (a sequence starting on a chunk
    edge, one spanning several chunks, one token long, one ending the input
    mid-chunk)."""
    from oracle.ssd_reference import chunk_state_varlen_ref

    lengths = [5, 11, 16, 1, 20, 6]
    L = sum(lengths)
    inp = _inputs(1, L, 4, 3, 5, 2, seed=46, features=("bias",))
    ids = _ids_from_lengths(lengths)[None]
    cu = torch.tensor([0] + list(torch.tensor(lengths).cumsum(0)))
    _, states = ssd_chunk_scan_ref(**inp, chunk_size=chunk, dt_softplus=True, compute_dtype=F64,
                                   seq_idx=ids, return_chunk_states=True)
    got = chunk_state_varlen_ref(inp["x"], inp["dt"], inp["A"], inp["B"], chunk, cu, states,
                                 dt_bias=inp["dt_bias"], dt_softplus=True)
    assert got.shape == (len(lengths), 4, 3, 5)
    t0 = 0
    for i, n in enumerate(lengths):
        part = {k: (v[:, t0:t0 + n] if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}
        _, fin = ssd_sequential_ref(**part, dt_softplus=True, return_final_state=True)
        torch.testing.assert_close(got[i], fin[0], rtol=1e-10, atol=1e-10)
        t0 += n


@pytest.mark.parametrize("first_len,keeps_init", [(5, False), (11, True)])
def test_varlen_states_initial_state_only_through_chunk_states(first_len, keeps_init):
    """chunk_state_varlen adds the initial state only through chunk_states,
    i.e. only when the first sequence runs past the first chunk (chunk 8: a
    5-token first sequence ends without it, an 11-token one with it)."""
    from oracle.ssd_reference import chunk_state_varlen_ref

    lengths = [first_len, 7]
    L = sum(lengths)
    inp = _inputs(1, L, 2, 3, 4, 1, seed=47, features=("init",))
    ids = _ids_from_lengths(lengths)[None]
    cu = torch.tensor([0, first_len, L])
    _, states = ssd_chunk_scan_ref(**inp, chunk_size=8, dt_softplus=True, compute_dtype=F64,
                                   seq_idx=ids, return_chunk_states=True)
    got = chunk_state_varlen_ref(inp["x"], inp["dt"], inp["A"], inp["B"], 8, cu, states,
                                 dt_softplus=True)
    part = {k: (v[:, :first_len] if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}
    part["initial_states"] = inp["initial_states"] if keeps_init else None
    _, fin = ssd_sequential_ref(**part, dt_softplus=True, return_final_state=True)
    torch.testing.assert_close(got[0], fin[0], rtol=1e-10, atol=1e-10)
