"""GPU parity of packed sequences (``seq_idx``) and varlen states (``cu_seqlens``).

The HIP forward with per-token sequence ids is checked against the oracle's
``ssd_chunk_scan_ref(..., seq_idx=...)`` (the masks of the reference's Triton
port): non-decreasing ids at the logical chunk size the caller passes (the
result does not depend on it), ids that interleave, repeat and go negative at
chunk 64 (the execution chunk, where the masks are defined per 64 tokens),
dstate 128, the segmented path of few long streams with cuts inside and on
segment edges, and all-equal ids against the unmasked kernel.  The state at
the end of every packed sequence is checked against the oracle's
``chunk_state_varlen_ref`` at logical chunks 64 and 256.  Bar: max-abs <= 2e-2
and relative-L2 <= 5e-3 against the fp32 oracle, plus a tighter relative-L2
that the split-fp16 scheme reaches on these sizes.

The backward with packed sequences is checked against float64 autograd of the
same oracle on each of its three paths (chunk-parallel dSoff with the
elementwise reverse recurrence, the reverse dstate pass, the fused reverse
chunk kernel at 1, 2 and 4 heads per group), at relative-L2 <= 2e-4 for
every gradient.
"""

import sys

import pytest
import torch

from oracle.ssd_reference import (
    chunk_state_varlen_ref,
    make_inputs,
    parity_metrics,
    ssd_chunk_scan_ref,
)

pytestmark = pytest.mark.gpu

MAXABS = 2e-2
RELL2 = 5e-3
TIGHT = 2e-4


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _ids_from_lengths(lengths, first=0):
    return torch.cat([torch.full((n,), first + i, dtype=torch.int32) for i, n in enumerate(lengths)])


def _lengths(total, gen, lo=1, hi=300):
    out = []
    while sum(out) < total:
        out.append(int(torch.randint(lo, hi, (1,), generator=gen)))
    out[-1] -= sum(out) - total
    return [n for n in out if n > 0]


def _run(inp, chunk, seq_idx, **kw):
    import ascend_kernel

    dev = {k: v.cuda() for k, v in inp.items()}
    res = ascend_kernel.mamba2_ssd_fwd(
        dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], chunk, D=dev.get("D"), z=dev.get("z"),
        dt_bias=dev.get("dt_bias"), dt_softplus=True, initial_states=dev.get("initial_states"),
        return_final_state=True, seq_idx=None if seq_idx is None else seq_idx.cuda(), **kw)
    torch.cuda.synchronize()
    return tuple(t.cpu() for t in res)


def _ref(inp, chunk, seq_idx, **kw):
    return ssd_chunk_scan_ref(
        inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], chunk, D=inp.get("D"), z=inp.get("z"),
        dt_bias=inp.get("dt_bias"), dt_softplus=True, initial_states=inp.get("initial_states"),
        return_final_state=True, seq_idx=seq_idx, **kw)


def _check(name, got, want, tight=True):
    ma, rl = parity_metrics(got, want)
    _say(f"  {name}: maxabs {ma:.3e} relL2 {rl:.3e}")
    assert ma <= MAXABS and rl <= RELL2, (name, ma, rl)
    if tight:
        assert rl <= TIGHT, (name, rl)


PACKED = [
    # shape [B, L, H, P, N, chunk, G], features, seed
    ([2, 700, 8, 64, 64, 64, 2], ("D2", "z", "bias", "init"), 1),
    ([2, 700, 8, 64, 64, 256, 2], ("D", "bias", "init"), 2),
    ([1, 1000, 4, 64, 128, 128, 1], ("z", "init"), 3),
    ([3, 333, 4, 64, 128, 64, 4], ("D2", "bias"), 4),
    ([2, 300, 4, 128, 64, 64, 2], ("D", "z", "init"), 5),   # headdim 128 (two heads of 64)
]


@pytest.mark.parametrize("shape,features,seed", PACKED,
                         ids=[f"{'x'.join(map(str, c[0]))}-{'+'.join(c[1])}" for c in PACKED])
def test_packed_sequences_match_oracle(shape, features, seed):
    """Non-decreasing ids (random lengths, one sequence per row starting at
    id 0 so the initial state applies to it) at the caller's chunk size."""
    _need_gpu()
    b, l = shape[0], shape[1]
    _say(f"packed sequences {shape} {features}")
    inp = make_inputs(shape, seed=300 + seed, features=features)
    gen = torch.Generator().manual_seed(seed)
    ids = torch.stack([_ids_from_lengths(_lengths(l, gen)) for _ in range(b)])
    got_y, got_f = _run(inp, shape[5], ids)
    want_y, want_f = _ref(inp, shape[5], ids)
    _check("out", got_y, want_y)
    _check("final", got_f, want_f)


def test_interleaved_and_negative_ids_at_chunk_64():
    """Ids that come back, repeat across chunk edges and go negative, at the
    64-token execution chunk."""
    _need_gpu()
    shape = [2, 400, 4, 64, 64, 64, 2]
    _say(f"interleaved / negative ids {shape}")
    inp = make_inputs(shape, seed=311, features=("D", "z", "bias", "init"))
    gen = torch.Generator().manual_seed(5)
    ids = torch.randint(-1, 3, (2, 400), generator=gen, dtype=torch.int32)
    ids[0, 64:128] = -1                  # a whole padding chunk
    ids[1, :130] = 0                     # the initial state carried over two chunk edges
    got_y, got_f = _run(inp, 64, ids)
    want_y, want_f = _ref(inp, 64, ids)
    _check("out", got_y, want_y)
    _check("final", got_f, want_f)


def test_segmented_streams_with_cuts():
    """Few long streams run as several segments per stream (the segment
    recurrence between them; here 8 streams of 300 chunks: full segments of 10
    chunks, state-only pre-segments of 5): sequences cut inside segments, on a
    full-segment edge (token 1920), on a pre-segment edge inside a full segment
    (token 7360), and one sequence spanning several segments."""
    _need_gpu()
    shape = [1, 19200, 8, 64, 64, 64, 8]
    _say(f"segmented packed {shape}")
    inp = make_inputs(shape, seed=312, features=("bias", "init"))
    lengths = [100, 92, 1728, 5000, 1, 439, 19200 - 7360]
    ids = _ids_from_lengths(lengths)[None]
    got_y, got_f = _run(inp, 64, ids)
    want_y, want_f = _ref(inp, 64, ids)
    _check("out", got_y, want_y)
    _check("final", got_f, want_f)


def test_all_equal_ids_match_unmasked_forward():
    _need_gpu()
    shape = [2, 300, 4, 64, 64, 64, 2]
    inp = make_inputs(shape, seed=313, features=("D", "z", "init"))
    y0, f0 = _run(inp, 64, None)
    y1, f1 = _run(inp, 64, torch.zeros(2, 300, dtype=torch.int32))
    assert torch.allclose(y1, y0, rtol=1e-6, atol=1e-6)
    assert torch.allclose(f1, f0, rtol=1e-6, atol=1e-6)


VARLEN = [
    # L, H, N, G, logical chunk, seed
    (900, 8, 64, 2, 64, 1),
    (900, 8, 64, 2, 256, 2),
    (1500, 4, 128, 1, 128, 3),
]


@pytest.mark.parametrize("l,h,n,g,chunk,seed", VARLEN,
                         ids=[f"L{c[0]}h{c[1]}n{c[2]}g{c[3]}c{c[4]}" for c in VARLEN])
def test_varlen_states_match_oracle(l, h, n, g, chunk, seed):
    """State at the end of every sequence of a packed batch-1 input, with
    seq_idx from the same cu_seqlens (a one-token sequence, one on a chunk
    edge, one spanning several chunks)."""
    _need_gpu()
    shape = [1, l, h, 64, n, chunk, g]
    _say(f"varlen states {shape}")
    inp = make_inputs(shape, seed=320 + seed, features=("D", "bias", "init"))
    gen = torch.Generator().manual_seed(seed)
    lengths = [1, 63, 64] + _lengths(l - 128, gen, hi=400)
    ids = _ids_from_lengths(lengths)[None]
    cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32)
    got_y, got_f, got_v = _run(inp, chunk, ids, cu_seqlens=cu.cuda(), return_varlen_states=True)
    want_y, want_f, states = _ref(inp, chunk, ids, return_chunk_states=True)
    want_v = chunk_state_varlen_ref(inp["x"], inp["dt"], inp["A"], inp["B"], chunk, cu, states,
                                    dt_bias=inp["dt_bias"], dt_softplus=True)
    assert got_v.shape == (len(lengths), h, 64, n)
    _check("out", got_y, want_y)
    _check("final", got_f, want_f)
    _check("varlen states", got_v, want_v)


def test_varlen_return_conventions():
    """(out, varlen) without the final state, (out, final, varlen) with it,
    and the port's return_final_states spelling."""
    _need_gpu()
    import ascend_kernel

    inp = make_inputs([1, 200, 2, 64, 64, 64, 1], seed=330)
    dev = {k: v.cuda() for k, v in inp.items()}
    cu = torch.tensor([0, 70, 200], dtype=torch.int32, device="cuda")
    ids = torch.cat([torch.zeros(70), torch.ones(130)]).to(torch.int32)[None].cuda()
    args = (dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], 64)
    two = ascend_kernel.mamba2_ssd_fwd(*args, seq_idx=ids, cu_seqlens=cu, return_varlen_states=True)
    three = ascend_kernel.mamba_chunk_scan_combined(*args, seq_idx=ids, cu_seqlens=cu,
                                                    return_varlen_states=True, return_final_states=True)
    torch.cuda.synchronize()
    assert len(two) == 2 and len(three) == 3
    assert two[1].shape == (2, 2, 64, 64)
    assert torch.equal(two[0], three[0]) and torch.equal(two[1], three[2])
    # the last sequence's varlen state is the final state
    assert torch.allclose(three[2][1], three[1][0], rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------------------------- backward

def _grads(inp, chunk, ids, gy, gf, on_gpu):
    import ascend_kernel

    dev = (lambda t: t.cuda()) if on_gpu else (lambda t: t.to(torch.float64))
    leaves = {k: dev(v).clone().requires_grad_(True) for k, v in inp.items()}
    fn = ascend_kernel.mamba2_ssd_fwd if on_gpu else None
    kw = dict(D=leaves.get("D"), z=leaves.get("z"), dt_bias=leaves.get("dt_bias"), dt_softplus=True,
              initial_states=leaves.get("initial_states"), return_final_state=True)
    args = (leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], chunk)
    if on_gpu:
        out, fin = fn(*args, seq_idx=ids.cuda(), **kw)
    else:
        out, fin = ssd_chunk_scan_ref(*args, seq_idx=ids, compute_dtype=torch.float64, **kw)
    ((out * dev(gy)).sum() + (fin * dev(gf)).sum()).backward()
    if on_gpu:
        torch.cuda.synchronize()
    return {k: v.grad.cpu() for k, v in leaves.items()}


BWD = [
    # shape [B, L, H, P, N, chunk, G], features, ids ("packed" or "mixed"), path exercised
    ([2, 200, 4, 64, 64, 64, 2], ("D", "z", "bias", "init"), "mixed"),      # reverse runs of 1 chunk
    ([2, 330, 8, 64, 64, 256, 8], ("D2", "bias", "init"), "packed"),         # reverse runs, R = 1
    ([4, 1100, 8, 64, 64, 64, 4], ("D", "z", "init"), "packed"),             # reverse runs of 2 chunks
    ([4, 2900, 8, 64, 64, 64, 4], ("z", "init"), "packed"),                  # reverse runs of 3 chunks
    ([2, 200, 8, 64, 64, 64, 1], ("D", "z", "init"), "mixed"),               # R = 8: chunk-parallel dSoff
    ([2, 130, 256, 64, 64, 64, 32], ("z", "init"), "mixed"),                 # reverse dstate pass
    ([2, 200, 256, 64, 64, 64, 128], ("D2", "z", "bias", "init"), "mixed"),  # fused reverse, R = 2
    ([4, 130, 256, 64, 64, 128, 64], ("D", "init"), "packed"),               # fused reverse, R = 4
    ([4, 140, 256, 64, 64, 64, 64], ("z", "bias"), "mixed"),                 # fused reverse, R = 4, z
    ([1, 150, 256, 64, 64, 64, 256], ("z", "bias", "init"), "mixed"),        # fused reverse, R = 1
]


@pytest.mark.parametrize("shape,features,kind", BWD,
                         ids=[f"{'x'.join(map(str, c[0]))}-{'+'.join(c[1])}-{c[2]}" for c in BWD])
def test_packed_sequence_gradients(shape, features, kind):
    """Gradients of every input with packed sequences against float64 autograd
    of the oracle: non-decreasing ids at the caller's chunk size, or ids that
    interleave and go negative at chunk 64."""
    _need_gpu()
    b, l, h, p, n, chunk, g = shape
    _say(f"packed-sequence backward {shape} {features} {kind}")
    inp = make_inputs(shape, seed=340, features=features)
    gen = torch.Generator().manual_seed(7)
    if kind == "packed":
        ids = torch.stack([_ids_from_lengths(_lengths(l, gen, hi=150)) for _ in range(b)])
    else:
        ids = torch.randint(-1, 3, (b, l), generator=gen, dtype=torch.int32)
        ids[0, : min(l, 130)] = 0  # the initial state carried over two chunk edges
    gy = torch.randn(b, l, h, p, generator=gen)
    gf = torch.randn(b, h, p, n, generator=gen)
    got = _grads(inp, chunk, ids, gy, gf, on_gpu=True)
    want = _grads(inp, chunk, ids, gy, gf, on_gpu=False)
    for k in inp:
        ma, rl = parity_metrics(got[k], want[k])
        _say(f"  d{k:<15} maxabs {ma:.3e} relL2 {rl:.3e}")
        assert torch.isfinite(got[k]).all(), k
        assert rl <= 2e-4, (k, rl)


def test_varlen_states_under_autograd():
    """With grads enabled the varlen states come back (not differentiable) and
    the gradients of out and final match the no-varlen call."""
    _need_gpu()
    import ascend_kernel

    inp = make_inputs([1, 300, 4, 64, 64, 64, 2], seed=350, features=("bias",))
    lengths = [100, 28, 172]
    ids = _ids_from_lengths(lengths)[None].cuda()
    cu = torch.tensor([0, 100, 128, 300], dtype=torch.int32, device="cuda")
    res = []
    for varlen in (False, True):
        leaves = {k: v.cuda().requires_grad_(True) for k, v in inp.items()}
        r = ascend_kernel.mamba2_ssd_fwd(
            leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], 64,
            dt_bias=leaves["dt_bias"], dt_softplus=True, return_final_state=True, seq_idx=ids,
            cu_seqlens=cu if varlen else None, return_varlen_states=varlen)
        (r[0].square().sum() + r[1].square().sum()).backward()
        if varlen:
            assert len(r) == 3 and not r[2].requires_grad and r[2].shape == (3, 4, 64, 64)
        res.append({k: v.grad.clone() for k, v in leaves.items()})
    torch.cuda.synchronize()
    for k in res[0]:
        assert torch.equal(res[0][k], res[1][k]), k


def test_varlen_states_empty_sequences():
    """An empty sequence (equal consecutive cu_seqlens) has the zero state; the
    others match the oracle."""
    _need_gpu()
    inp = make_inputs([1, 150, 2, 64, 64, 64, 1], seed=360)
    lengths = [40, 0, 110]
    ids = torch.cat([torch.zeros(40), torch.full((110,), 2)]).to(torch.int32)[None]
    cu = torch.tensor([0, 40, 40, 150], dtype=torch.int32)
    _, _, got_v = _run(inp, 64, ids, cu_seqlens=cu.cuda(), return_varlen_states=True)
    _, _, states = _ref(inp, 64, ids, return_chunk_states=True)
    want_v = chunk_state_varlen_ref(inp["x"], inp["dt"], inp["A"], inp["B"], 64,
                                    torch.tensor([0, 40, 150]), states, dt_softplus=True)
    assert torch.equal(got_v[1], torch.zeros_like(got_v[1]))
    _check("varlen states", torch.stack([got_v[0], got_v[2]]), want_v)
    assert got_v.shape[0] == len(lengths)
