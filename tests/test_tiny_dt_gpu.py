"""GPU parity of the forward when softplus(dt) is tiny.

The fused forward multiplies q = softplus(dt) into two of its split-fp16
operands (the decayed mask W and the state update's right operand), and the
state it stages for C . S scales with q as well.  Left as they are, values
of 1e-9 fall into fp16's subnormal range and lose their low bits: the output
keeps a tiny absolute error but its relative error grows without bound as q
shrinks (rel-L2 0.95 at q ~ 2e-9 in the CPU emulation).  The kernels scale q
per chunk and the staged state per chunk by powers of two, so the relative
error does not depend on the magnitude of q; these cases pin that, for the
dstate-64 and dstate-128 kernels, one segment and several, with and without
an initial state, and with q jumping up or down inside a sequence.  The
reference's own boundary case (dt = -20 under softplus,
mamba_ascendc/csrc/ops/mamba2_ssd_fwd/test/mamba2_ssd_fwd-test-cases.md) runs
in tests/test_ref_cases_gpu.py.
"""

import sys

import pytest
import torch

from oracle.ssd_reference import dominant_q_dt, make_inputs, parity_metrics, ssd_chunk_scan_ref

pytestmark = pytest.mark.gpu

RELL2 = 1e-5  # the bound of the normal-magnitude small cases


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _check(inp, chunk, label):
    import ascend_kernel

    dev = {k: v.cuda() for k, v in inp.items()}
    out, fin = ascend_kernel.mamba2_ssd_fwd(
        dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], chunk, D=dev.get("D"), z=dev.get("z"),
        dt_softplus=True, initial_states=dev.get("initial_states"), return_final_state=True)
    torch.cuda.synchronize()
    ref, ref_fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], chunk,
                                      D=inp.get("D"), z=inp.get("z"), dt_softplus=True,
                                      initial_states=inp.get("initial_states"), return_final_state=True)
    ma, rl = parity_metrics(out.cpu(), ref)
    fma, frl = parity_metrics(fin.cpu(), ref_fin)
    _say(f"  {label}: |y| max {float(ref.abs().max()):.2e} out rel {rl:.2e} maxabs {ma:.2e} | "
         f"final rel {frl:.2e}")
    assert rl <= RELL2 and frl <= RELL2, (label, rl, frl)
    assert ma <= 2e-2 and fma <= 2e-2


SHAPES = [
    # [B, L, H, P, N, chunk, G]
    [8, 256, 32, 64, 64, 64, 8],   # 256 streams: one segment each
    [2, 1024, 4, 64, 64, 64, 2],   # 8 streams: segments folded from pre-segments
    [1, 256, 4, 64, 128, 64, 1],   # dstate 128, one segment
    [2, 1024, 8, 64, 128, 64, 1],  # dstate 128, segments, C . B^T precomputed
    [1, 96, 2, 32, 16, 32, 1],     # zero-padded into the fused kernel
]


@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
@pytest.mark.parametrize("offset", [-12.0, -20.0])
def test_uniformly_tiny_q(shape, offset):
    """Every token's dt lowered: q down to ~6e-6 (offset -12) or ~2e-9 (-20)."""
    _need_gpu()
    _say(f"tiny q {shape} dt offset {offset}")
    inp = make_inputs(shape, seed=11)
    inp["dt"] = inp["dt"] + offset
    _check(inp, shape[5], "plain")


@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[1], SHAPES[3]], ids=["one-seg", "segments", "n128"])
def test_tiny_q_with_initial_states_and_features(shape):
    """An O(1e-9) initial state and tiny q (the state stays tiny), with D and
    z; then an O(1) initial state with tiny q (the state stays O(1))."""
    _need_gpu()
    _say(f"tiny q with initial states {shape}")
    inp = make_inputs(shape, seed=12, features=("D", "z", "init"))
    inp["dt"] = inp["dt"] - 20.0
    init = inp["initial_states"]
    inp["initial_states"] = init * 1e-9
    _check(inp, shape[5], "tiny init")
    inp["initial_states"] = init
    _check(inp, shape[5], "O(1) init")


@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[1], SHAPES[3]], ids=["one-seg", "segments", "n128"])
@pytest.mark.parametrize("order,offset", [("drop", -20.0), ("rise", -20.0), ("drop", -45.0)],
                         ids=["drop", "rise", "deep-drop"])
def test_q_jumps_inside_the_sequence(shape, order, offset):
    """q of ~1 on one half of every sequence and ~2e-9 (offset -20) or ~3e-20
    (-45) on the other, with a strongly decaying head among slow ones, so the
    state is carried across the jump (drop: large-q history under tiny-q
    chunks; rise: the reverse).  The deep drop puts the state more than 2^60
    above the chunk's own terms, the case where W is formed in the state's
    scale."""
    _need_gpu()
    _say(f"q jump {order} {offset} {shape}")
    inp = make_inputs(shape, seed=13)
    L = shape[1]
    tiny = torch.zeros(L, dtype=torch.bool)
    if order == "drop":
        tiny[L // 2 + 7:] = True
    else:
        tiny[: L // 2 + 7] = True
    inp["dt"] = torch.where(tiny[None, :, None], inp["dt"] + offset, inp["dt"])
    inp["A"][0] = -8.0
    _check(inp, shape[5], order)


def _grads(inp, chunk, gy, gf, on_gpu):
    import ascend_kernel

    if on_gpu:
        leaves = {k: v.cuda().requires_grad_(True) for k, v in inp.items()}
        out, fin = ascend_kernel.mamba2_ssd_fwd(
            leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], chunk, D=leaves.get("D"),
            dt_softplus=True, initial_states=leaves.get("initial_states"), return_final_state=True)
        ((out * gy.cuda()).sum() + (fin * gf.cuda()).sum()).backward()
        torch.cuda.synchronize()
        return {k: v.grad.cpu() for k, v in leaves.items()}
    leaves = {k: v.double().requires_grad_(True) for k, v in inp.items()}
    out, fin = ssd_chunk_scan_ref(leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], chunk,
                                  D=leaves.get("D"), dt_softplus=True,
                                  initial_states=leaves.get("initial_states"), return_final_state=True,
                                  compute_dtype=torch.float64)
    ((out * gy.double()).sum() + (fin * gf.double()).sum()).backward()
    return {k: v.grad for k, v in leaves.items()}


@pytest.mark.parametrize("shape", [[2, 256, 4, 64, 64, 64, 2], [4, 200, 256, 64, 64, 64, 64]],
                         ids=["runs", "fused-reverse"])
def test_backward_with_tiny_q(shape):
    """Training forward (chunk states saved) and M1 backward at q ~ 2e-9
    against float64 autograd of the oracle, at the small cases' bound."""
    _need_gpu()
    _say(f"backward tiny q {shape}")
    inp = make_inputs(shape, seed=14, features=("D", "init"))
    inp["dt"] = inp["dt"] - 20.0
    gen = torch.Generator().manual_seed(6)
    b, l, h, p, n, chunk, g = shape
    gy = torch.randn(b, l, h, p, generator=gen)
    gf = torch.randn(b, h, p, n, generator=gen)
    got = _grads(inp, chunk, gy, gf, True)
    want = _grads(inp, chunk, gy, gf, False)
    for k in inp:
        ma, rl = parity_metrics(got[k], want[k])
        _say(f"  d{k:<15} maxabs {ma:.3e} relL2 {rl:.3e}")
        assert torch.isfinite(got[k]).all(), k
        assert rl <= 2e-4, (k, rl)


@pytest.mark.parametrize("shape", [[2, 640, 8, 64, 64, 64, 2], [1, 640, 4, 64, 128, 64, 1]], ids=["n64", "n128"])
def test_packed_sequences_alternating_tiny_q(shape):
    """Packed sequences whose q alternates between ~1 and ~2e-9 from one
    sequence to the next: where a sequence cuts the state its scale restarts
    from that chunk's q, so a tiny-q sequence after a large-q one keeps full
    relative precision.  Checked per sequence (a global rel-L2 would be
    dominated by the large-q sequences)."""
    import ascend_kernel

    _need_gpu()
    _say(f"packed tiny q {shape}")
    inp = make_inputs(shape, seed=15)
    b, l = shape[0], shape[1]
    bounds = [0, 150, 290, 300, 470, l]  # sequences of 150, 140, 10, 170, 170 tokens
    ids = torch.zeros(b, l, dtype=torch.int32)
    for i in range(len(bounds) - 1):
        ids[:, bounds[i]:bounds[i + 1]] = i
        if i % 2 == 1:
            inp["dt"][:, bounds[i]:bounds[i + 1]] -= 20.0
    dev = {k: v.cuda() for k, v in inp.items()}
    out, fin = ascend_kernel.mamba2_ssd_fwd(dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], shape[5],
                                            dt_softplus=True, return_final_state=True, seq_idx=ids.cuda())
    torch.cuda.synchronize()
    ref, ref_fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], shape[5],
                                      dt_softplus=True, return_final_state=True, seq_idx=ids)
    out = out.cpu()
    for i in range(len(bounds) - 1):
        sl = slice(bounds[i], bounds[i + 1])
        ma, rl = parity_metrics(out[:, sl], ref[:, sl])
        _say(f"  sequence {i} ({'tiny' if i % 2 else 'normal'} q): |y| max "
             f"{float(ref[:, sl].abs().max()):.2e} rel {rl:.2e} maxabs {ma:.2e}")
        assert rl <= RELL2, (i, rl)
    _, frl = parity_metrics(fin.cpu(), ref_fin)
    assert frl <= RELL2, frl


@pytest.mark.parametrize("shape", [[2, 400, 4, 64, 64, 64, 2], [1, 400, 4, 64, 128, 64, 1]], ids=["n64", "n128"])
def test_interleaved_ids_with_tiny_q(shape):
    """Ids drawn per token from {-1, 0, 1, 2} (most chunks hold three or four
    of them, and an id comes back after others), with id 1's q ~2e-9 and the
    others' ~1: each id's tokens are scaled by that id's own sum, so every id
    keeps the small cases' bound (checked per id)."""
    import ascend_kernel

    _need_gpu()
    _say(f"interleaved ids, tiny q on id 1 {shape}")
    inp = make_inputs(shape, seed=16)
    b, l = shape[0], shape[1]
    gen = torch.Generator().manual_seed(7)
    ids = torch.randint(-1, 3, (b, l), generator=gen, dtype=torch.int32)
    inp["dt"] = torch.where((ids == 1)[:, :, None], inp["dt"] - 20.0, inp["dt"])
    dev = {k: v.cuda() for k, v in inp.items()}
    out, fin = ascend_kernel.mamba2_ssd_fwd(dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], shape[5],
                                            dt_softplus=True, return_final_state=True, seq_idx=ids.cuda())
    torch.cuda.synchronize()
    ref, ref_fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], shape[5],
                                      dt_softplus=True, return_final_state=True, seq_idx=ids)
    out = out.cpu()
    for i in (-1, 0, 1, 2):
        sel = ids == i
        ma, rl = parity_metrics(out[sel], ref[sel])
        _say(f"  id {i}: {int(sel.sum())} tokens, |y| max {float(ref[sel].abs().max()):.2e} rel {rl:.2e} "
             f"maxabs {ma:.2e}")
        assert rl <= RELL2, (i, rl)
    _, frl = parity_metrics(fin.cpu(), ref_fin)
    assert frl <= RELL2, frl


@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_one_dominant_token_per_chunk_with_large_x(shape):
    """Every chunk's q sum comes from one token (q 0.99, the others 1e-4) and
    |x| reaches 1e4: the per-chunk scale keeps the largest scaled q below 1,
    so the staged operands (x, decay q x or decay q B, the state) stay inside
    fp16's range (scaling the q sum alone into [8, 16) lifted that token to
    nearly 16 and overflowed them).  |y| is in the 1e4-1e5 range, so the
    bound is relative (the small cases' rel-L2)."""
    _need_gpu()
    _say(f"dominant token, |x| ~ 1e4 {shape}")
    b, l, h = shape[0], shape[1], shape[2]
    inp = make_inputs(shape, seed=17)
    inp["x"] = inp["x"] * 2e3
    inp["dt"] = dominant_q_dt(b, l, h, 64, seed=18)
    import ascend_kernel

    dev = {k: v.cuda() for k, v in inp.items()}
    out, fin = ascend_kernel.mamba2_ssd_fwd(dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], shape[5],
                                            dt_softplus=True, return_final_state=True)
    torch.cuda.synchronize()
    ref, ref_fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], shape[5],
                                      dt_softplus=True, return_final_state=True)
    assert torch.isfinite(out).all() and torch.isfinite(fin).all()
    _, rl = parity_metrics(out.cpu(), ref)
    _, frl = parity_metrics(fin.cpu(), ref_fin)
    _say(f"  |y| max {float(ref.abs().max()):.2e} out rel {rl:.2e} | final rel {frl:.2e}")
    assert rl <= RELL2 and frl <= RELL2, (rl, frl)


@pytest.mark.parametrize("shape", [[2, 640, 8, 64, 64, 64, 2], [1, 640, 4, 64, 128, 64, 1]], ids=["n64", "n128"])
def test_packed_sequences_with_one_dominant_token_each(shape):
    """Sequences of 40 tokens (most chunks hold two or three ids), each with
    one token at q 0.99 among q 1e-4, |x| ~ 1e4: each id's scale is capped by
    that id's largest q."""
    import ascend_kernel

    _need_gpu()
    _say(f"packed, dominant token per sequence {shape}")
    b, l, h = shape[0], shape[1], shape[2]
    inp = make_inputs(shape, seed=19)
    inp["x"] = inp["x"] * 2e3
    inp["dt"] = dominant_q_dt(b, l, h, 40, seed=20)
    ids = (torch.arange(l, dtype=torch.int32) // 40).expand(b, l).contiguous()
    dev = {k: v.cuda() for k, v in inp.items()}
    out, fin = ascend_kernel.mamba2_ssd_fwd(dev["x"], dev["dt"], dev["A"], dev["B"], dev["C"], shape[5],
                                            dt_softplus=True, return_final_state=True, seq_idx=ids.cuda())
    torch.cuda.synchronize()
    ref, ref_fin = ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], shape[5],
                                      dt_softplus=True, return_final_state=True, seq_idx=ids)
    assert torch.isfinite(out).all() and torch.isfinite(fin).all()
    _, rl = parity_metrics(out.cpu(), ref)
    _, frl = parity_metrics(fin.cpu(), ref_fin)
    _say(f"  |y| max {float(ref.abs().max()):.2e} out rel {rl:.2e} | final rel {frl:.2e}")
    assert rl <= RELL2 and frl <= RELL2, (rl, frl)
