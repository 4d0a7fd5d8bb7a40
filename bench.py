#!/usr/bin/env python3
"""Benchmark of the MI355X Mamba-2 SSD hot path on one GPU.

Workload: the headline configuration [B,L,H,P,N,chunk,G] = [8,4096,256,64,64,64,64]
(x, dt, A, B, C; dt_softplus=True, return_final_state=True; fp32 public tensors),
synthetic inputs drawn on the CPU with torch.Generator("cpu").manual_seed(20260806 +
config index) in the order x = randn, dt = rand, A = -rand, B = randn, C = randn, then
copied to the GPU, so the GPU and the CPU baseline see bit-identical tensors.  A "step" is one forward call over that batch; when the
backward is available the fwd+bwd time (loss mean(y^2) + mean(final^2)) is reported
beside it.

Protocol (the reference's: benchmarks/mamba2_backward_bench.py:354-389, warmup 10 /
repeat 30, median of per-call device events): every kernel of a call is bracketed by
HIP events on the launch stream (the library's *_traced entry points), so the per-kernel
durations used for the roofline come from the timed region itself.  The wall-clock
time of the K steps, bracketed by device synchronisation, gives ms_per_step.

CPU baseline: the repository's fp32 CPU oracle (oracle/ssd_reference.py, a restatement
of the reference's mamba_torch/ssd_reference.py) timed on this host's cores on the same
CPU tensors, for every BASELINE config: the forward (C1, C2, C3, C5) and the forward plus
autograd backward of mean(y^2) + mean(final^2) (C4), time.perf_counter_ns around each call,
median of warmup 1 / repeat 3 at C3 and warmup 3 / repeat 10 elsewhere.

Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "mamba-ascendc_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "SSD fwd ms + % MFMA/HBM roofline at [8,4096,256,64,64,64,64]; fwd+bwd ms"
# BASELINE configs, [B, L, H, P, N, chunk, G]
CONFIGS = {
    1: [1, 128, 2, 64, 128, 128, 1],
    2: [4, 2048, 16, 64, 128, 128, 4],
    3: [8, 4096, 256, 64, 64, 64, 64],
    4: [4, 2048, 16, 64, 64, 64, 4],
    5: [1, 16384, 32, 64, 128, 256, 1],
}
HEADLINE = 3
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense fp16/bf16 MFMA
EXEC_CHUNK = 64             # execution chunk of the HIP kernels


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- HIP events

class HipEvents:
    """hipEvent_t handles from the HIP runtime torch already loaded."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.pool = []

    def make(self, n):
        arr = (ctypes.c_void_p * n)()
        for i in range(n):
            ev = ctypes.c_void_p()
            rc = self.hip.hipEventCreate(ctypes.byref(ev))
            if rc != 0:
                raise RuntimeError(f"hipEventCreate failed ({rc})")
            arr[i] = ev.value
        self.pool.append(arr)
        return arr

    def elapsed(self, a, b) -> float:
        ms = ctypes.c_float(0.0)
        rc = self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)

    def close(self):
        for arr in self.pool:
            for ev in arr:
                if ev:
                    self.hip.hipEventDestroy(ev)
        self.pool = []


# ----------------------------------------------------------------------------- work model

def bwd_runs(shape):
    """Runs per (b, h) stream of the reverse fused backward (mamba2_ssd.hip
    bwd_rev_plan): with fewer than 256 (b, g) streams each is cut into about
    256 / (B G) runs of equal length, whose own contributions the run
    pre-pass forms."""
    b, l, h, _p, _n, _chunk, g = shape
    k = math.ceil(l / EXEC_CHUNK)
    bg = b * g
    nseg = min(-(-256 // bg), k)
    m = math.ceil(k / nseg)
    return math.ceil(k / m)


def fwd_folds(shape):
    """True when the fused forward of this shape launches no segment
    recurrence (one segment, or full segments that fold the pre-segments
    into their entering states)."""
    return _fwd_plan(shape)[3]


def fwd_segments(shape):
    """(nseg, nseg_pre, nsplit) of the fused forward's plan (mamba2_ssd.hip
    fwd_plan): dstate 128 runs two workgroups per head; with fewer than 256
    (b, h, half) streams the sequence is cut into segments (when that saves at
    least 6 chunk steps), and the state-only pass runs on segments twice as
    fine (only those before the last full segment when the full segments
    fold them into their entering states themselves)."""
    return _fwd_plan(shape)[:3]


def _fwd_plan(shape):
    b, l, h, p, n, _chunk, g = shape
    k = math.ceil(l / EXEC_CHUNK)
    nsplit = n // 64
    streams = b * h * nsplit
    nseg = 1 if streams >= 256 else -(-256 // streams)
    nseg = min(nseg, k)
    if k - math.ceil(k / nseg) < 6:
        nseg = 1
    if nseg == 1:
        return 1, 1, nsplit, True
    mt = math.ceil(k / nseg)
    mult = 1 if mt <= 8 else min(2, mt)  # segments of at most 8 chunks: pre-segments as long
    mp = math.ceil(mt / mult)
    nseg = math.ceil(k / (mult * mp))
    if (nseg - 1) * mult <= 12:
        # each full segment folds the pre-segments before it: the last full
        # segment's own pre-segments are not computed
        return nseg, (nseg - 1) * mult, nsplit, True
    return nseg, math.ceil(k / mp), nsplit, False


def fwd_kernel_model(name: str, shape) -> dict:
    """Algorithmic bytes and flops of one launch of a forward kernel.

    Per unit (b, h, k) of one 64-token execution chunk; B and C are per group,
    so their bytes count once per group (1/R per head).  Flops are dense-tile
    products (no causal halving), counted once (the split-fp16 scheme issues
    three MFMAs per product; that is not algorithmic work).
    """
    b, l, h, p, n, _chunk, g = shape
    T = EXEC_CHUNK
    k = math.ceil(l / T)
    r = h // g
    units = b * h * k
    f4 = 4
    if name.endswith("_seq"):
        # packed sequences: the same tensors plus the [B, L] ids, shared by
        # every head (a few bytes per unit, not counted)
        name = name[: -len("_seq")]
    if name == "k_chunk_state":
        per = f4 * (T * p + T + T * n / r + p * n + 1)
        fl = 2 * T * p * n
    elif name == "k_state_pass_op":
        # the standalone state-passing op over every chunk state: chunk
        # states in, states entering the chunks out, the log decays and the
        # final state
        su = b * h * k
        per = f4 * (2 * p * n + 1)
        return {"bytes": su * per + b * h * p * n * f4, "flops": su * 2 * p * n, "units": su,
                "bytes_per_unit": per}
    elif name == "k_state_pass":
        # between the fused forward's segments: segment states in and out
        _, nseg_pre, _ = fwd_segments(shape)
        su = b * h * nseg_pre
        per = f4 * (2 * p * n + 1)
        return {"bytes": su * per + b * h * p * n * f4, "flops": su * 2 * p * n, "units": su,
                "bytes_per_unit": per}
    elif name == "k_chunk_cb":
        # C . B^T of every (b, g, chunk): B, C in, the 64 x 64 product out,
        # once per group (1/R per head unit)
        per = f4 * (2 * T * n + T * T) / r
        fl = 2 * T * T * n / r
    elif name in ("k_fwd_seg", "k_fwd_wide"):
        # fused: x, dt, B, C in, y out; the state stays on chip (segment
        # entry/exit states are a few per stream and not counted).  dstate
        # 128 (k_fwd_wide) splits a head's channels over two workgroups,
        # which share B and C through L2: the same bytes per (b, h, k)
        per = f4 * (2 * T * p + T + 2 * T * n / r)
        fl = 2 * (T * T * n / r + T * T * p + 2 * T * n * p)
    elif name in ("k_fwd_seg_save", "k_fwd_wide_save"):
        # training forward: as k_fwd_seg plus the state entering every chunk
        per = f4 * (2 * T * p + T + 2 * T * n / r + p * n)
        fl = 2 * (T * T * n / r + T * T * p + 2 * T * n * p)
    elif name in ("k_fwd_seg_gate", "k_fwd_seg_save_gate", "k_fwd_wide_gate", "k_fwd_wide_save_gate"):
        # z-gated forms: as k_fwd_seg / k_fwd_seg_save plus z in, and for
        # training the pre-gate output y + D x out (D, dt_bias and the
        # initial states are a few values per head or stream)
        save = name.endswith("save_gate")
        per = f4 * ((4 if save else 3) * T * p + T + 2 * T * n / r + (p * n if save else 0))
        fl = 2 * (T * T * n / r + T * T * p + 2 * T * n * p)
    elif name == "k_fwd_seg_state":
        per = f4 * (T * p + T + T * n / r)
        fl = 2 * T * p * n
    elif name in ("k_fwd_seg_state_save", "k_fwd_state_group"):
        # the backward's recompute of the chunk-start states: x, dt, B in,
        # the state entering every chunk out (k_fwd_state_group: the same
        # pass, one workgroup per group walking its heads)
        per = f4 * (T * p + T + T * n / r + p * n)
        fl = 2 * T * p * n
    elif name == "k_bwd_run_grad":
        # dout, dt, C in; one state-sized contribution and log decay per run out
        runs = b * h * bwd_runs(shape)
        per = f4 * (T * p + T + T * n / r)
        return {"bytes": units * per + runs * f4 * (p * n + 1), "flops": units * 2 * T * p * n,
                "units": units, "bytes_per_unit": per}
    elif name == "k_state_pass_bwd":
        # the backward's recurrence over runs, in place: each run's
        # contribution and log decay in, the gradient entering it out, plus
        # the final-state gradient
        su = b * h * bwd_runs(shape)
        per = f4 * (2 * p * n + 1)
        return {"bytes": su * per + b * h * p * n * f4, "flops": su * 2 * p * n, "units": su,
                "bytes_per_unit": per}
    elif name == "k_bwd_dstate_rev":
        # dout, dt, C in; dU (state gradient leaving each chunk) out
        per = f4 * (T * p + T + T * n / r + p * n)
        fl = 2 * T * p * n
    elif name == "k_bwd_ws":
        # x, dout, dt, S, dU, B, C in; dx, ddt, dB, dC out.  Products per unit
        # (dense tiles): C.B^T per group, dW twice, W^T gy, dCB.B, dCB^T.C,
        # B.dU^T, gy.S, x.dU
        per = f4 * (3 * T * p + 2 * T + 2 * p * n + 4 * T * n / r)
        fl = 2 * (2 * T * T * n / r + 2 * T * T * p + 2 * T * T * n + 3 * T * n * p)
    elif name == "k_bwd_ws_rev":
        # reverse fused: as k_bwd_ws without dU in (the state gradient is
        # carried on chip), plus the dSoff product (gy exp(cs))^T C
        per = f4 * (3 * T * p + 2 * T + p * n + 4 * T * n / r)
        fl = 2 * (2 * T * T * n / r + 2 * T * T * p + 2 * T * T * n + 4 * T * n * p)
    elif name == "k_bwd_ws_rev_z":
        # with the z gate: z and the pre-gate output in, dz out, besides
        # k_bwd_ws_rev's tensors
        per = f4 * (6 * T * p + 2 * T + p * n + 4 * T * n / r)
        fl = 2 * (2 * T * T * n / r + 2 * T * T * p + 2 * T * T * n + 4 * T * n * p)
    else:
        per, fl = float("nan"), float("nan")
    if name.startswith("k_fwd_wide") and n == 128 and r >= 8:
        # C . B^T comes from k_chunk_cb (read once per group, not formed)
        per += f4 * T * T / r
        fl -= 2 * T * T * n / r
    return {"bytes": units * per, "flops": units * fl, "units": units, "bytes_per_unit": per}


def measured_traffic(kernel, shape):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary of this configuration (profiles/pmc_traffic_c<cfg>.json), or None."""
    for cfg, shp in CONFIGS.items():
        if shp == list(shape):
            path = os.path.join(ROOT, "profiles", f"pmc_traffic_c{cfg}.json")
            if os.path.exists(path):
                with open(path) as fh:
                    data = json.load(fh)
                return data.get("traffic_bytes", {}).get(kernel)
    return None


def op_work(shape):
    """Op-level algorithmic work: F = 2*B*L*[G*T*N + H*(T*P + 2*N*P)] and the
    compulsory fp32 public I/O bytes (x, out, dt, A, B, C, final)."""
    b, l, h, p, n, chunk, g = shape
    T = EXEC_CHUNK
    flops = 2 * b * l * (g * T * n + h * (T * p + 2 * n * p))
    nbytes = 4 * (2 * b * l * h * p + b * l * h + h + 2 * b * l * g * n + b * h * p * n)
    return flops, nbytes


# ----------------------------------------------------------------------------- GPU runs

def make_cpu_inputs(torch, shape, seed):
    """The BASELINE inputs: one CPU generator seeded with `seed`, drawn in the
    order x = randn, dt = rand, A = -rand, B = randn, C = randn (fp32)."""
    b, l, h, p, n, _chunk, g = shape
    gen = torch.Generator("cpu").manual_seed(seed)
    return {
        "x": torch.randn(b, l, h, p, generator=gen),
        "dt": torch.rand(b, l, h, generator=gen),
        "A": -torch.rand(h, generator=gen),
        "B": torch.randn(b, l, g, n, generator=gen),
        "C": torch.randn(b, l, g, n, generator=gen),
    }


def to_gpu(torch, cpu):
    gpu = {k: v.cuda() for k, v in cpu.items()}
    torch.cuda.synchronize()
    return gpu


def summarize(samples):
    """Tail statistics of per-call times (the reference bench's summary,
    benchmarks/mamba2_backward_bench.py:380-389)."""
    vals = list(samples)
    ordered = sorted(vals)
    return {"median_ms": round(statistics.median(vals), 6), "mean_ms": round(statistics.fmean(vals), 6),
            "p90_ms": round(ordered[min(len(ordered) - 1, math.ceil(0.9 * len(ordered)) - 1)], 6),
            "min_ms": round(min(vals), 6), "max_ms": round(max(vals), 6), "n": len(vals)}


def checksums(torch, tensors):
    """Sum of every tensor (float64 accumulation), and their total: the
    reference bench's gradient checksums (mamba2_backward_bench.py:569-579)."""
    sums = {k: float(v.double().sum()) for k, v in tensors.items()}
    total = sum(sums.values())
    return {k: (v if math.isfinite(v) else None) for k, v in sums.items()}, (total if math.isfinite(total) else None)


def run_traced(torch, lib, rt, hip, call, nsteps, max_kernels=16):
    """Run `call(events_ptr, nevents, names, nk)` nsteps times; return per-step
    (total_ms, [kernel_ms...]) and the kernel names."""
    steps = []
    names_out = None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(nsteps):
        ev = hip.make(max_kernels + 1)
        names = (ctypes.c_char_p * max_kernels)()
        nk = ctypes.c_int(0)
        call(ev, max_kernels + 1, names, nk)
        steps.append((ev, nk.value, names))
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    results = []
    for ev, nkern, names in steps:
        per = [hip.elapsed(ev[i], ev[i + 1]) for i in range(nkern)]
        results.append((hip.elapsed(ev[0], ev[nkern]), per))
        names_out = [names[i].decode() for i in range(nkern)]
    hip.close()
    return results, names_out, wall_ms


def bench_forward(torch, lib, rt, api, hip, inp, shape, steps, warmup):
    x, dt, A, B, C = (inp[k] for k in ("x", "dt", "A", "B", "C"))
    b, l, h, p, n, chunk, g = shape
    shp = rt.Mamba2SsdShape(b, l, h, p, g, n, chunk)
    flags = rt.DT_SOFTPLUS
    nbytes = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(shp), flags, ctypes.byref(nbytes)),
             "workspace", lib)
    out = torch.empty_like(x)
    final = torch.empty(b, h, p, n, device=x.device, dtype=torch.float32)
    ws = torch.empty(max(1, nbytes.value), dtype=torch.uint8, device=x.device)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    args = rt.Mamba2SsdFwdArgs(shp, flags, 0.0, math.inf, P(x), P(dt), P(A), P(B), P(C),
                               None, None, None, None, P(out), P(final))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call(ev, nev, names, nk):
        rt.check(lib.mamba2_ssd_fwd_traced(ctypes.byref(args), P(ws), ws.numel(), stream,
                                           ev, nev, names, ctypes.byref(nk)),
                 "mamba2_ssd_fwd_traced", lib)

    run_traced(torch, lib, rt, hip, call, warmup)
    res, names, wall = run_traced(torch, lib, rt, hip, call, steps)
    ok = bool(torch.isfinite(out).all()) and bool(torch.isfinite(final).all())
    return res, names, wall, ok, ws.numel(), out, final


PARITY_MAXABS, PARITY_RELL2 = 2e-2, 5e-3  # the contract: max-abs and relative-L2 vs the fp32 oracle


def parity_slices(torch, cpu_inp, out, final, shape, slices):
    """Same-run parity gate: the CPU oracle on slices (batch, head0, head1) of the
    timed inputs against the same slices of the GPU output.  Heads share nothing
    but their group's B and C, so a slice of heads of one group is an
    independent problem."""
    from oracle.ssd_reference import parity_metrics, ssd_chunk_scan_ref

    b, l, h, p, n, chunk, g = shape
    r = h // g
    rows, worst = [], [0.0, 0.0, 0.0, 0.0]
    for bi, h0, h1 in slices:
        gi = h0 // r
        assert (h1 - 1) // r == gi, "a parity slice stays within one group"
        sub = {"x": cpu_inp["x"][bi:bi + 1, :, h0:h1], "dt": cpu_inp["dt"][bi:bi + 1, :, h0:h1],
               "A": cpu_inp["A"][h0:h1], "B": cpu_inp["B"][bi:bi + 1, :, gi:gi + 1],
               "C": cpu_inp["C"][bi:bi + 1, :, gi:gi + 1]}
        sub = {k: v.contiguous() for k, v in sub.items()}
        with torch.no_grad():
            ref, ref_fin = ssd_chunk_scan_ref(sub["x"], sub["dt"], sub["A"], sub["B"], sub["C"], chunk,
                                              dt_softplus=True, return_final_state=True)
        m = parity_metrics(out[bi:bi + 1, :, h0:h1].cpu(), ref) + \
            parity_metrics(final[bi:bi + 1, h0:h1].cpu(), ref_fin)
        worst = [max(a, c) for a, c in zip(worst, m)]
        rows.append(f"batch {bi} heads {h0}..{h1 - 1}")
    ok = (worst[0] <= PARITY_MAXABS and worst[1] <= PARITY_RELL2 and worst[2] <= PARITY_MAXABS
          and worst[3] <= PARITY_RELL2)
    return {"slices": rows, "out_maxabs": worst[0], "out_relL2": worst[1],
            "final_maxabs": worst[2], "final_relL2": worst[3],
            "bound": {"maxabs": PARITY_MAXABS, "relL2": PARITY_RELL2}, "pass": bool(ok),
            "oracle": "oracle/ssd_reference.py fp32 on the CPU, same inputs"}


# parity slices (batch, head0, head1) per BASELINE config: the first and the
# last heads of the problem
PARITY_SLICES = {
    1: [(0, 0, 2)],
    2: [(0, 0, 4), (3, 12, 16)],
    3: [(0, 0, 4), (7, 252, 256)],
    4: [(0, 0, 4), (3, 12, 16)],
    5: [(0, 0, 2), (0, 30, 32)],
}


def summarize_kernels(res, names, shape):
    kern = {}
    for i, name in enumerate(names):
        durs = [r[1][i] for r in res]
        model = fwd_kernel_model(name, shape)
        avg = statistics.fmean(durs)
        kern[name] = {"avg_ms": round(avg, 6), "median_ms": round(statistics.median(durs), 6)}
        if model["bytes"] == model["bytes"]:
            kern[name]["GB_s"] = round(model["bytes"] / (avg * 1e-3) / 1e9, 1)
    return kern


def bench_config(torch, lib, rt, api, hip, cfg, steps, warmup, cpu=True):
    """One BASELINE config besides the headline: the forward (dt_softplus, final
    state) timed with the reference protocol, its per-kernel durations, the
    op-level algorithmic GB/s and HBM fraction, and a same-run parity slice; for
    config 4 (the M1 backward config) also the training forward + backward;
    and the CPU oracle on the same inputs (forward; config 4 forward plus
    autograd backward)."""
    shape = CONFIGS[cfg]
    seed = 20260806 + (cfg - 1)
    cpu_inp = make_cpu_inputs(torch, shape, seed)
    inp = to_gpu(torch, cpu_inp)
    res, names, _wall, finite, ws_bytes, out, final = bench_forward(
        torch, lib, rt, api, hip, inp, shape, steps, warmup)
    fwd_ms = statistics.median(r[0] for r in res)
    flops, nbytes = op_work(shape)
    row = {"shape": shape, "seed": seed, "fwd_ms": round(fwd_ms, 5), "fwd": summarize(r[0] for r in res),
           "fwd_kernels": summarize_kernels(res, names, shape),
           "op_GB_s": round(nbytes / (fwd_ms * 1e-3) / 1e9, 1),
           "op_TFLOP_s": round(flops / (fwd_ms * 1e-3) / 1e12, 2),
           "hbm_roofline_frac": round(nbytes / (fwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "op_bytes": nbytes, "workspace_bytes": ws_bytes, "finite": finite,
           "output_checksums": checksums(torch, {"out": out, "final": final})[0],
           "parity": parity_slices(torch, cpu_inp, out, final, shape, PARITY_SLICES[cfg])}
    del out, final
    row["api_fwd_ms"] = round(bench_api(torch, api, inp, shape[5], max(5, steps // 3), 3), 5)
    row["api_host_us"] = round(api_host_cost(torch, api, inp, shape[5]), 1)
    train = shape[3] == 64 and shape[4] == 64
    if train:
        tr = bench_fwd_bwd_traced(torch, lib, rt, hip, inp, shape, steps, warmup)
        if tr is not None:
            fres, bres, bnames, bfinite = tr[:4]
            row["fwd_train_ms"] = round(statistics.median(r[0] for r in fres), 5)
            row["bwd_ms"] = round(statistics.median(r[0] for r in bres), 5)
            row["fwd_bwd_ms"] = round(statistics.median(f[0] + bk[0] for f, bk in zip(fres, bres)), 5)
            row["fwd_train"] = summarize(r[0] for r in fres)
            row["bwd"] = summarize(r[0] for r in bres)
            row["fwd_bwd"] = summarize(f[0] + bk[0] for f, bk in zip(fres, bres))
            row["bwd_kernels"] = summarize_kernels(bres, bnames, shape)
            row["grads_finite"] = bool(bfinite)
            row["gradient_checksums"], row["gradient_checksum"] = tr[6]
    del inp
    torch.cuda.empty_cache()
    if cpu:
        row["cpu_baseline"] = cpu_oracle_baseline(torch, cpu_inp, shape, seed, with_bwd=train)
        log(f"config C{cfg} cpu baseline {row['cpu_baseline']['value']:.2f} ms "
            f"({row['cpu_baseline']['cores']} threads)")
    del cpu_inp
    return row


def full_features(torch, shape, seed):
    """The reference benchmark's "full" feature set (mamba2_backward_bench.py:
    159-165, 219-241): D [H, P], z, dt_bias, initial states, softplus and
    dt_limit (1e-3, 1); drawn on a CPU generator seeded with seed + 1 and
    copied to the GPU (tests/test_bwd_gpu.py checks this set at C3)."""
    b, l, h, p, n, _chunk, g = shape
    gen = torch.Generator("cpu").manual_seed(seed + 1)
    feats = {"D": torch.randn(h, p, generator=gen), "z": torch.randn(b, l, h, p, generator=gen),
             "dt_bias": torch.randn(h, generator=gen) * 0.1,
             "initial_states": torch.randn(b, h, p, n, generator=gen) / 5}
    return {**to_gpu(torch, feats), "dt_limit": (1e-3, 1.0)}


def feature_flags(rt, feats):
    if not feats:
        return rt.DT_SOFTPLUS, 0.0, math.inf
    return (rt.DT_SOFTPLUS | rt.HAS_D | rt.D_PER_CHANNEL | rt.HAS_Z | rt.HAS_DT_BIAS
            | rt.HAS_INITIAL), feats["dt_limit"][0], feats["dt_limit"][1]


def packed_ids(torch, shape, seed, lo=256, hi=2048):
    """Packed-sequence ids [B, L] (int32, GPU): every row cut into sequences
    of U[lo, hi) tokens, the last one shortened to fit."""
    b, l = shape[0], shape[1]
    gen = torch.Generator().manual_seed(seed + 2)
    rows = []
    for _ in range(b):
        lengths = []
        while sum(lengths) < l:
            lengths.append(int(torch.randint(lo, hi, (1,), generator=gen)))
        lengths[-1] -= sum(lengths) - l
        rows.append(torch.cat([torch.full((n,), i, dtype=torch.int32) for i, n in enumerate(lengths)]))
    return torch.stack(rows).cuda()


def bench_fwd_features(torch, lib, rt, inp, shape, feats, steps, warmup, seq=None):
    """Inference forward through the C ABI with the given feature tensors
    (and packed-sequence ids `seq`): median ms of `steps` calls (HIP events on
    the launch stream)."""
    x, dt, A, B, C = (inp[k] for k in ("x", "dt", "A", "B", "C"))
    b, l, h, p, n, chunk, g = shape
    shp = rt.Mamba2SsdShape(b, l, h, p, g, n, chunk)
    flags, lo, hi = feature_flags(rt, feats)
    if seq is not None:
        flags |= rt.HAS_SEQ_IDX
    feats = feats or {"D": None, "z": None, "dt_bias": None, "initial_states": None}
    nb = ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(shp), flags, ctypes.byref(nb)), "ws", lib)
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out = torch.empty_like(x)
    final = torch.empty(b, h, p, n, device=x.device, dtype=torch.float32)
    ws = torch.empty(max(1, nb.value), dtype=torch.uint8, device=x.device)
    fargs = rt.Mamba2SsdFwdArgs(shp, flags, lo, hi, P(x), P(dt), P(A), P(B), P(C),
                                P(feats["D"]), P(feats["z"]), P(feats["dt_bias"]),
                                P(feats["initial_states"]), P(out), P(final), None, None)
    fargs.seq_idx = P(seq)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(warmup):
        rt.check(lib.mamba2_ssd_fwd(ctypes.byref(fargs), P(ws), ws.numel(), stream), "fwd", lib)
    torch.cuda.synchronize()
    samples = []
    for _ in range(steps):
        s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        rt.check(lib.mamba2_ssd_fwd(ctypes.byref(fargs), P(ws), ws.numel(), stream), "fwd", lib)
        e0.record()
        e0.synchronize()
        samples.append(s0.elapsed_time(e0))
    return summarize(samples)


def bench_fwd_bwd_traced(torch, lib, rt, hip, inp, shape, steps, warmup, feats=None, seq=None):
    """Training forward (saving the chunk-start states) + M1 bwd through the C
    ABI with per-kernel events; upstream gradients of the loss mean(y^2) +
    mean(final^2).  `feats`: optional full-feature tensors (full_features);
    `seq`: optional packed-sequence ids.  None if unsupported; else (forward
    steps, backward steps, backward kernel names, gradients finite, workspace
    bytes, forward kernel names, (gradient checksums, their total))."""
    x, dt, A, B, C = (inp[k] for k in ("x", "dt", "A", "B", "C"))
    b, l, h, p, n, chunk, g = shape
    shp = rt.Mamba2SsdShape(b, l, h, p, g, n, chunk)
    if p != 64 or n != 64:
        return None
    flags, lo, hi = feature_flags(rt, feats)
    flags |= rt.SAVED_STATES
    if seq is not None:
        flags |= rt.HAS_SEQ_IDX
    fb, bb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    rt.check(lib.mamba2_ssd_fwd_workspace_size(ctypes.byref(shp), flags, ctypes.byref(fb)), "ws", lib)
    rt.check(lib.mamba2_ssd_bwd_m1_workspace_size(ctypes.byref(shp), flags, ctypes.byref(bb)), "ws", lib)
    P = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    states = torch.empty(b, h, (l + 63) // 64, p, n, device=x.device, dtype=torch.float32)
    out = torch.empty_like(x)
    final = torch.empty(b, h, p, n, device=x.device, dtype=torch.float32)
    ws = torch.empty(max(1, fb.value, bb.value), dtype=torch.uint8, device=x.device)
    grads = {k: torch.empty_like(v) for k, v in inp.items()}
    dout = torch.empty_like(x)
    dfinal = torch.empty_like(final)
    f = feats or {"D": None, "z": None, "dt_bias": None, "initial_states": None}
    fg = {k: (None if v is None else torch.empty_like(v)) for k, v in f.items() if k != "dt_limit"}
    grads.update({"d" + k: v for k, v in fg.items() if v is not None})
    pre_gate = torch.empty_like(x) if f["z"] is not None else None
    fargs = rt.Mamba2SsdFwdArgs(shp, flags, lo, hi, P(x), P(dt), P(A), P(B), P(C),
                                P(f["D"]), P(f["z"]), P(f["dt_bias"]), P(f["initial_states"]),
                                P(out), P(final), P(pre_gate), P(states))
    bargs = rt.Mamba2SsdBwdArgs(shp, flags, lo, hi, P(x), P(dt), P(A), P(B), P(C),
                                P(f["D"]), P(f["z"]), P(f["dt_bias"]), P(f["initial_states"]),
                                P(dout), P(dfinal), P(pre_gate), P(states),
                                P(grads["x"]), P(grads["dt"]), P(grads["A"]), P(grads["B"]),
                                P(grads["C"]), P(fg["D"]), P(fg["z"]), P(fg["dt_bias"]),
                                P(fg["initial_states"]))
    fargs.seq_idx = P(seq)
    bargs.seq_idx = P(seq)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rt.check(lib.mamba2_ssd_fwd(ctypes.byref(fargs), P(ws), ws.numel(), stream), "fwd", lib)
    torch.mul(out, 2.0 / out.numel(), out=dout)
    torch.mul(final, 2.0 / final.numel(), out=dfinal)

    def call_f(ev, nev, names, nk):
        rt.check(lib.mamba2_ssd_fwd_traced(ctypes.byref(fargs), P(ws), ws.numel(), stream,
                                           ev, nev, names, ctypes.byref(nk)), "fwd", lib)

    def call_b(ev, nev, names, nk):
        rt.check(lib.mamba2_ssd_bwd_m1_traced(ctypes.byref(bargs), P(ws), ws.numel(), stream,
                                              ev, nev, names, ctypes.byref(nk)), "bwd", lib)

    run_traced(torch, lib, rt, hip, call_b, warmup)
    fres, fnames, _ = run_traced(torch, lib, rt, hip, call_f, steps)
    bres, bnames, _ = run_traced(torch, lib, rt, hip, call_b, steps)
    ok = all(bool(torch.isfinite(v).all()) for v in grads.values())
    sums = checksums(torch, {("d" + k if not k.startswith("d") or k == "dt" else k): v
                             for k, v in grads.items()})
    return fres, bres, bnames, ok, ws.numel(), fnames, sums


def copy_calibration(torch, nbytes):
    """A plain device copy of known size, for scaling the FETCH_SIZE/WRITE_SIZE
    counters of a rocprofv3 --pmc run (it shows up there as torch's copy kernel)."""
    src = torch.empty(nbytes // 4, device="cuda", dtype=torch.float32).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return nbytes


def copy_bandwidth(torch, nbytes=1 << 30, reps=5):
    """Best GB/s (bytes read + written) of torch's device-to-device copy of
    `nbytes`: the streaming rate this GPU reaches in practice, reported next
    to the published HBM peak."""
    src = torch.empty(nbytes // 4, device="cuda", dtype=torch.float32).fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    best = float("inf")
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        dst.copy_(src)
        e.record()
        e.synchronize()
        best = min(best, s.elapsed_time(e))
    del src, dst
    torch.cuda.empty_cache()
    return 2 * nbytes / (best * 1e-3) / 1e9


def bench_state_passing(torch, lib, shape, steps=10, warmup=3):
    """The standalone inter-chunk state-passing op (C ABI
    mamba2_ssd_state_passing, the reference's mamba2_ssd_state_passing stage) on
    this configuration's [B, H, K, P, N] chunk states: ms per call and GB/s of
    its algorithmic traffic (chunk states in, states_start out, the log decays
    and final state)."""
    b, l, h, p, n, _chunk, _g = shape
    k = math.ceil(l / EXEC_CHUNK)
    gen = torch.Generator(device="cuda").manual_seed(11)
    states = torch.randn(b, h, k, p, n, device="cuda", generator=gen)
    log_decay = -torch.rand(b, h, k, device="cuda", generator=gen)
    start = torch.empty_like(states)
    final = torch.empty(b, h, p, n, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    V = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def call():
        rc = lib.mamba2_ssd_state_passing(V(states), V(log_decay), None, V(start), V(final),
                                          b, h, k, p, n, stream)
        if rc != 0:
            raise RuntimeError(f"mamba2_ssd_state_passing failed ({rc})")

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    samples = []
    for _ in range(steps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        call()
        e.record()
        e.synchronize()
        samples.append(s.elapsed_time(e))
    ms = statistics.median(samples)
    nbytes = 4 * (2 * b * h * k * p * n + b * h * k + b * h * p * n)
    del states, start, final, log_decay
    torch.cuda.empty_cache()
    return {"ms": round(ms, 5), "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes,
            "frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def bench_decode(torch, shape, batch=64, steps=20, warmup=5):
    """The decode step (selective_state_update, Mamba-2 tied form with D, z and
    dt_bias) for `batch` sequences on this configuration's model dims (H, P, N,
    G): median ms and GB/s of its algorithmic traffic (the state in and out,
    plus x, z, out, B, C)."""
    from ascend_kernel import selective_state_update

    _b, _l, h, p, n, _chunk, g = shape
    gen = torch.Generator(device="cuda").manual_seed(13)
    kw = dict(device="cuda", dtype=torch.float32, generator=gen)
    state = torch.randn(batch, h, p, n, **kw)
    x, z = torch.randn(batch, h, p, **kw), torch.randn(batch, h, p, **kw)
    dt = torch.rand(batch, h, **kw)[..., None].expand(batch, h, p)
    A = (-torch.rand(h, **kw))[:, None, None].expand(h, p, n)
    B, C = torch.randn(batch, g, n, **kw), torch.randn(batch, g, n, **kw)
    D = torch.randn(h, **kw)[:, None].expand(h, p)
    bias = torch.randn(h, **kw)[:, None].expand(h, p)

    def call():
        return selective_state_update(state, x, dt, A, B, C, D=D, z=z, dt_bias=bias, dt_softplus=True)

    from ascend_kernel.selective_state_update import prepare_state_update

    launch = prepare_state_update(state, x, dt, A, B, C, D=D, z=z, dt_bias=bias, dt_softplus=True)

    def timed(f, run=10):
        # `run` consecutive steps per sample (tokens one after another, the
        # state updated in place): the per-step time once the queue is fed
        for _ in range(warmup):
            f()
        torch.cuda.synchronize()
        samples = []
        for _ in range(steps):
            s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s0.record()
            for _ in range(run):
                f()
            e0.record()
            e0.synchronize()
            samples.append(s0.elapsed_time(e0) / run)
        return statistics.median(samples)

    ms = timed(launch)    # the launch alone (arguments laid out once)
    api_ms = timed(call)  # the whole Python call, host work included
    nbytes = 4 * (2 * batch * h * p * n + 3 * batch * h * p + 2 * batch * g * n)
    del state, x, z, B, C, launch
    torch.cuda.empty_cache()
    return {"batch": batch, "shape": [batch, h, p, n, g], "ms": round(ms, 5),
            "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1), "api_ms": round(api_ms, 5),
            "note": "per step over runs of 10 consecutive steps; ms: the step with its "
                    "arguments laid out once; api_ms: the whole selective_state_update call"}


def bench_api(torch, api, inp, chunk, steps, warmup, run=5):
    """Per-call device-event time through the public Python API, over runs of
    `run` consecutive calls (as a model issues them layer after layer), so the
    host's argument work overlaps the queued GPU work instead of being
    waited for."""
    def call():
        return api.mamba2_ssd_fwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], chunk,
                                  dt_softplus=True, return_final_state=True)
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    samples = []
    for _ in range(steps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(run):
            call()
        e.record()
        e.synchronize()
        samples.append(s.elapsed_time(e) / run)
    return statistics.median(samples)


def api_host_cost(torch, api, inp, chunk, calls=50):
    """Host microseconds to issue one forward through the public Python API
    (validation, workspace query through ctypes, output and workspace
    allocation, the launch): wall time of `calls` calls queued back to back,
    divided by `calls`.  When it is below the kernel time the host work hides
    under the queued GPU work."""
    def call():
        return api.mamba2_ssd_fwd(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], chunk,
                                  dt_softplus=True, return_final_state=True)
    for _ in range(5):
        call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        call()
    host = (time.perf_counter() - t0) / calls
    torch.cuda.synchronize()
    return host * 1e6


def bench_fwd_bwd(torch, api, inp, chunk, steps, warmup, save=True):
    """fwd + bwd through autograd; None if the backward is not available for
    this shape.  The upstream gradients are those of the loss
    mean(y^2) + mean(final^2), formed once outside the timed calls, so the
    timing covers the op's forward and backward and not torch's elementwise
    loss kernels.  save: the training policy (keep the chunk-start states, or
    recompute them in the backward)."""
    leaves = {k: v.detach().clone().requires_grad_(True) for k, v in inp.items()}

    def fwd():
        return api.mamba2_ssd_fwd(leaves["x"], leaves["dt"], leaves["A"], leaves["B"],
                                  leaves["C"], chunk, dt_softplus=True, return_final_state=True,
                                  save_chunk_states=save)

    grads = []

    def call():
        for v in leaves.values():
            v.grad = None
        out, fin = fwd()
        torch.autograd.backward((out, fin), grads)

    try:
        with torch.no_grad():
            out, fin = fwd()
            grads.extend([out * (2.0 / out.numel()), fin * (2.0 / fin.numel())])
            del out, fin
        call()
        torch.cuda.synchronize()
    except (NotImplementedError, RuntimeError) as exc:
        log(f"fwd+bwd unavailable: {exc}")
        return None, str(exc).splitlines()[0][:200]
    run = 3  # consecutive training steps per sample (host work overlaps the queue)
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    samples = []
    for _ in range(steps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(run):
            call()
        e.record()
        e.synchronize()
        samples.append(s.elapsed_time(e) / run)
    return statistics.median(samples), None


def autograd_memory(torch, api, inp, chunk, save=True):
    """Saved-tensor bytes and peak memory of one autograd forward + backward
    (the reference backward bench's saved-tensor and extra-peak figures,
    mamba2_backward_bench.py:168-215, 420-489) under the training policy
    ``save`` (keep the chunk-start states or recompute them).  saved: bytes of
    the distinct storages autograd keeps between the passes beyond the inputs;
    peak_extra: the allocator's peak during forward + backward above what was
    allocated before (inputs and upstream gradients)."""
    leaves = {k: v.detach().clone().requires_grad_(True) for k, v in inp.items()}
    inputs = {v.untyped_storage().data_ptr() for v in leaves.values()}
    seen = {}

    def pack(t):
        st = t.untyped_storage()
        if st.data_ptr() not in inputs:
            seen[st.data_ptr()] = st.nbytes()
        return t

    with torch.no_grad():
        out, fin = api.mamba2_ssd_fwd(leaves["x"], leaves["dt"], leaves["A"], leaves["B"],
                                      leaves["C"], chunk, dt_softplus=True, return_final_state=True)
        gy, gf = out * (2.0 / out.numel()), fin * (2.0 / fin.numel())
        del out, fin
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        out, fin = api.mamba2_ssd_fwd(leaves["x"], leaves["dt"], leaves["A"], leaves["B"],
                                      leaves["C"], chunk, dt_softplus=True, return_final_state=True,
                                      save_chunk_states=save)
    torch.autograd.backward((out, fin), (gy, gf))
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    del out, fin, gy, gf, leaves
    torch.cuda.empty_cache()
    return {"saved_bytes": int(sum(seen.values())), "peak_extra_bytes": int(peak)}


# ----------------------------------------------------------------------------- CPU baseline

def host_info():
    model, sockets = "unknown", set()
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                if line.startswith("physical id"):
                    sockets.add(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return {"cpu_model": model, "sockets": max(1, len(sockets)), "logical_cpus": os.cpu_count()}


def cpu_oracle_baseline(torch, cpu_inp, shape, seed, with_bwd=False, warmup=None, repeat=None):
    """The fp32 CPU oracle on the whole configuration, on the same CPU tensors
    the GPU copies came from: the forward (dt_softplus, final state), or with
    `with_bwd` the forward plus the autograd backward of mean(y^2) +
    mean(final^2) (the loss of the reference's backward benchmark; C4).  time.perf_counter_ns around each
    call (benchmarks/mamba2_backward_bench.py:373-376), median; warmup 1 /
    repeat 3 for the 8.6 GB config 3, warmup 3 / repeat 10 otherwise."""
    from oracle.ssd_reference import ssd_chunk_scan_ref

    chunk = shape[5]
    big = shape == CONFIGS[3]
    warmup = (1 if big else 3) if warmup is None else warmup
    repeat = (3 if big else 10) if repeat is None else repeat
    torch.set_num_threads(os.cpu_count() or 1)

    def call():
        if with_bwd:
            lv = {k: v.clone().requires_grad_(True) for k, v in cpu_inp.items()}
            t0 = time.perf_counter_ns()
            out, fin = ssd_chunk_scan_ref(lv["x"], lv["dt"], lv["A"], lv["B"], lv["C"], chunk,
                                          dt_softplus=True, return_final_state=True)
            (out.pow(2).mean() + fin.pow(2).mean()).backward()
        else:
            t0 = time.perf_counter_ns()
            with torch.no_grad():
                ssd_chunk_scan_ref(cpu_inp["x"], cpu_inp["dt"], cpu_inp["A"], cpu_inp["B"], cpu_inp["C"], chunk,
                                   dt_softplus=True, return_final_state=True)
        return (time.perf_counter_ns() - t0) / 1e6

    for _ in range(warmup):
        call()
    times = [call() for _ in range(repeat)]
    what = "forward + autograd backward (loss mean(y^2) + mean(final^2))" if with_bwd else "forward"
    return {
        "value": round(statistics.median(times), 4),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle fp32 {what} on the whole config {shape} (seed {seed}, the GPU's inputs), "
                   f"median of {repeat} after {warmup} warmup"),
        "stats": summarize(times),
        "host": host_info(),
        "torch": torch.__version__,
    }


# ----------------------------------------------------------------------------- profiles

def _short(name: str) -> str:
    """`ssd::k_chunk_scan<64, 64>(...)` -> `k_chunk_scan<64, 64>`."""
    base = name.split("(")[0].replace("void ", "").strip()
    return base.replace("ssd::bwd::", "").replace("ssd::", "")


def model_key(short: str) -> str:
    """Kernel-model / trace name of a (templated) kernel.

    k_fwd_seg<state only, save states, z gate, packed sequences, latency form
    (one-round grids; the same pass)>: <true, false,
    ...> is k_fwd_seg_state, <true, true, ...> k_fwd_seg_state_save (the
    backward's recompute of the chunk states), <false, true, ...> k_fwd_seg_save, <false, false, ...>
    k_fwd_seg, with a "_gate" suffix for the z-gated form and "_seq" for
    packed sequences.  k_bwd_ws<has z, heads per group, packed sequences>: a
    group size above 0 is the reverse fused k_bwd_ws_rev ("_z" with z, "_seq"
    with packed sequences).  The others drop their template arguments."""
    if short.startswith("k_fwd_wide<"):
        args = [a.strip() for a in short[len("k_fwd_wide<"):-1].split(",")]
        key = "k_fwd_wide_save" if args[0] == "true" else "k_fwd_wide"
        key = key + "_gate" if len(args) > 1 and args[1] == "true" else key
        return key + ("_seq" if len(args) > 2 and args[2] == "true" else "")
    if short.startswith("k_fwd_seg<"):
        args = [a.strip() for a in short[len("k_fwd_seg<"):-1].split(",")]
        seq = "_seq" if len(args) > 3 and args[3] == "true" else ""
        if args[0] == "true":
            save = "_save" if len(args) > 1 and args[1] == "true" else ""
            return "k_fwd_seg_state" + save + seq
        key = "k_fwd_seg_save" if len(args) > 1 and args[1] == "true" else "k_fwd_seg"
        return (key + "_gate" if len(args) > 2 and args[2] == "true" else key) + seq
    base = short.split("<")[0]
    if base == "k_bwd_ws":
        args = [a.strip() for a in short[len("k_bwd_ws<"):-1].split(",")]
        seq = "_seq" if len(args) > 2 and args[2] == "true" else ""
        if len(args) > 1 and args[1] != "0":
            return ("k_bwd_ws_rev_z" if args[0] == "true" else "k_bwd_ws_rev") + seq
        return "k_bwd_ws" + seq
    return base if base in ("k_bwd_dstate_rev", "k_bwd_run_grad", "k_chunk_cb", "k_fwd_state_group",
                            "k_state_pass_bwd") else short


SIMDS = 1024          # MI355X: 256 CUs x 4 SIMDs
PEAK_CLOCK_GHZ = 2.4  # MI355X peak engine clock


def summarize_sq(sq_dir, durations_ms):
    """Markdown table of per-kernel SQ counters (one rocprofv3 --pmc pass):
    MFMA pipe busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x duration x peak clock),
    wait = SQ_WAIT_ANY / SQ_WAVE_CYCLES, VALU = SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES
    (both wave-time fractions), LDS bank-conflict cycles per LDS-busy SIMD."""
    import csv
    import glob

    f = [x for x in glob.glob(os.path.join(sq_dir, "**", "*counter_collection.csv"), recursive=True)][0]
    per = {}
    for r in csv.DictReader(open(f)):
        if "ssd::" not in r["Kernel_Name"]:
            continue
        per.setdefault(_short(r["Kernel_Name"]), {}).setdefault(r["Counter_Name"], []).append(
            float(r["Counter_Value"]))
    lines = ["| kernel | MFMA instr | MFMA pipe busy | VALU instr | VALU active / wave time | "
             "waiting / wave time | LDS bank-conflict cycles |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for k, cs in per.items():
        m = {c: statistics.fmean(v) for c, v in cs.items()}
        dur = durations_ms.get(k)
        busy = (m.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (SIMDS * dur * 1e-3 * PEAK_CLOCK_GHZ * 1e9)
                if dur else float("nan"))
        wc = m.get("SQ_WAVE_CYCLES", float("nan"))
        lines.append(f"| `{k}` | {m.get('SQ_INSTS_MFMA', 0):.3e} | {100 * busy:.1f} % | "
                     f"{m.get('SQ_INSTS_VALU', 0):.3e} | {100 * m.get('SQ_ACTIVE_INST_VALU', 0) / wc:.1f} % | "
                     f"{100 * m.get('SQ_WAIT_ANY', 0) / wc:.1f} % | {m.get('SQ_LDS_BANK_CONFLICT', 0):.3e} |")
    return "\n".join(["### SQ counters (rocprofv3 --pmc, one pass)", "", *lines, ""])


def summarize_profiles(trace_dir, fetch_dir, write_dir, shape, copy_bytes=1 << 30, sq_dir=None):
    """Markdown summary of a rocprofv3 kernel-trace (--stats, csv) run and two
    --pmc runs (FETCH_SIZE, WRITE_SIZE; csv) of `bench.py --copy-calib`.

    Counter scale factors come from the last three dispatches of the runtime's
    copy kernel, which are the calibration copies of `copy_bytes` each.
    Returns (markdown, traffic dict keyed by kernel base name)."""
    import csv
    import glob

    def one(pattern):
        files = glob.glob(os.path.join(pattern, "**", "*"), recursive=True)
        return files

    stats_f = [f for f in one(trace_dir) if f.endswith("kernel_stats.csv")][0]
    rows = [r for r in csv.DictReader(open(stats_f)) if "ssd::" in r["Name"]]
    lines = ["| kernel | calls | avg ms | min ms | max ms | share of profiled time |",
             "|---|---:|---:|---:|---:|---:|"]
    for r in rows:
        lines.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e6:.4f} | "
                     f"{float(r['MinNs']) / 1e6:.4f} | {float(r['MaxNs']) / 1e6:.4f} | "
                     f"{float(r['Percentage']):.2f} % |")
    md = ["### Kernel durations (rocprofv3 --kernel-trace --stats)", "", *lines, ""]
    durations = {_short(r["Name"]): float(r["AverageNs"]) / 1e6 for r in rows}

    def counters(d):
        f = [x for x in one(d) if x.endswith("counter_collection.csv")][0]
        per, copies = {}, []
        for r in csv.DictReader(open(f)):
            v = float(r["Counter_Value"])
            if "ssd::" in r["Kernel_Name"]:
                per.setdefault(_short(r["Kernel_Name"]), []).append(v)
            elif "copyBuffer" in r["Kernel_Name"]:
                copies.append((int(r["Dispatch_Id"]), v))
        copies.sort()
        cal = [v for _, v in copies[-3:]]
        return {k: statistics.fmean(v) for k, v in per.items()}, statistics.fmean(cal)

    fetch, fcal = counters(fetch_dir)
    write, wcal = counters(write_dir)
    kib = copy_bytes / 1024
    fscale, wscale = kib / fcal, kib / wcal
    traffic = {}
    md += ["### HBM traffic per launch (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE)", "",
           f"Calibration: a plain {copy_bytes >> 20} MiB device copy reads FETCH_SIZE = {fcal:.0f} KiB "
           f"and WRITE_SIZE = {wcal:.0f} KiB per dispatch, so the counters are scaled by "
           f"{fscale:.3f} (fetch) and {wscale:.3f} (write).", "",
           "| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | scaled traffic GB | algorithmic GB (kernel model) |",
           "|---|---:|---:|---:|---:|"]
    folds = fwd_folds(shape)
    for k in fetch:
        t = (fetch[k] * fscale + write.get(k, 0.0) * wscale) * 1024
        key = model_key(k)
        if key == "k_state_pass" and folds:
            # the forward folds its segments itself, so every k_state_pass
            # launch of the run is the standalone op
            key = "k_state_pass_op"
        traffic[key] = t
        alg = fwd_kernel_model(key, shape)["bytes"]
        alg_s = "" if alg != alg else f"{alg / 1e9:.3f}"
        md.append(f"| `{k}` | {fetch[k]:.0f} | {write.get(k, 0.0):.0f} | {t / 1e9:.3f} | {alg_s} |")
    md.append("")
    if sq_dir:
        md.append(summarize_sq(sq_dir, durations))
    return "\n".join(md), traffic


# ----------------------------------------------------------------------------- main

def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=HEADLINE, choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--no-bwd", action="store_true", help="skip the fwd+bwd timing")
    ap.add_argument("--no-configs", action="store_true",
                    help="time only --config, not the other BASELINE configs")
    ap.add_argument("--no-full", action="store_true",
                    help="skip the full-feature (D, z, dt_bias, initial states, dt_limit) timings")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run 3 plain 1 GiB device copies (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--summarize-profile", nargs=3, metavar=("TRACE_DIR", "FETCH_DIR", "WRITE_DIR"),
                    help="print a markdown summary of rocprofv3 csv output and exit (no GPU)")
    ap.add_argument("--traffic-json", help="with --summarize-profile: also write per-kernel traffic")
    ap.add_argument("--sq-dir", help="with --summarize-profile: also summarize an SQ counter pass")
    args = ap.parse_args(argv)

    if args.summarize_profile:
        md, traffic = summarize_profiles(*args.summarize_profile, CONFIGS[args.config],
                                         sq_dir=args.sq_dir)
        print(md)
        if args.traffic_json:
            with open(args.traffic_json, "w") as fh:
                json.dump({"config": CONFIGS[args.config], "traffic_bytes": traffic}, fh, indent=1)
        return 0

    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (asked for --gpus {args.gpus}): the SSD hot path "
              "is a single-device operator here (it would shard over (batch, group) streams, "
              "which share nothing in the forward).",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    import ascend_kernel
    from ascend_kernel import _runtime as rt
    from ascend_kernel import mamba2 as api

    lib = rt.load_library()
    hip = HipEvents()
    shape = CONFIGS[args.config]
    b, l, h, p, n, chunk, g = shape
    seed = 20260806 + (args.config - 1)
    dev = torch.cuda.get_device_properties(0)
    log(f"device {dev.name} ({getattr(dev, 'gcnArchName', '?')}), config C{args.config} {shape}, "
        f"seed {seed}")

    cpu_inp = make_cpu_inputs(torch, shape, seed)
    inp = to_gpu(torch, cpu_inp)
    log("inputs ready (CPU generator, copied to the GPU); forward warmup + timed steps")
    res, names, wall_ms, finite, ws_bytes, out, final = bench_forward(
        torch, lib, rt, api, hip, inp, shape, args.steps, args.warmup)
    step_ms = [r[0] for r in res]
    fwd_ms = statistics.median(step_ms)
    kern = {}
    for i, name in enumerate(names):
        durs = [r[1][i] for r in res]
        model = fwd_kernel_model(name, shape)
        avg = statistics.fmean(durs)
        kern[name] = {
            "avg_ms": avg,
            "median_ms": statistics.median(durs),
            "GB_s": model["bytes"] / (avg * 1e-3) / 1e9,
            "TFLOP_s": model["flops"] / (avg * 1e-3) / 1e12,
            "bytes": model["bytes"],
            "flops": model["flops"],
        }
        log(f"  {name:<16} avg {avg:8.4f} ms  {kern[name]['GB_s']:8.1f} GB/s  "
            f"{kern[name]['TFLOP_s']:7.2f} TFLOP/s")
    log(f"forward median {fwd_ms:.4f} ms (wall {wall_ms / args.steps:.4f} ms/step), finite={finite}")
    fwd_stats = summarize(step_ms)
    out_sums = checksums(torch, {"out": out, "final": final})[0]
    parity = parity_slices(torch, cpu_inp, out, final, shape, PARITY_SLICES[args.config])
    log(f"same-run parity vs the CPU oracle on {parity['slices']}: out maxabs {parity['out_maxabs']:.3e} "
        f"relL2 {parity['out_relL2']:.3e}, final maxabs {parity['final_maxabs']:.3e} relL2 "
        f"{parity['final_relL2']:.3e} -> {'pass' if parity['pass'] else 'FAIL'}")
    del out, final

    api_ms = bench_api(torch, api, inp, chunk, max(5, args.steps // 3), 3)
    log(f"public API forward median {api_ms:.4f} ms per call (runs of 5 consecutive calls)")

    fwd_bwd_ms, bwd_note, api_fwd_bwd_ms, bwd_kern, bwd_ms = None, "skipped (--no-bwd)", None, {}, None
    memory = None
    fwd_train_ms = None
    train_stats, grad_sums = {}, None
    if not args.no_bwd:
        tr = bench_fwd_bwd_traced(torch, lib, rt, hip, inp, shape, args.steps, args.warmup)
        if tr is None:
            bwd_note = "M1 backward needs headdim == dstate == 64"
        else:
            fres, bres, bnames, bfinite = tr[:4]
            bwd_ms = statistics.median(r[0] for r in bres)
            fwd_train_ms = statistics.median(r[0] for r in fres)
            fwd_bwd_ms = statistics.median(f[0] + bk[0] for f, bk in zip(fres, bres))
            train_stats = {"fwd_train": summarize(r[0] for r in fres), "bwd": summarize(r[0] for r in bres),
                           "fwd_bwd": summarize(f[0] + bk[0] for f, bk in zip(fres, bres))}
            grad_sums = {"gradient_checksums": tr[6][0], "gradient_checksum": tr[6][1]}
            bwd_note = ("C-ABI training fwd (saves chunk-start states) + M1 bwd, loss "
                        f"mean(y^2)+mean(final^2), grads finite={bfinite}")
            log(f"training forward (saving chunk states) median {fwd_train_ms:.4f} ms")
            for i, name in enumerate(bnames):
                durs = [r[1][i] for r in bres]
                avg = statistics.fmean(durs)
                model = fwd_kernel_model(name, shape)
                bwd_kern[name] = {"avg_ms": round(avg, 6),
                                  "median_ms": round(statistics.median(durs), 6)}
                if model["bytes"] == model["bytes"]:
                    bwd_kern[name]["GB_s"] = round(model["bytes"] / (avg * 1e-3) / 1e9, 1)
                    bwd_kern[name]["TFLOP_s"] = round(model["flops"] / (avg * 1e-3) / 1e12, 2)
                    bwd_kern[name]["traffic"] = measured_traffic(name, shape)
                log(f"  bwd {name:<18} avg {avg:8.4f} ms"
                    + (f"  {bwd_kern[name]['GB_s']:8.1f} GB/s  {bwd_kern[name]['TFLOP_s']:7.2f} TFLOP/s"
                       if "GB_s" in bwd_kern[name] else ""))
            fnames = tr[5]
            for i, name in enumerate(fnames):
                durs = [r[1][i] for r in fres]
                avg = statistics.fmean(durs)
                model = fwd_kernel_model(name, shape)
                log(f"  train {name:<16} avg {avg:8.4f} ms  {model['bytes'] / (avg * 1e-3) / 1e9:8.1f} GB/s")
            log(f"bwd median {bwd_ms:.4f} ms; fwd+bwd median {fwd_bwd_ms:.4f} ms")
            api_fwd_bwd_ms, _ = bench_fwd_bwd(torch, api, inp, chunk, max(5, args.steps // 3), 3)
            log(f"public API (autograd) fwd+bwd median {api_fwd_bwd_ms:.4f} ms per step "
                "(runs of 3 consecutive steps)")
            memory = autograd_memory(torch, api, inp, chunk)
            log(f"autograd memory (keep chunk states): saved {memory['saved_bytes'] / 2**30:.3f} GiB "
                f"beyond the inputs, peak {memory['peak_extra_bytes'] / 2**30:.3f} GiB above inputs + "
                "upstream grads")
            # the other training policy: chunk-start states recomputed in the backward
            rec_ms, _ = bench_fwd_bwd(torch, api, inp, chunk, max(5, args.steps // 3), 3, save=False)
            rec_mem = autograd_memory(torch, api, inp, chunk, save=False)
            memory = {**memory, "policy": "save_chunk_states=True",
                      "recompute": {**rec_mem, "api_fwd_bwd_ms": rec_ms, "policy": "save_chunk_states=False"}}
            log(f"recompute policy: fwd+bwd {rec_ms:.4f} ms per step, saved "
                f"{rec_mem['saved_bytes'] / 2**30:.3f} GiB, peak {rec_mem['peak_extra_bytes'] / 2**30:.3f} GiB")
    packed = None
    if not args.no_full and shape[3] == 64 and shape[4] in (64, 128):
        # packed sequences (seq_idx) on the same shape: the cost of the masks
        seq = packed_ids(torch, shape, seed)
        nfs = max(10, args.steps // 2)
        # the same call path without ids, timed back to back with the packed
        # calls, so the pair shows the masks' cost under the same conditions
        plain = bench_fwd_features(torch, lib, rt, inp, shape, None, nfs, 3)
        pk = bench_fwd_features(torch, lib, rt, inp, shape, None, nfs, 3, seq=seq)
        packed = {"ids": "every row cut into sequences of U[256, 2048) tokens",
                  "nseqs": int((seq[:, 1:] != seq[:, :-1]).sum().item()) + shape[0],
                  "fwd_ms": pk["median_ms"], "fwd": pk,
                  "fwd_ms_without_ids": plain["median_ms"], "fwd_without_ids": plain}
        log(f"packed sequences ({packed['nseqs']}): forward median {packed['fwd_ms']:.4f} ms "
            f"(same path without ids {plain['median_ms']:.4f} ms)")
        if not args.no_bwd:
            tr = bench_fwd_bwd_traced(torch, lib, rt, hip, inp, shape, nfs, 3, seq=seq)
            if tr is not None:
                fres, bres = tr[0], tr[1]
                packed["fwd_train_ms"] = round(statistics.median(r[0] for r in fres), 5)
                packed["bwd_ms"] = round(statistics.median(r[0] for r in bres), 5)
                packed["fwd_bwd_ms"] = round(statistics.median(f[0] + bk[0] for f, bk in zip(fres, bres)), 5)
                packed["fwd_train"] = summarize(r[0] for r in fres)
                packed["bwd"] = summarize(r[0] for r in bres)
                packed["fwd_bwd"] = summarize(f[0] + bk[0] for f, bk in zip(fres, bres))
                packed["grads_finite"] = bool(tr[3])
                packed["gradient_checksums"], packed["gradient_checksum"] = tr[6]
                log(f"packed sequences: training forward {packed['fwd_train_ms']:.4f} ms, bwd "
                    f"{packed['bwd_ms']:.4f} ms, fwd+bwd {packed['fwd_bwd_ms']:.4f} ms")
        del seq
        torch.cuda.empty_cache()
    full = None
    if not args.no_full:
        # the reference's headline feature set on the same shape
        feats = full_features(torch, shape, seed)
        nfs = max(5, args.steps // 3)
        ff = bench_fwd_features(torch, lib, rt, inp, shape, feats, nfs, 3)
        full = {"features": "D [H,P], z, dt_bias, initial_states, softplus, dt_limit (1e-3, 1)",
                "fwd_ms": ff["median_ms"], "fwd": ff}
        log(f"full features: forward median {full['fwd_ms']:.4f} ms")
        if not args.no_bwd:
            tr = bench_fwd_bwd_traced(torch, lib, rt, hip, inp, shape, nfs, 3, feats)
            if tr is not None:
                fres, bres = tr[0], tr[1]
                full["fwd_train_ms"] = round(statistics.median(r[0] for r in fres), 5)
                full["bwd_ms"] = round(statistics.median(r[0] for r in bres), 5)
                full["fwd_bwd_ms"] = round(statistics.median(f[0] + bk[0] for f, bk in zip(fres, bres)), 5)
                full["fwd_train"] = summarize(r[0] for r in fres)
                full["bwd"] = summarize(r[0] for r in bres)
                full["fwd_bwd"] = summarize(f[0] + bk[0] for f, bk in zip(fres, bres))
                full["grads_finite"] = bool(tr[3])
                full["gradient_checksums"], full["gradient_checksum"] = tr[6]
                log(f"full features: training forward {full['fwd_train_ms']:.4f} ms, bwd "
                    f"{full['bwd_ms']:.4f} ms, fwd+bwd {full['fwd_bwd_ms']:.4f} ms")
        del feats
        torch.cuda.empty_cache()
    if args.copy_calib:
        copy_calibration(torch, 1 << 30)
        log("copy calibration: 3 x 1 GiB device copies")

    flops, nbytes = op_work(shape)
    dom = max(kern, key=lambda k: kern[k]["avg_ms"])
    d = kern[dom]
    roofline = {
        "kernel": dom,
        "bound": "hbm",
        "achieved": d["GB_s"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": d["GB_s"] / HBM_PEAK_GBS,
        "traffic": measured_traffic(dom, shape),
    }
    del inp
    torch.cuda.empty_cache()
    others = {}
    if not args.no_configs:
        # the other BASELINE configs, each with its own inputs and parity slice
        for cfg in sorted(CONFIGS):
            if cfg == args.config:
                continue
            row = bench_config(torch, lib, rt, api, hip, cfg, args.steps, args.warmup, cpu=not args.no_cpu)
            others[f"C{cfg}"] = row
            log(f"config C{cfg} {row['shape']}: forward {row['fwd_ms']:.4f} ms (public API "
                f"{row['api_fwd_ms']:.4f} ms per call, {row['api_host_us']:.0f} us of host work per call), "
                f"{row['op_GB_s']:.0f} GB/s "
                f"({100 * row['hbm_roofline_frac']:.1f} % of 8 TB/s), parity "
                f"{'pass' if row['parity']['pass'] else 'FAIL'} (out relL2 {row['parity']['out_relL2']:.2e})"
                + (f"; training fwd {row['fwd_train_ms']:.4f} + bwd {row['bwd_ms']:.4f} ms"
                   if "bwd_ms" in row else ""))
    copy_gbs = copy_bandwidth(torch)
    log(f"device copy (1 GiB, read + write) {copy_gbs:.0f} GB/s: the dominant kernel streams at "
        f"{d['GB_s'] / copy_gbs:.2f} of it")
    roofline["copy_GB_s"] = round(copy_gbs, 1)
    roofline["frac_of_copy"] = d["GB_s"] / copy_gbs
    decode = bench_decode(torch, shape)
    log(f"decode step (selective_state_update) batch {decode['batch']} on [H,P,N,G] = "
        f"{decode['shape'][1:]}: {decode['ms']:.4f} ms, {decode['GB_s']:.0f} GB/s "
        f"(whole Python call {decode['api_ms']:.4f} ms)")
    state_pass = bench_state_passing(torch, lib, shape)
    state_pass["frac_of_copy"] = state_pass["GB_s"] / copy_gbs
    log(f"state passing op on [B,H,K,P,N] = {shape[0]},{shape[2]},{math.ceil(shape[1] / EXEC_CHUNK)},"
        f"{shape[3]},{shape[4]}: {state_pass['ms']:.4f} ms, {state_pass['GB_s']:.0f} GB/s "
        f"({100 * state_pass['frac']:.0f} % of 8 TB/s)")

    cpu = None
    if not args.no_cpu:
        log(f"CPU oracle baseline: the whole C{args.config} forward on the same inputs")
        cpu = cpu_oracle_baseline(torch, cpu_inp, shape, seed)
        log(f"cpu baseline {cpu['value']:.1f} ms (median of {cpu['stats']['n']}), {cpu['cores']} threads")
    del cpu_inp

    line = {
        "metric": METRIC,
        "value": round(fwd_ms, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms / args.steps, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic (seeded CPU generator, copied to the GPU; x,B,C~N(0,1), dt~U[0,1), "
                 "A=-U[0,1))"),
        "config": {
            "workload": f"C{args.config} SSD forward [B,L,H,P,N,chunk,G]={shape}, dt_softplus, "
                        "final state, fp32 public tensors, split-fp16 MFMA operands",
            "shape": shape,
            "seed": seed,
        },
        "fwd": fwd_stats,
        "output_checksums": out_sums,
        **train_stats,
        **(grad_sums or {}),
        "fwd_bwd_ms": None if fwd_bwd_ms is None else round(fwd_bwd_ms, 5),
        "fwd_train_ms": None if fwd_train_ms is None else round(fwd_train_ms, 5),
        "bwd_ms": None if bwd_ms is None else round(bwd_ms, 5),
        "fwd_bwd_note": bwd_note,
        "api_fwd_bwd_ms": None if api_fwd_bwd_ms is None else round(api_fwd_bwd_ms, 5),
        "bwd_kernels": bwd_kern,
        "api_fwd_ms": round(api_ms, 5),
        "state_passing": state_pass,
        "decode_step": decode,
        "autograd_memory": memory,
        "full_features": full,
        "packed_sequences": packed,
        "op": {
            "flops": flops,
            "bytes": nbytes,
            "TFLOP_s": flops / (fwd_ms * 1e-3) / 1e12,
            "GB_s": nbytes / (fwd_ms * 1e-3) / 1e9,
            "hbm_roofline_frac": (nbytes / (fwd_ms * 1e-3) / 1e9) / HBM_PEAK_GBS,
        },
        "kernels": {k: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kern.items()},
        "workspace_bytes": ws_bytes,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": parity,
        "configs": others,
        "finite": finite,
        "device": dev.name,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
