#!/usr/bin/env python3
"""Benchmark of the MI355X Mamba-2 SSD hot path on one GPU.

Workload: the headline configuration [B,L,H,P,N,chunk,G] = [8,4096,256,64,64,64,64]
(x, dt, A, B, C; dt_softplus=True, return_final_state=True; fp32 public tensors),
synthetic inputs drawn on the GPU with the benchmark distributions (x, B, C ~ N(0,1),
dt ~ U[0,1), A = -U[0,1)).  A "step" is one forward call over that batch; when the
backward is available the fwd+bwd time (loss mean(y^2) + mean(final^2)) is reported
beside it.

Protocol (the reference's: benchmarks/mamba2_backward_bench.py:354-389, warmup 10 /
repeat 30, median of per-call device events): every kernel of a call is bracketed by
HIP events on the launch stream (the library's *_traced entry points), so the per-kernel
durations used for the roofline come from the timed region itself.  The wall-clock
time of the K steps, bracketed by device synchronisation, gives ms_per_step.

CPU baseline: the repository's fp32 CPU oracle (oracle/ssd_reference.py, a restatement
of the reference's mamba_torch/ssd_reference.py) timed on a bounded sample of the same
workload (batch 0, the first few groups) on this host's cores, scaled to the full
configuration by the number of independent (batch, group) units.

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
    if name == "k_chunk_state":
        per = f4 * (T * p + T + T * n / r + p * n + 1)
        fl = 2 * T * p * n
    elif name == "k_state_pass":
        per = f4 * (2 * p * n + 1)
        fl = 2 * p * n
        return {"bytes": units * per + b * h * p * n * f4, "flops": units * fl, "units": units,
                "bytes_per_unit": per}
    elif name == "k_chunk_scan":
        per = f4 * (2 * T * p + T + p * n + 2 * T * n / r)
        fl = 2 * (T * T * n / r + T * T * p + T * n * p)
    else:
        per, fl = float("nan"), float("nan")
    return {"bytes": units * per, "flops": units * fl, "units": units, "bytes_per_unit": per}


def op_work(shape):
    """Op-level algorithmic work: F = 2*B*L*[G*T*N + H*(T*P + 2*N*P)] and the
    compulsory fp32 public I/O bytes (x, out, dt, A, B, C, final)."""
    b, l, h, p, n, chunk, g = shape
    T = EXEC_CHUNK
    flops = 2 * b * l * (g * T * n + h * (T * p + 2 * n * p))
    nbytes = 4 * (2 * b * l * h * p + b * l * h + h + 2 * b * l * g * n + b * h * p * n)
    return flops, nbytes


# ----------------------------------------------------------------------------- GPU runs

def make_gpu_inputs(torch, shape, seed):
    b, l, h, p, n, _chunk, g = shape
    gen = torch.Generator(device="cuda").manual_seed(seed)
    kw = dict(device="cuda", dtype=torch.float32, generator=gen)
    return {
        "x": torch.randn(b, l, h, p, **kw),
        "dt": torch.rand(b, l, h, **kw),
        "A": -torch.rand(h, **kw),
        "B": torch.randn(b, l, g, n, **kw),
        "C": torch.randn(b, l, g, n, **kw),
    }


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
    return res, names, wall, ok, ws.numel()


def bench_api(torch, api, inp, chunk, steps, warmup):
    """Per-call device-event time through the public Python API."""
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
        call()
        e.record()
        e.synchronize()
        samples.append(s.elapsed_time(e))
    return statistics.median(samples)


def bench_fwd_bwd(torch, api, inp, chunk, steps, warmup):
    """fwd + bwd through autograd (loss mean(y^2) + mean(final^2)); None if the
    backward is not available for this shape."""
    leaves = {k: v.detach().clone().requires_grad_(True) for k, v in inp.items()}

    def call():
        for v in leaves.values():
            v.grad = None
        out, fin = api.mamba2_ssd_fwd(leaves["x"], leaves["dt"], leaves["A"], leaves["B"],
                                      leaves["C"], chunk, dt_softplus=True,
                                      return_final_state=True)
        (out.pow(2).mean() + fin.pow(2).mean()).backward()

    try:
        call()
        torch.cuda.synchronize()
    except (NotImplementedError, RuntimeError) as exc:
        log(f"fwd+bwd unavailable: {exc}")
        return None, str(exc).splitlines()[0][:200]
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
    return statistics.median(samples), None


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


def cpu_baseline(torch, shape, seed, budget_s):
    """Oracle forward on batch 0 and the first `gs` groups; scaled to the full config."""
    from oracle.ssd_reference import make_inputs, ssd_chunk_scan_ref

    b, l, h, p, n, chunk, g = shape
    r = h // g
    torch.set_num_threads(os.cpu_count() or 1)

    def sample(gs):
        sub = [1, l, gs * r, p, n, chunk, gs]
        inp = make_inputs(sub, seed)
        t0 = time.perf_counter_ns()
        with torch.no_grad():
            ssd_chunk_scan_ref(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], chunk,
                               dt_softplus=True, return_final_state=True)
        return (time.perf_counter_ns() - t0) / 1e6

    one = sample(1)  # also the warmup
    gs = int(max(1, min(g, (budget_s / 3 * 1e3) // max(one, 1e-3))))
    times = [sample(gs) for _ in range(3)]
    med = statistics.median(times)
    scale = (b * g) / gs
    return {
        "value": med * scale,
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle fp32 forward on batch 0, groups 0..{gs - 1} ({gs * r} heads, "
                   f"L={l}) of the workload: median of 3 = {med:.1f} ms, x{scale:g} "
                   f"(independent (batch, group) units) to the full config"),
        "host": host_info(),
        "torch": torch.__version__,
    }


# ----------------------------------------------------------------------------- main

def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=HEADLINE, choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--no-bwd", action="store_true", help="skip the fwd+bwd timing")
    ap.add_argument("--cpu-budget", type=float, default=20.0,
                    help="approximate seconds of CPU-oracle work for the baseline")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (asked for --gpus {args.gpus}): the SSD hot path "
              "is a single-device operator here; see DESIGN.md for how it would shard.",
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

    inp = make_gpu_inputs(torch, shape, seed)
    torch.cuda.synchronize()
    log("inputs ready; forward warmup + timed steps")
    res, names, wall_ms, finite, ws_bytes = bench_forward(torch, lib, rt, api, hip, inp, shape,
                                                          args.steps, args.warmup)
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

    api_ms = bench_api(torch, api, inp, chunk, max(5, args.steps // 3), 3)
    log(f"public API forward median {api_ms:.4f} ms")

    fwd_bwd_ms, bwd_note = (None, "skipped (--no-bwd)")
    if not args.no_bwd:
        fwd_bwd_ms, bwd_note = bench_fwd_bwd(torch, api, inp, chunk, max(5, args.steps // 3), 3)
        if fwd_bwd_ms is not None:
            log(f"fwd+bwd median {fwd_bwd_ms:.4f} ms")

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
        "traffic": None,
    }
    del inp
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("CPU oracle baseline (bounded sample)")
        cpu = cpu_baseline(torch, shape, seed, args.cpu_budget)
        log(f"cpu baseline {cpu['value']:.1f} ms (scaled), {cpu['cores']} threads")

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
        "data": "synthetic (seeded GPU generator; x,B,C~N(0,1), dt~U[0,1), A=-U[0,1))",
        "config": {
            "workload": f"C{args.config} SSD forward [B,L,H,P,N,chunk,G]={shape}, dt_softplus, "
                        "final state, fp32 public tensors, split-fp16 MFMA operands",
            "shape": shape,
            "seed": seed,
        },
        "fwd_bwd_ms": None if fwd_bwd_ms is None else round(fwd_bwd_ms, 5),
        "fwd_bwd_note": bwd_note,
        "api_fwd_ms": round(api_ms, 5),
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
        "finite": finite,
        "device": dev.name,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
