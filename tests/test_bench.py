"""CPU checks of bench.py: the one-GPU contract, the kernel models the roofline
line uses, and the mapping of traced kernel names onto them."""

import math

import bench


def test_more_than_one_gpu_exits_with_a_message(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "exactly one GPU" in capsys.readouterr().err


def test_forward_model_matches_the_documented_bytes():
    """C3: 4 (2 T P + T + 2 T N / R) bytes per (b, h, chunk) unit, 131072
    units (41.2 KB and 5.402 GB); the flops are the op-level formula's."""
    shape = bench.CONFIGS[3]
    m = bench.fwd_kernel_model("k_fwd_seg", shape)
    T, P, N, R = 64, 64, 64, 4
    assert m["units"] == 8 * 256 * 64
    assert m["bytes_per_unit"] == 4 * (2 * T * P + T + 2 * T * N / R)
    assert math.isclose(m["bytes"] / 1e9, 5.402, rel_tol=1e-3)
    flops, _ = bench.op_work(shape)
    assert math.isclose(m["flops"], flops, rel_tol=1e-12)
    # the training forward adds the state entering each chunk
    save = bench.fwd_kernel_model("k_fwd_seg_save", shape)
    assert save["bytes"] - m["bytes"] == 4 * P * N * m["units"]
    # packed sequences move the same tensors
    assert bench.fwd_kernel_model("k_fwd_seg_seq", shape)["bytes"] == m["bytes"]


def test_traced_names_map_to_distinct_models():
    key = bench.model_key
    assert key("k_fwd_seg<false, false, false, false>") == "k_fwd_seg"
    assert key("k_fwd_seg<false, true, false, false>") == "k_fwd_seg_save"
    assert key("k_fwd_seg<false, false, true, false>") == "k_fwd_seg_gate"
    assert key("k_fwd_seg<false, true, true, true>") == "k_fwd_seg_save_gate_seq"
    assert key("k_fwd_seg<true, false, false, true>") == "k_fwd_seg_state_seq"
    # the backward's recompute pass writes the chunk states: its own model
    assert key("k_fwd_seg<true, true, false, false>") == "k_fwd_seg_state_save"
    assert key("k_bwd_ws<false, 4, false>") == "k_bwd_ws_rev"
    assert key("k_bwd_ws<true, 2, false>") == "k_bwd_ws_rev_z"
    assert key("k_bwd_ws<false, 4, true>") == "k_bwd_ws_rev_seq"
    assert key("k_bwd_ws<true, 0, false>") == "k_bwd_ws"
    assert key("k_fwd_wide<false, false, false>") == "k_fwd_wide"
    assert key("k_fwd_wide<true, true, false>") == "k_fwd_wide_save_gate"
    assert key("k_fwd_wide<false, false, true>") == "k_fwd_wide_seq"
    assert bench._short("void ssd::bwd::k_bwd_ws<false, 4, false>(ssd::BwdParams, int, int)") == \
        "k_bwd_ws<false, 4, false>"
    assert key("k_state_pass") == "k_state_pass"
    # the latency form of one-round grids is the same pass
    assert key("k_fwd_seg<false, false, false, false, true>") == "k_fwd_seg"
    assert key("k_fwd_seg<false, true, false, false, true>") == "k_fwd_seg_save"
    shape = bench.CONFIGS[3]
    for name in ("k_fwd_seg_gate", "k_fwd_seg_save_gate", "k_bwd_ws_rev", "k_bwd_ws_rev_z", "k_fwd_wide",
                 "k_fwd_wide_gate"):
        assert not math.isnan(bench.fwd_kernel_model(name, shape)["bytes"]), name


def test_recompute_pass_model_counts_the_state_writes():
    """k_fwd_seg<state only, save> reads x, dt and B and writes the state
    entering every chunk: 4 (T P + T + T N / R + P N) bytes per unit (4.87 GB
    at C3, of which 2.15 GB are the states)."""
    shape = bench.CONFIGS[3]
    st = bench.fwd_kernel_model("k_fwd_seg_state", shape)
    sv = bench.fwd_kernel_model("k_fwd_seg_state_save", shape)
    assert sv["bytes"] - st["bytes"] == 4 * 64 * 64 * sv["units"]
    assert math.isclose(sv["bytes"] / 1e9, 4.865, rel_tol=1e-3)
    # the group-major form of the same pass moves the same algorithmic bytes
    assert bench.fwd_kernel_model("k_fwd_state_group", shape) == sv
    assert bench.model_key(bench._short("void ssd::k_fwd_state_group<4>(ssd::FwdParams)")) == "k_fwd_state_group"


def test_summary_statistics():
    s = bench.summarize([5.0, 1.0, 3.0, 2.0, 4.0, 6.0, 7.0, 8.0, 9.0, 10.0])
    assert s["median_ms"] == 5.5 and s["min_ms"] == 1.0 and s["max_ms"] == 10.0
    assert s["p90_ms"] == 9.0 and s["n"] == 10 and s["mean_ms"] == 5.5


def test_standalone_state_pass_model_matches_the_op_timing():
    """Profiles attribute the k_state_pass launches of a config run to the
    standalone state-passing op whenever the forward folds its segments (all
    five configs); that model is the op's own byte count, the one
    bench_state_passing divides by (chunk states in, states entering the
    chunks out, log decays, final state)."""
    for cfg in sorted(bench.CONFIGS):
        shape = bench.CONFIGS[cfg]
        assert bench.fwd_folds(shape), cfg
        b, l, h, p, n, _chunk, _g = shape
        k = math.ceil(l / bench.EXEC_CHUNK)
        want = 4 * (2 * b * h * k * p * n + b * h * k + b * h * p * n)
        assert bench.fwd_kernel_model("k_state_pass_op", shape)["bytes"] == want
    # many pre-segments: the forward runs the segment recurrence itself
    assert not bench.fwd_folds([1, 65536, 8, 64, 64, 64, 1])
