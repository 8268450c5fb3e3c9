"""Host-side checks of bench.py's workload definitions (no GPU)."""

import math
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_c4_clips_follow_the_reference_draws():
    clips = bench.c4_clips()
    assert len(clips) == 128
    # 23 one-second buckets and 1706 s of audio for the random.Random(0)
    # sequence of scripts/bench_e2e.py:137-143 (uniform length, then a start)
    assert len({L for L, _ in clips}) == 23
    assert abs(sum(lk for _, lk in clips) / 50.0 - 1706.36) < 1e-6
    for L, lk in clips:
        assert L % 50 == 0 and 1 <= lk <= L and L - 50 < lk
        assert 75 <= lk <= 1250


def test_attention_flops_at_c3():
    # 4 B H L^2 D + 2 B H L 73 D at L=4800: 95.09 GFLOP per layer
    assert math.isclose(bench.attention_flops(16, 4800, 4800), 95.09e9, rel_tol=1e-3)


def test_encoder_flops_at_96s():
    # per layer: FFN 2 x (2 x 1024 x 4096), QKV 3 x 1024^2, out 1024^2, pointwise
    # convs 2 x 1024^2 + 1024^2 (multiply-adds), plus the feature projection, the
    # depthwise conv and the attention: 2617 GFLOP per 96 s chunk
    gemm = 2.0 * 4800 * (160 * 1024 + 8 * (4 * 1024 * 4096 + 4 * 1024 * 1024 + 3 * 1024 * 1024))
    conv = 8 * 2.0 * 4800 * 1024 * 31
    attn = 8 * bench.attention_flops(16, 4800, 4800)
    assert math.isclose(bench.encoder_flops(4800), gemm + conv + attn, rel_tol=1e-12)
    assert math.isclose(bench.encoder_flops(4800), 2617e9, rel_tol=1e-3)


def test_encoder_model_weights_shapes():
    import torch

    w = bench.encoder_model_weights(torch, layers=1)
    p = w["layers"][0]
    assert w["heads"] == 16 and w["fp_w"].shape == (1024, 160)
    assert p["ffn1_w1"].shape == (4096, 1024) and p["ffn2_w2"].shape == (1024, 4096)
    assert p["pw1_w"].shape == (2048, 1024) and p["dw_w"].shape == (1024, 31) and p["rel"].shape == (73, 64)


def test_host_cpu_reports_this_host():
    import os

    info = bench.host_cpu()
    assert info["cpu_count"] == os.cpu_count()
    assert 1 <= info["affinity"] <= os.cpu_count()
    assert info["model"] is None or isinstance(info["model"], str)


def test_summarize_counters_known_answer():
    """Traffic = KiB read by each counter x 1024 x (copy bytes / copy KiB),
    medians over the attention dispatches only; clock = GRBM_GUI_ACTIVE / 8
    XCDs / duration.  Fabricated readings with a closed-form answer: the copy
    passes read half the copied KiB for FETCH_SIZE (factor 2) and all of it
    for WRITE_SIZE (factor 1)."""
    import bench

    copy_kib = bench.COPY_PROBE_BYTES / 1024.0
    names = {"1": "flexrel_w64_kernel", "2": "flexrel_w64_kernel", "3": "flexrel_w64_kernel", "9": "Cijk_gemm"}
    fetch = {"1": {"FETCH_SIZE": 100.0, "GRBM_GUI_ACTIVE": 8 * 2000.0}, "2": {"FETCH_SIZE": 110.0, "GRBM_GUI_ACTIVE": 8 * 2100.0},
             "3": {"FETCH_SIZE": 120.0, "GRBM_GUI_ACTIVE": 8 * 2200.0}, "9": {"FETCH_SIZE": 1e9, "GRBM_GUI_ACTIVE": 1.0}}
    dur = {"1": 1000.0, "2": 1000.0, "3": 1000.0, "9": 5.0}
    write = {"1": {"WRITE_SIZE": 40.0}, "2": {"WRITE_SIZE": 50.0}, "3": {"WRITE_SIZE": 60.0}, "9": {"WRITE_SIZE": 1e9}}
    cnames = {"7": "__amd_rocclr_copyBuffer"}
    per = {"kernel_fetch": (fetch, names, dur), "kernel_write": (write, names, {}),
           "copy_fetch": ({"7": {"FETCH_SIZE": copy_kib / 2}}, cnames, {}),
           "copy_write": ({"7": {"WRITE_SIZE": copy_kib}}, cnames, {})}
    res = bench.summarize_counters(per)
    assert res["dispatches"] == 3
    assert math.isclose(res["fetch_factor"], 2.0) and math.isclose(res["write_factor"], 1.0)
    assert math.isclose(res["traffic_bytes"], 110.0 * 1024 * 2 + 50.0 * 1024)
    assert math.isclose(res["sclk_mhz"], 2100.0 / 1000.0 * 1e3)   # 2100 cycles per XCD in 1000 ns
    assert math.isclose(res["traffic_over_algorithmic"], res["traffic_bytes"] / bench.ALGO_BYTES)
    # the c3 algorithmic bytes: q, k, v read and the output written once, the table, the length
    assert bench.ALGO_BYTES == 4 * 4800 * 1024 * 2 + 73 * 64 * 2 + 4


def test_summarize_counters_mfma_busy_known_answer():
    """Matrix-core occupancy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8)
    / 1024 SIMDs, and the useful fraction = the launch's flops / (1024 flop
    per SIMD-cycle x 1024 SIMDs x cycles).  Fabricated readings: 200 k cycles
    per XCD and a busy count of half of 1024 x 200 k give 0.5."""
    import bench

    copy_kib = bench.COPY_PROBE_BYTES / 1024.0
    names = {"1": "flexrel_w64_kernel", "2": "flexrel_w64_kernel", "3": "flexrel_w64_kernel"}
    cyc = 200e3
    fetch = {d: {"FETCH_SIZE": 1.0, "GRBM_GUI_ACTIVE": 8 * cyc} for d in names}
    write = {d: {"WRITE_SIZE": 1.0, "GRBM_GUI_ACTIVE": 8 * cyc, "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * 1024 * cyc,
                 "SQ_BUSY_CYCLES": 7.0} for d in names}
    dur = {d: 1e5 for d in names}
    cnames = {"7": "__amd_rocclr_copyBuffer"}
    per = {"kernel_fetch": (fetch, names, dur), "kernel_write": (write, names, {}),
           "copy_fetch": ({"7": {"FETCH_SIZE": copy_kib / 2}}, cnames, {}),
           "copy_write": ({"7": {"WRITE_SIZE": copy_kib}}, cnames, {})}
    res = bench.summarize_counters(per)
    assert math.isclose(res["mfma_busy_frac"], 0.5)
    assert math.isclose(res["cycles_per_launch"], cyc)
    assert math.isclose(res["mfma_useful_frac"], bench.FLOPS_LAUNCH / 1024.0 / cyc / 1024.0)
    # 95.09 GFLOP in 200 k cycles: 0.4534 of the matrix cores' capacity at that clock
    assert math.isclose(res["mfma_useful_frac"], 0.4534, rel_tol=1e-3)
    assert res["sq_busy_cycles"] == 7.0
