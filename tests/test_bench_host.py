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
