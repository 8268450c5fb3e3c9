"""Pin the CPU oracle (no GPU).

Each oracle function is checked against something that does not share its
code: golden vectors written by the installed transformers module, scalar
brute force, torch's scaled_dot_product_attention in closed-form special
cases, and invariants of the math.  Planted mistakes in the oracle's formula
must be caught by the golden check.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import seeded_inputs
from oracle.flexrel_oracle import (attention_flops, errors, flexrel_bruteforce,
                                   flexrel_reference, flexrel_tiled, torch_core_chunked)


def _valid_rows_err(ref, got, lens):
    worst = 0.0
    for b, lk in enumerate(lens):
        if lk:
            worst = max(worst, float(np.abs(ref[b, :, :lk] - got[b, :, :lk]).max()))
    return worst


def test_reference_matches_transformers_golden(golden_cases):
    assert len(golden_cases) >= 3
    for name, d in golden_cases.items():
        ref = flexrel_reference(d["q"], d["k"], d["v"], d["rel"], d["lens"])
        # expected is float32-rounded transformers float64 output
        assert _valid_rows_err(d["expected"], ref, d["lens"]) < 1e-6, name


def test_bruteforce_matches_transformers_golden(golden_cases):
    d = golden_cases["hf_b1_h2_l40"]
    # a 12-row slice keeps the scalar loops fast; keys are the full 40
    sl = slice(0, 12)
    brute = flexrel_bruteforce(d["q"][:, :, :], d["k"], d["v"], d["rel"], d["lens"])
    assert np.abs(brute[:, :, sl] - d["expected"][:, :, sl]).max() < 1e-6


def test_bruteforce_matches_reference_tiny():
    rng = np.random.default_rng(5)
    for length, lens in ((9, [9]), (7, [3]), (1, [1])):
        q, k, v = (rng.standard_normal((1, 1, length, 64)) for _ in range(3))
        rel = rng.standard_normal((73, 64))
        a = flexrel_bruteforce(q, k, v, rel, lens)
        b = flexrel_reference(q, k, v, rel, lens)
        assert np.abs(a - b).max() < 1e-12


@pytest.mark.parametrize("mutation", [
    dict(_distance_sign=-1),
    dict(scale_before_bias=True),
    dict(_left=63, _right=9),
    dict(_mask=False),
])
def test_planted_mistakes_are_caught(golden_cases, mutation):
    d = golden_cases["hf_b2_h2_l200"]
    # _left=63/_right=9 keeps the 73-row table but shifts the clamp window
    wrong = flexrel_reference(d["q"], d["k"], d["v"], d["rel"], d["lens"], **mutation)
    assert _valid_rows_err(d["expected"], wrong, d["lens"]) > 1e-3, mutation


def _sdpa(q, k, v):
    t = [torch.from_numpy(np.asarray(x, dtype=np.float64)) for x in (q, k, v)]
    return torch.nn.functional.scaled_dot_product_attention(*t).numpy()


def test_zero_table_is_plain_sdpa():
    q, k, v, _ = seeded_inputs(1, 2, 150, seed=3, dtype=np.float64)
    rel = np.zeros((73, 64))
    ref = flexrel_reference(q.numpy(), k.numpy(), v.numpy(), rel)
    assert np.abs(ref - _sdpa(q, k, v)).max() < 1e-12


def test_equal_table_rows_are_a_row_constant():
    # every row of E equal => bias q_i.e is constant over j => softmax shift
    q, k, v, _ = seeded_inputs(1, 2, 150, seed=4, dtype=np.float64)
    rel = np.tile(np.random.default_rng(4).standard_normal((1, 64)), (73, 1))
    ref = flexrel_reference(q.numpy(), k.numpy(), v.numpy(), rel)
    assert np.abs(ref - _sdpa(q, k, v)).max() < 1e-12
    tiled = flexrel_tiled(q.numpy(), k.numpy(), v.numpy(), rel, rows_per_block=32, keys_per_tile=64)
    assert np.abs(tiled - ref).max() < 1e-12


def test_single_key_returns_v0():
    q, k, v, rel = seeded_inputs(1, 3, 70, seed=5, dtype=np.float64)
    ref = flexrel_reference(q.numpy(), k.numpy(), v.numpy(), rel.numpy(), lens=[1])
    assert np.abs(ref - v.numpy()[:, :, :1]).max() < 1e-15


def test_zero_length_rows_are_zero():
    q, k, v, rel = seeded_inputs(2, 1, 40, seed=6, dtype=np.float64)
    ref = flexrel_reference(q.numpy(), k.numpy(), v.numpy(), rel.numpy(), lens=[0, 40])
    assert not ref[0].any()
    assert ref[1].any()


def test_heads_are_independent():
    q, k, v, rel = (t.numpy() for t in seeded_inputs(1, 3, 120, seed=7, dtype=np.float64))
    full = flexrel_reference(q, k, v, rel)
    for h in range(3):
        one = flexrel_reference(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], rel)
        assert np.abs(one[:, 0] - full[:, h]).max() < 1e-13


def test_valid_rows_ignore_keys_past_length():
    q, k, v, rel = (t.numpy() for t in seeded_inputs(1, 2, 160, seed=8, dtype=np.float64))
    lens = [131]
    a = flexrel_reference(q, k, v, rel, lens)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 131:] = 1e4
    v2[:, :, 131:] = -1e4
    b = flexrel_reference(q, k2, v2, rel, lens)
    assert np.array_equal(a, b)
    # an exact-length run agrees on the valid rows
    c = flexrel_reference(q[:, :, :131], k[:, :, :131], v[:, :, :131], rel)
    assert np.abs(a[:, :, :131] - c).max() < 1e-13


@pytest.mark.parametrize("rows,keys,splits", [(32, 64, 1), (32, 64, 2), (32, 64, 4), (64, 64, 3),
                                              (16, 32, 2), (128, 64, 1)])
@pytest.mark.parametrize("length,lens", [(1, [1]), (33, [33]), (65, [64]), (200, [200]),
                                         (300, [173]), (257, [1])])
def test_tiled_schedule_equals_closed_form(rows, keys, splits, length, lens):
    q, k, v, rel = (t.numpy() for t in seeded_inputs(1, 2, length, seed=length, dtype=np.float64,
                                                      rel_std=0.5))
    ref = flexrel_reference(q, k, v, rel, lens)
    got = flexrel_tiled(q, k, v, rel, lens, rows_per_block=rows, keys_per_tile=keys, key_splits=splits)
    assert np.abs(got - ref).max() < 1e-12


def test_tiled_fp16_probabilities_meet_the_bar():
    # rounding p to fp16 before PV (as the kernel does) stays far inside the
    # 60 dB / 2e-3 tolerance of the GPU parity tests
    q, k, v, rel = (t.numpy() for t in seeded_inputs(1, 2, 400, seed=9, dtype=np.float64))
    ref = flexrel_reference(q, k, v, rel)
    got = flexrel_tiled(q, k, v, rel, key_splits=2, p_dtype=np.float16)
    err = errors(ref, got)
    assert err["snr_db"] > 60 and err["max_abs"] < 2e-3, err


def test_torch_chunked_matches_reference():
    q, k, v, rel = seeded_inputs(2, 2, 700, seed=10, dtype=np.float32)
    lens = [700, 613]
    got = torch_core_chunked(q, k, v, rel, lens, chunk=256).numpy()
    ref = flexrel_reference(q.numpy(), k.numpy(), v.numpy(), rel.numpy(), lens)
    assert _valid_rows_err(ref, got, lens) < 2e-5


def test_flop_count():
    # BASELINE: 95.09 GFLOP per L=4800, H=16 layer
    assert math.isclose(attention_flops(16, 4800, 4800) / 1e9, 95.09, rel_tol=1e-3)
    assert math.isclose(attention_flops(16, 750, 750) / 1e9, 2.416, rel_tol=1e-3)


# ---- errors(): the SNR / relative RMSE / max |err| judge of every parity test
# (src/sidon_triton/engines.py:47-55), pinned by closed-form known answers.

def _known_answer_cases():
    """(reference, actual, expected max_abs, relative_rmse, snr_db)."""
    cases = []
    # constant reference c, actual = c (1 + eps): noise = c eps everywhere
    for c, eps in ((2.5, 1e-3), (0.75, 3e-4), (10.0, 0.05)):
        ref = np.full((3, 7, 11), c)
        cases.append((ref, ref * (1.0 + eps), c * eps, eps, -20.0 * math.log10(eps)))
    # reference +-1, actual = reference + delta: signal 1, noise |delta|
    rng = np.random.default_rng(5)
    for delta in (1e-3, 2e-2, -4e-4):
        ref = rng.choice([-1.0, 1.0], size=(64, 64))
        cases.append((ref, ref + delta, abs(delta), abs(delta), -20.0 * math.log10(abs(delta))))
    # uneven error: ref (3, 4), error (0, 1): rms(ref) = sqrt(12.5),
    # rms(err) = sqrt(0.5) -> relative RMSE exactly 0.2, SNR 20 log10(5);
    # mean |err| (0.5), rms(actual) = sqrt(17) and 10 log10 all differ
    cases.append((np.array([3.0, 4.0]), np.array([3.0, 5.0]), 1.0, 0.2, 20.0 * math.log10(5.0)))
    return cases


@pytest.mark.parametrize("case", range(7))
def test_errors_known_answers(case):
    ref, act, max_abs, rel, snr = _known_answer_cases()[case]
    got = errors(ref, act)
    assert math.isclose(got["max_abs"], max_abs, rel_tol=1e-9)
    assert math.isclose(got["relative_rmse"], rel, rel_tol=1e-9)
    assert math.isclose(got["snr_db"], snr, rel_tol=1e-9)
    # symmetric inputs in torch / fp32 arrays give the same numbers
    got32 = errors(torch.from_numpy(ref.astype(np.float32)), act.astype(np.float32))
    assert math.isclose(got32["snr_db"], snr, abs_tol=1e-3)


def test_errors_sixty_db_at_one_part_in_a_thousand():
    # relative error 1e-3 is exactly 60 dB
    ref = np.full(1000, 1.7)
    assert math.isclose(errors(ref, ref * 1.001)["snr_db"], 60.0, rel_tol=1e-9)
    assert errors(ref, ref * 1.0011)["snr_db"] < 60.0 < errors(ref, ref * 1.0009)["snr_db"]


def test_errors_identical_inputs_hit_the_noise_floor():
    ref = np.array([[1.0, -1.0], [1.0, -1.0]])
    got = errors(ref, ref.copy())
    assert got["max_abs"] == 0.0 and got["relative_rmse"] == 0.0
    # noise clamped at 1e-12: 20 log10(1 / 1e-12) = 240 dB
    assert math.isclose(got["snr_db"], 240.0, rel_tol=1e-12)
    assert errors(np.zeros(4), np.zeros(4))["snr_db"] < -300.0  # zero signal, no math error


def test_errors_max_abs_is_the_largest_elementwise_difference():
    ref = np.zeros((5, 5))
    act = ref.copy()
    act[3, 1] = -0.25
    act[0, 4] = 0.125
    got = errors(ref, act)
    assert got["max_abs"] == 0.25
    # signal 0: relative RMSE = noise / 1e-12
    assert math.isclose(got["relative_rmse"], math.sqrt((0.25**2 + 0.125**2) / 25) / 1e-12, rel_tol=1e-12)


@pytest.mark.parametrize("mutation", [dict(_noise="mean_abs"), dict(_db_factor=10.0),
                                      dict(_signal_from="actual")])
def test_errors_planted_mistakes_are_caught(mutation):
    # every mutation fails at least one known answer
    failed = 0
    for ref, act, max_abs, rel, snr in _known_answer_cases():
        got = errors(ref, act, **mutation)
        ok = (math.isclose(got["relative_rmse"], rel, rel_tol=1e-6)
              and math.isclose(got["snr_db"], snr, rel_tol=1e-6))
        failed += not ok
    assert failed > 0, mutation
