"""Pin the fbank oracle (oracle/frontend_oracle.py) on the CPU: transformers
golden vectors (SeamlessM4TFeatureExtractor, mel_filter_bank), planted
mistakes and closed forms; and the package's frame transform and mel bank
(host-side constants of the HIP front end) against it."""

from __future__ import annotations

import sys

import numpy as np
import pytest

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_fbank_golden import CASES, fbank_chunk  # noqa: E402
import oracle.frontend_oracle as fo  # noqa: E402

GOLDEN = ROOT / "tests" / "golden"
TOL = 1e-4  # the extractor computes and returns float32; measured max difference 1.8e-5


@pytest.mark.parametrize("name", sorted(CASES))
def test_matches_transformers_extractor(name):
    samples, seed = CASES[name]
    expected = np.load(GOLDEN / f"{name}.npz")["expected"]
    got = fo.fbank_exact(fbank_chunk(samples, seed))
    assert got.shape == expected.shape
    assert np.abs(got - expected).max() < TOL


def test_mel_bank_matches_transformers():
    expected = np.load(GOLDEN / "fbank_mel_bank.npz")["mel"]
    np.testing.assert_allclose(fo.kaldi_mel_banks(), expected, rtol=0, atol=1e-12)


def _hann(n=fo.FRAME_SIZE):
    i = np.arange(n)
    return 0.5 - 0.5 * np.cos(2 * np.pi * i / (n - 1))


@pytest.mark.parametrize("mistake", [{"preemph": 0.0}, {"window": "hann"}, {"remove_dc": False}, {"ddof": 0}])
def test_planted_mistakes_break_the_golden_match(mistake):
    samples, seed = CASES["fbank_n3280"]
    expected = np.load(GOLDEN / "fbank_n3280.npz")["expected"]
    kw = dict(mistake)
    if kw.get("window") == "hann":
        kw["window"] = _hann()
    got = fo.fbank_exact(fbank_chunk(samples, seed), **kw)
    assert np.abs(got - expected).max() > 1e-3


def test_constant_frame_has_the_floor_spectrum():
    # DC removal makes a constant frame exactly zero: every mel bin is the floor.
    padded = np.full(fo.FRAME_SIZE, 0.3)
    got = fo.frame_features(padded, 1)
    np.testing.assert_allclose(got, np.log(fo.MEL_FLOOR), rtol=0, atol=1e-9)


def test_normalized_bins_have_zero_mean_unit_variance():
    x = fbank_chunk(16000 * 2, 7)
    feats = fo.fbank_exact(x).reshape(-1, fo.NUM_MEL)
    frames = fo.num_frames(x.shape[0])
    valid = feats[:frames]
    np.testing.assert_allclose(valid.mean(axis=0), 0.0, atol=1e-9)
    var = valid.var(axis=0, ddof=1)
    assert np.all(np.abs(var - 1.0) < 1e-3)


def test_bucketed_rows_equal_the_exact_rows():
    x = fbank_chunk(16123, 41)
    chunk = np.zeros((1, 16320))
    chunk[0, :16123] = x
    got = fo.fbank_bucketed(chunk, [16123])
    exact = fo.fbank_exact(x)
    np.testing.assert_array_equal(got[0, :exact.shape[0]], exact)
    assert not got[0, exact.shape[0]:].any()


@pytest.fixture(scope="module")
def pkg():
    from __graft_entry__ import load_package

    return load_package()


def test_package_frame_transform_equals_the_kaldi_chain(pkg):
    # The HIP front end applies DC removal, pre-emphasis, window and the rDFT
    # as one [400, 514] matrix; on any frame it must equal the chain.
    w = pkg.frontend.frame_transform().numpy()
    rng = np.random.default_rng(3)
    frames = rng.standard_normal((5, fo.FRAME_SIZE))
    spec = frames @ w
    fr = frames * fo.KALDI_SCALE
    fr = fr - fr.mean(axis=1, keepdims=True)
    pre = fr.copy()
    pre[:, 1:] = fr[:, 1:] - fo.PREEMPH * fr[:, :-1]
    pre[:, 0] = fr[:, 0] * (1 - fo.PREEMPH)
    want = np.fft.rfft(pre * fo.povey_window(), n=fo.N_FFT, axis=1)
    np.testing.assert_allclose(spec[:, :fo.N_BINS], want.real, rtol=0, atol=1e-6)
    np.testing.assert_allclose(spec[:, fo.N_BINS:], want.imag, rtol=0, atol=1e-6)


def test_package_mel_bank_and_its_sparse_form(pkg):
    dense = pkg.frontend.mel_banks()
    np.testing.assert_allclose(dense, fo.kaldi_mel_banks(), rtol=0, atol=1e-12)
    lo, length, weights = pkg.frontend.sparse_mel(dense)
    rebuilt = np.zeros_like(dense)
    for m in range(dense.shape[1]):
        rebuilt[lo[m]:lo[m] + length[m], m] = weights[m, :length[m]]
    np.testing.assert_allclose(rebuilt, dense.astype(np.float32), rtol=0, atol=0)


@pytest.mark.parametrize("samples,frames,feats", [(16123, 101, 51), (8000, 50, 25), (320, 2, 1), (96 * 16000, 9600, 4800)])
def test_frame_counts(pkg, samples, frames, feats):
    assert pkg.frontend.num_frames(samples) == frames == fo.num_frames(samples)
    assert pkg.frontend.num_features(samples) == feats
