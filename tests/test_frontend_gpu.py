"""The fbank front end on the MI355X (needs a GPU): against the float64 oracle
and the transformers extractor's golden vectors on bucketed batches
(statistics over the true frames, the pad frame, zeros after), at a 96 s
chunk, bit-exact graph replays, and the runtime's waveform path (front end +
encoder in one graph) against eager calls."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_encoder_golden import encoder_weights  # noqa: E402
from make_fbank_golden import CASES, fbank_chunk  # noqa: E402
import oracle.frontend_oracle as fo  # noqa: E402
from oracle.flexrel_oracle import errors  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _bucket(chunks, samples=None):
    n = max(c.shape[0] for c in chunks)
    s = samples or -(-n // 320) * 320
    out = np.zeros((len(chunks), s), np.float32)
    for b, c in enumerate(chunks):
        out[b, :c.shape[0]] = c
    return out


def _check(got, want, valid, label):
    got = got.double().cpu().numpy()
    for b, n in enumerate(valid):
        tf = fo.num_frames(int(n))
        rows = (tf + 1) // 2
        flat_g = got[b].reshape(-1, fo.NUM_MEL)
        flat_w = want[b].reshape(-1, fo.NUM_MEL)
        err = errors(flat_w[:tf], flat_g[:tf])
        print(label, b, err)
        assert err["snr_db"] > 95 and err["max_abs"] < 2e-3, (b, err)  # measured 107-112 dB, 2.2e-4
        if tf % 2:
            assert (flat_g[tf] == 1.0).all()
        assert not got[b, rows:].any()


def test_fbank_matches_oracle_on_a_bucketed_batch(sidon):
    valid = [16123, 8000, 3280]
    chunks = [fbank_chunk(n, 40 + i) for i, n in enumerate(valid)]
    host = _bucket(chunks)
    fb = sidon.frontend.Fbank(DEV)
    got = fb(torch.from_numpy(host).to(DEV), torch.tensor(valid, dtype=torch.int32, device=DEV))
    assert got.shape == (3, host.shape[1] // 320, 160)
    _check(got, fo.fbank_bucketed(host, valid), valid, "oracle")


@pytest.mark.parametrize("name", sorted(CASES))
def test_fbank_matches_extractor_golden(sidon, name):
    samples, seed = CASES[name]
    expected = np.load(ROOT / "tests" / "golden" / f"{name}.npz")["expected"]
    host = _bucket([fbank_chunk(samples, seed)], samples=-(-samples // 320) * 320 + 640)
    fb = sidon.frontend.Fbank(DEV)
    got = fb(torch.from_numpy(host).to(DEV), torch.tensor([samples], dtype=torch.int32, device=DEV))
    want = np.zeros((1,) + tuple(got.shape[1:]))
    want[0, :expected.shape[0]] = expected
    _check(got, want, [samples], name)


def test_fbank_96s_chunk(sidon):
    samples = 96 * 16000
    valid = samples - 12345
    x = fbank_chunk(valid, 77)
    host = _bucket([x], samples=samples)
    fb = sidon.frontend.Fbank(DEV)
    got = fb(torch.from_numpy(host).to(DEV), torch.tensor([valid], dtype=torch.int32, device=DEV))
    assert got.shape == (1, 4800, 160)
    _check(got, fo.fbank_bucketed(host, [valid]), [valid], "96s")


def test_fbank_graph_replays_match_eager(sidon):
    fb = sidon.frontend.Fbank(DEV)
    ws = fb.workspace(2, 48000)
    gen = torch.Generator().manual_seed(1)
    chunk = torch.zeros(2, 32000, device=DEV)
    valid = torch.tensor([31000, 20111], dtype=torch.int32, device=DEV)
    out = torch.empty(2, 100, 160, device=DEV)
    src = torch.randn(2, 32000, generator=gen) * 0.1
    chunk.copy_(src)
    chunk[1, 20111:] = 0
    eager = fb(chunk, valid, workspace=ws).clone()
    graphs = sidon.graphs.BucketGraphs()
    for rep in range(3):
        out.zero_()
        graphs.run("fbank", lambda: fb(chunk, valid, out=out, workspace=ws))
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        _ = (chunk * 2).sum().item()


def test_runtime_wave_path_matches_eager(sidon):
    enc = sidon.encoder.HipEncoder(sidon.encoder.pack_weights(encoder_weights(2, 2, seed=9)), DEV)
    fb = sidon.frontend.Fbank(DEV)
    rt = sidon.runtime.EncoderRuntime(enc, max_batch=2, max_seconds=10, max_graphs=4, frontend=fb)
    for rep, (valid) in enumerate([[30123], [52000, 41017], [30123 - 999]]):
        n = max(valid)
        wave = np.zeros((len(valid), n), np.float32)
        for b, v in enumerate(valid):
            wave[b, :v] = fbank_chunk(v, 60 + rep + b)
        got = rt.run_wave(torch.from_numpy(wave), valid).clone()
        bucket = sidon.runtime.bucket_samples(n, rt.max_samples)
        padded = torch.zeros(len(valid), bucket, device=DEV)
        padded[:, :n] = torch.from_numpy(wave).to(DEV)
        vt = torch.tensor(valid, dtype=torch.int32, device=DEV)
        feats = fb(padded, vt)
        lens = torch.tensor([sidon.frontend.num_features(v) for v in valid], dtype=torch.int32, device=DEV)
        want = enc(feats, lens)
        torch.cuda.synchronize()
        for b, v in enumerate(valid):
            rows = sidon.frontend.num_features(v)
            assert torch.equal(got[b, :rows], want[b, :rows]), (rep, b)
