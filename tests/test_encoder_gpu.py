"""The conformer ops and the whole encoder on the MI355X (needs a GPU).

Kernel parity: glu / silu / causal_dw_norm against float32 torch of the same
op, rounded to fp16 like the kernels' outputs (within 2 fp16 ulps; the fused
GLU variant bit-identical to the two-step one).  Encoder parity: against the
transformers golden vectors (float64) at a small width, and against the fp32
torch oracle at Sidon's full width, by output SNR and max error; a bucketed
run against an exact-length run; the graph runtime against eager calls, bit
for bit.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_encoder_golden import CASES, encoder_features, encoder_weights  # noqa: E402
from oracle.encoder_oracle import encoder_reference  # noqa: E402
from oracle.flexrel_oracle import errors  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _ulp_close(got, want, ulps=2):
    """|got - want| <= ulps fp16 ulps of want (subnormal floor 2^-24)."""
    want16 = want.half().float()
    ulp = torch.clamp(want16.abs(), min=2.0 ** -14) * 2.0 ** -10
    bad = (got.float() - want16).abs() > ulps * ulp
    assert not bad.any(), (int(bad.sum()), (got.float() - want16).abs().max().item())


@pytest.mark.parametrize("rows,c", [(333, 1024), (17, 60), (4800, 2048)])
def test_glu_matches_torch(sidon, rows, c):
    gen = torch.Generator().manual_seed(rows + c)
    h = (torch.randn(rows, 2 * c, generator=gen) * 3).half().to(DEV)
    got = sidon.conformer.glu(h)
    hf = h.float()
    _ulp_close(got, hf[:, :c] * torch.sigmoid(hf[:, c:]))


@pytest.mark.parametrize("n", [4800 * 4096, 1001])
def test_silu_matches_torch(sidon, n):
    gen = torch.Generator().manual_seed(n % 1000)
    h = (torch.randn(n, generator=gen) * 4).half().to(DEV)
    want = F.silu(h.float())
    sidon.conformer.silu_(h)
    _ulp_close(h, want)


def _dw_reference(g, batch, dwt, ln_w, ln_b, eps):
    rows, c = g.shape
    k = dwt.shape[0]
    x = g.float().view(batch, rows // batch, c).transpose(1, 2)      # [B, C, T]
    y = F.conv1d(F.pad(x, (k - 1, 0)), dwt.t()[:, None, :], groups=c)
    y = F.layer_norm(y.transpose(1, 2), (c,), ln_w, ln_b, eps)
    return F.silu(y).reshape(rows, c)


@pytest.mark.parametrize("batch,t,c,k", [(2, 37, 128, 31), (1, 100, 1024, 31), (3, 16, 2048, 3), (2, 1, 64, 7),
                                         (1, 4800, 1024, 31), (2, 45, 1000, 15)])
def test_causal_dw_norm_matches_fp32_torch(sidon, batch, t, c, k):
    gen = torch.Generator().manual_seed(batch * 1000 + t + c + k)
    h = (torch.randn(batch * t, 2 * c, generator=gen) * 2).half().to(DEV)
    dwt = (torch.randn(k, c, generator=gen) * 0.2).to(DEV)
    ln_w = (1 + 0.1 * torch.randn(c, generator=gen)).to(DEV)
    ln_b = (0.1 * torch.randn(c, generator=gen)).to(DEV)
    g = sidon.conformer.glu(h)
    got = sidon.conformer.causal_dw_norm(g, batch, dwt, ln_w, ln_b, 1e-5)
    want = _dw_reference(g, batch, dwt, ln_w, ln_b, 1e-5)
    err = errors(want.double().cpu().numpy(), got.double().cpu().numpy())
    assert err["snr_db"] > 60 and err["max_abs"] < 8e-3 * want.abs().max().item(), err
    fused = sidon.conformer.glu_causal_dw_norm(h, batch, dwt, ln_w, ln_b, 1e-5)
    assert torch.equal(fused, got)


def test_causal_dw_norm_items_are_independent(sidon):
    batch, t, c = 3, 50, 256
    gen = torch.Generator().manual_seed(11)
    g = torch.randn(batch * t, c, generator=gen).half().to(DEV)
    dwt = (torch.randn(31, c, generator=gen) * 0.2).to(DEV)
    ln_w, ln_b = torch.ones(c, device=DEV), torch.zeros(c, device=DEV)
    a = sidon.conformer.causal_dw_norm(g, batch, dwt, ln_w, ln_b, 1e-5)
    g2 = g.clone()
    g2[:t] = 100.0     # item 0
    g2[2 * t:] = -7.0  # item 2
    b = sidon.conformer.causal_dw_norm(g2, batch, dwt, ln_w, ln_b, 1e-5)
    assert torch.equal(a[t:2 * t], b[t:2 * t])


def test_conformer_ops_reject_bad_arguments(sidon):
    h = torch.zeros(8, 64, dtype=torch.float16, device=DEV)
    dwt = torch.zeros(5, 32, device=DEV)  # K = 5 is not a supported size
    ln = torch.ones(32, device=DEV)
    with pytest.raises(sidon._lib.SidonError):
        sidon.conformer.glu_causal_dw_norm(h, 1, dwt, ln, ln, 1e-5)
    with pytest.raises(ValueError):
        sidon.conformer.causal_dw_norm(h[:, :32].contiguous(), 3, dwt, ln, ln, 1e-5)  # 8 rows, 3 items


def _encoder(sidon, weights):
    return sidon.encoder.HipEncoder(sidon.encoder.pack_weights(weights), DEV)


@pytest.mark.parametrize("name", sorted(CASES))
def test_encoder_matches_transformers_golden(sidon, name):
    batch, heads, length, n_layers, lens, seed = CASES[name]
    expected = np.load(ROOT / "tests" / "golden" / f"{name}.npz")["expected"]
    lens = [length] * batch if lens is None else list(lens)
    enc = _encoder(sidon, encoder_weights(heads, n_layers, seed))
    feats = encoder_features(batch, length, seed).float().to(DEV)
    got = enc(feats, torch.tensor(lens, dtype=torch.int32, device=DEV)).double().cpu().numpy()
    assert np.isfinite(got).all()
    for b, n in enumerate(lens):
        err = errors(expected[b, :n], got[b, :n])
        print(name, b, err)
        assert err["snr_db"] > 65 and err["max_abs"] < 5e-3, (b, err)  # measured 69.4-69.7 dB, 1.5e-3


@pytest.fixture(scope="module")
def full_width(sidon):
    import bench

    weights = bench.encoder_model_weights(torch, seed=7, device=DEV)
    return weights, _encoder(sidon, weights)


@pytest.mark.parametrize("length,valid", [(1500, 1463), (750, 750)])
def test_full_width_encoder_matches_fp32_oracle(sidon, full_width, length, valid):
    weights, enc = full_width
    gen = torch.Generator().manual_seed(length)
    feats = torch.randn(1, length, 160, generator=gen).to(DEV)
    got = enc(feats, torch.tensor([valid], dtype=torch.int32, device=DEV))
    want = encoder_reference(feats, weights, [valid], dtype=torch.float32)
    err = errors(want[0, :valid].double().cpu().numpy(), got[0, :valid].double().cpu().numpy())
    print(length, valid, err)
    assert torch.isfinite(got).all()
    # measured 62.2-62.3 dB, max |err| 5e-3 (the reference reports 66.6-67.1 dB with real weights)
    assert err["snr_db"] > 58 and err["max_abs"] < 0.02 * want.abs().max().item(), err


def test_bucketed_run_matches_exact_length_run(sidon, full_width):
    _, enc = full_width
    gen = torch.Generator().manual_seed(3)
    valid, bucket = 1463, 1500
    feats = torch.randn(1, valid, 160, generator=gen).to(DEV)
    exact = enc(feats)
    padded = torch.zeros(1, bucket, 160, device=DEV)
    padded[:, :valid] = feats
    got = enc(padded, torch.tensor([valid], dtype=torch.int32, device=DEV))
    err = errors(exact[0].double().cpu().numpy(), got[0, :valid].double().cpu().numpy())
    print(err)
    assert err["snr_db"] > 70, err


def test_runtime_graph_replays_match_eager(sidon):
    weights = encoder_weights(2, 2, seed=9)
    enc = _encoder(sidon, weights)
    rt = sidon.runtime.EncoderRuntime(enc, max_batch=2, max_seconds=12, max_graphs=2)
    gen = torch.Generator().manual_seed(4)
    for rep, (batch, n, frames) in enumerate([(1, 123, [123]), (2, 480, [480, 301]), (1, 123, [97]),
                                              (2, 480, [480, 480]), (1, 600, [600])]):
        feats = torch.randn(batch, n, 160, generator=gen)
        got = rt.run(feats, frames).clone()
        length = rt.bucket(n)
        padded = torch.zeros(batch, length, 160, device=DEV)
        padded[:, :n] = feats.to(DEV)
        want = enc(padded, torch.tensor(frames, dtype=torch.int32, device=DEV))[:, :n]
        torch.cuda.synchronize()
        for b, f in enumerate(frames):
            assert torch.equal(got[b, :f], want[b, :f]), (rep, b)
        _ = (padded * 2).sum().item()  # unrelated eager work between replays
    assert len(rt.graphs) == 2  # (1, 150), (2, 500), (1, 600): LRU keeps two
