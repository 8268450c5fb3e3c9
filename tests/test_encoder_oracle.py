"""Pin the encoder oracle (oracle/encoder_oracle.py) on the CPU: transformers
golden vectors (one exact-length item, one padded batch run with an attention
mask), planted mistakes, and a closed form."""

from __future__ import annotations

import copy
import sys

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_encoder_golden import CASES, encoder_features, encoder_weights  # noqa: E402
import oracle.encoder_oracle as eo  # noqa: E402

GOLDEN = ROOT / "tests" / "golden"


def _case(name):
    batch, heads, length, n_layers, lens, seed = CASES[name]
    expected = np.load(GOLDEN / f"{name}.npz")["expected"]
    lens = [length] * batch if lens is None else list(lens)
    return encoder_features(batch, length, seed), encoder_weights(heads, n_layers, seed), lens, expected


def _valid_max_err(got, expected, lens):
    return max(np.abs(got[b, :n] - expected[b, :n]).max() for b, n in enumerate(lens))


@pytest.mark.parametrize("name", sorted(CASES))
def test_matches_transformers_golden(name):
    feats, weights, lens, expected = _case(name)
    got = eo.encoder_reference(feats, weights, lens).numpy()
    assert _valid_max_err(got, expected, lens) < 1e-10
    for b, n in enumerate(lens):
        assert not got[b, n:].any()


def _planted(weights, what):
    weights = copy.deepcopy(weights)
    for p in weights["layers"]:
        hid = p["out_w"].shape[0]
        if what == "glu_halves_swapped":
            p["pw1_w"] = torch.cat([p["pw1_w"][hid:], p["pw1_w"][:hid]])
        elif what == "taps_reversed":
            p["dw_w"] = p["dw_w"].flip(1)
        elif what == "ffn_half_dropped":
            p["ffn1_w2"] = 2 * p["ffn1_w2"]
            p["ffn1_b2"] = 2 * p["ffn1_b2"]
        elif what == "final_ln_swapped":
            w, b, eps = p["final_ln"]
            p["final_ln"] = (b, w, eps)
        elif what == "qk_swapped":
            p["q_w"], p["k_w"] = p["k_w"], p["q_w"]
            p["q_b"], p["k_b"] = p["k_b"], p["q_b"]
    return weights


@pytest.mark.parametrize("what", ["glu_halves_swapped", "taps_reversed", "ffn_half_dropped", "final_ln_swapped",
                                  "qk_swapped"])
def test_planted_weight_mistakes_break_the_golden_match(what):
    feats, weights, lens, expected = _case("enc_b1_h2_l96_x2")
    got = eo.encoder_reference(feats, _planted(weights, what), lens).numpy()
    assert _valid_max_err(got, expected, lens) > 1e-3


def _same_padding_conv(x, p, dtype):
    """A planted mistake: the depthwise conv centred ('same' padding) instead
    of causal."""
    hid = x.shape[-1]
    u = eo._ln(x, p["conv_ln"], dtype)
    h = u @ p["pw1_w"].to(dtype).t()
    g = h[:, :hid] * torch.sigmoid(h[:, hid:])
    taps = p["dw_w"].to(dtype)
    k = taps.shape[1]
    gp = F.pad(g.t()[None], ((k - 1) // 2, (k - 1) // 2))
    y = F.conv1d(gp, taps[:, None, :], groups=hid)[0].t()
    y = eo._silu(eo._ln(y, p["dw_ln"], dtype))
    return y @ p["pw2_w"].to(dtype).t()


def test_planted_non_causal_conv_breaks_the_golden_match(monkeypatch):
    feats, weights, lens, expected = _case("enc_b1_h2_l96_x2")
    monkeypatch.setattr(eo, "conv_module_reference", _same_padding_conv)
    got = eo.encoder_reference(feats, weights, lens).numpy()
    assert _valid_max_err(got, expected, lens) > 1e-3


def test_padded_rows_do_not_reach_valid_rows():
    # The masked golden pins the exact-length semantics for the second item;
    # the oracle's exact-length run of it alone agrees with its batched run.
    feats, weights, lens, _ = _case("enc_b2_h2_l80_x2_masked")
    both = eo.encoder_reference(feats, weights, lens).numpy()
    alone = eo.encoder_reference(feats[1:, :lens[1]], weights).numpy()
    np.testing.assert_array_equal(both[1, :lens[1]], alone[0])


def test_zero_residual_branches_leave_the_final_norms():
    # With every residual branch's output projection zero, each layer maps
    # x -> LayerNorm_final(x): the encoder is the feature projection followed
    # by the final norms alone.
    feats, weights, lens, _ = _case("enc_b1_h2_l96_x2")
    for p in weights["layers"]:
        for name in ("ffn1_w2", "ffn1_b2", "out_w", "out_b", "pw2_w", "ffn2_w2", "ffn2_b2"):
            p[name] = torch.zeros_like(p[name])
    got = eo.encoder_reference(feats, weights, lens)
    w, b, eps = weights["fp_ln"]
    x = F.layer_norm(feats, (feats.shape[-1],), w, b, eps) @ weights["fp_w"].t() + weights["fp_b"]
    for p in weights["layers"]:
        w, b, eps = p["final_ln"]
        x = F.layer_norm(x, (x.shape[-1],), w, b, eps)
    np.testing.assert_allclose(got.numpy(), x.numpy(), rtol=0, atol=1e-12)
