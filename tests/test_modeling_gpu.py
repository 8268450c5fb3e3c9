"""The module drop-in inside a transformers w2v-BERT encoder (needs a GPU):
the swapped model against the original on the same weights, unmasked and with
a padded batch's attention mask (valid rows compared)."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_encoder_golden import encoder_weights, hf_config, load_hf  # noqa: E402
from oracle.flexrel_oracle import errors  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _model(seed):
    from transformers import Wav2Vec2BertModel

    weights = encoder_weights(2, 2, seed=seed)
    model = Wav2Vec2BertModel(hf_config(2, 2, 256)).double().eval()
    load_hf(weights, model.feature_projection, model.encoder)
    return model


@pytest.mark.parametrize("lens", [None, (300, 221)])
def test_swapped_encoder_matches_transformers(sidon, lens):
    ref = _model(11)
    hip = _model(11).float().to(DEV)
    assert sidon.modeling.replace_attention_with_hip(hip) == 2
    batch, length = 2, 300
    gen = torch.Generator().manual_seed(12)
    feats = torch.randn(batch, length, 160, generator=gen, dtype=torch.float64)
    mask = None
    if lens is not None:
        mask = (torch.arange(length)[None, :] < torch.tensor(lens)[:, None]).long()
    with torch.no_grad():
        want = ref(feats, attention_mask=mask).last_hidden_state.numpy()
        got = hip(feats.float().to(DEV), attention_mask=None if mask is None else mask.to(DEV))
        got = got.last_hidden_state.double().cpu().numpy()
    assert np.isfinite(got).all()
    for b in range(batch):
        n = length if lens is None else lens[b]
        err = errors(want[b, :n], got[b, :n])
        print(lens, b, err)
        assert err["snr_db"] > 80 and err["max_abs"] < 2e-3, (b, err)  # measured 89.8-90.0 dB, 1.7e-4
