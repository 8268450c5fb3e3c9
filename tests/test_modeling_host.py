"""The module drop-in's host side (no GPU): weights load strictly from
transformers' Wav2Vec2BertSelfAttention, the swap helper, and the mask to
valid-length conversion."""

from __future__ import annotations

import sys

import pytest
import torch

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_encoder_golden import hf_config  # noqa: E402


@pytest.fixture(scope="module")
def pkg():
    from __graft_entry__ import load_package

    return load_package()


def test_state_dict_loads_strictly_from_transformers(pkg):
    from transformers.models.wav2vec2_bert.modeling_wav2vec2_bert import Wav2Vec2BertSelfAttention

    src = Wav2Vec2BertSelfAttention(hf_config(2, 1, 256))
    mod = pkg.modeling.HipRelSelfAttention(128, 2)
    mod.load_state_dict(src.state_dict(), strict=True)
    assert torch.equal(mod.distance_embedding.weight, src.distance_embedding.weight)


def test_replace_swaps_every_layer_with_the_same_weights(pkg):
    from transformers import Wav2Vec2BertModel

    model = Wav2Vec2BertModel(hf_config(2, 3, 256)).eval()
    before = [layer.self_attn.linear_k.weight.clone() for layer in model.encoder.layers]
    assert pkg.modeling.replace_attention_with_hip(model) == 3
    for layer, w in zip(model.encoder.layers, before):
        assert isinstance(layer.self_attn, pkg.modeling.HipRelSelfAttention)
        assert torch.equal(layer.self_attn.linear_k.weight, w)


def test_rejects_other_widths_and_windows(pkg):
    with pytest.raises(ValueError):
        pkg.modeling.HipRelSelfAttention(100, 2)
    with pytest.raises(ValueError):
        pkg.modeling.HipRelSelfAttention(128, 2, 32, 8)


def test_key_padding_masks_become_lengths(pkg):
    lens_of = pkg.modeling._lens_from_mask
    keep = torch.tensor([[1, 1, 1, 0, 0], [1, 1, 1, 1, 1]])
    assert lens_of(keep, 2, 5).tolist() == [3, 5]
    # transformers' extended additive mask: 0 kept, finfo.min padded, same row for every query
    additive = (1.0 - keep[:, None, None, :].float()) * torch.finfo(torch.float32).min
    assert lens_of(additive.expand(2, 1, 5, 5), 2, 5).tolist() == [3, 5]
    with pytest.raises(ValueError):  # not a prefix
        lens_of(torch.tensor([[1, 0, 1, 0, 0]]), 1, 5)
    query_dependent = torch.zeros(1, 1, 5, 5)
    query_dependent[0, 0, 2, 4] = -1e9
    with pytest.raises(ValueError):
        lens_of(query_dependent, 1, 5)
