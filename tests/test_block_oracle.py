"""Pin the attention sub-block oracle (oracle/encoder_block_oracle.py) on the CPU:
transformers golden vectors, a closed form, and planted mistakes."""

from __future__ import annotations

import copy
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_block_golden import CASES, block_input, block_layers  # noqa: E402
from oracle.encoder_block_oracle import attention_blocks_reference  # noqa: E402

GOLDEN = ROOT / "tests" / "golden"


@pytest.mark.parametrize("name", sorted(CASES))
def test_matches_transformers_golden(name):
    batch, heads, length, n_layers, seed = CASES[name]
    expected = np.load(GOLDEN / f"{name}.npz")["expected"]
    got = attention_blocks_reference(block_input(batch, length, heads, seed),
                                      block_layers(heads, n_layers, seed), heads)
    np.testing.assert_allclose(got.numpy(), expected, rtol=0, atol=1e-10)


def _planted(layers, what):
    layers = copy.deepcopy(layers)
    for p in layers:
        if what == "no_out_bias":
            p["out_b"] = torch.zeros_like(p["out_b"])
        elif what == "ln_swapped":
            w, b, eps = p["attn_ln"]
            p["attn_ln"] = (b, w, eps)
        elif what == "qk_swapped":
            hid = p["out_w"].shape[0]
            w = p["qkv_w"].clone()
            w[:hid], w[hid:2 * hid] = p["qkv_w"][hid:2 * hid], p["qkv_w"][:hid]
            p["qkv_w"] = w
        elif what == "out_transposed":
            p["out_w"] = p["out_w"].t().contiguous()
    return layers


@pytest.mark.parametrize("what", ["no_out_bias", "ln_swapped", "qk_swapped", "out_transposed"])
def test_planted_mistakes_break_the_golden_match(what):
    name = sorted(CASES)[0]
    batch, heads, length, n_layers, seed = CASES[name]
    expected = np.load(GOLDEN / f"{name}.npz")["expected"]
    got = attention_blocks_reference(block_input(batch, length, heads, seed),
                                      _planted(block_layers(heads, n_layers, seed), what), heads)
    assert np.abs(got.numpy() - expected).max() > 1e-3


def test_zero_query_key_projection_gives_mean_of_values():
    # With W_q = W_k = 0 and zero q/k biases every score of a row is equal
    # (the table term q.E vanishes with q), so the context is the mean of the
    # valid V rows: x_out = x + mean(V) W_out^T + b_out for every row.
    heads, length, lk = 2, 40, 29
    layers = block_layers(heads, 1, 5)
    p = layers[0]
    hid = 64 * heads
    p["qkv_w"][:2 * hid] = 0
    p["qkv_b"][:2 * hid] = 0
    x = block_input(1, length, heads, 5)
    got = attention_blocks_reference(x, layers, heads, lens=[lk])
    w, b, eps = p["attn_ln"]
    u = torch.nn.functional.layer_norm(x, (hid,), w, b, eps)
    v = u @ p["qkv_w"][2 * hid:].t() + p["qkv_b"][2 * hid:]
    ctx = v[:, :lk].mean(dim=1, keepdim=True)
    want = x + ctx @ p["out_w"].t() + p["out_b"]
    np.testing.assert_allclose(got.numpy(), want.expand_as(got).numpy(), rtol=0, atol=1e-12)
