"""Host logic of the encoder (no GPU): weight extraction from a transformers
model, packing, the safetensors round trip, and the bucket rule."""

from __future__ import annotations

import sys

import pytest
import torch

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_encoder_golden import encoder_weights, hf_config, load_hf  # noqa: E402


@pytest.fixture(scope="module")
def pkg():
    from __graft_entry__ import load_package

    return load_package()


def _eq(a, b):
    return torch.equal(torch.as_tensor(a), torch.as_tensor(b))


def test_model_weights_read_a_transformers_model(pkg):
    from transformers import Wav2Vec2BertModel

    weights = encoder_weights(2, 2, seed=3)
    model = Wav2Vec2BertModel(hf_config(2, 2, 256)).double().eval()
    load_hf(weights, model.feature_projection, model.encoder)
    got = pkg.encoder.model_weights(model)
    assert got["heads"] == 2
    for key in ("fp_w", "fp_b"):
        assert _eq(got[key], weights[key])
    for gl, wl in zip(got["layers"], weights["layers"]):
        assert set(gl) == set(wl)
        for key, val in wl.items():
            if isinstance(val, tuple):
                assert _eq(gl[key][0], val[0]) and _eq(gl[key][1], val[1]) and gl[key][2] == val[2]
            else:
                assert _eq(gl[key], val), key


def test_pack_weights_layout(pkg):
    weights = encoder_weights(2, 2, seed=4)
    packed = pkg.encoder.pack_weights(weights)
    assert packed["heads"] == 2
    for p, w in zip(packed["layers"], weights["layers"]):
        hid = w["out_w"].shape[0]
        assert p["qkv_w"].dtype == torch.float16 and p["qkv_w"].shape == (3 * hid, hid)
        assert _eq(p["qkv_w"][hid:2 * hid], w["k_w"].half())
        assert _eq(p["qkv_b"][2 * hid:], w["v_b"].half())
        assert _eq(p["ffn1_w2"], (w["ffn1_w2"] * 0.5).half())
        assert _eq(p["ffn2_w2"], (w["ffn2_w2"] * 0.5).half())
        assert p["dwt"].dtype == torch.float32 and _eq(p["dwt"], w["dw_w"].t().float())
        b1, b2, b4 = p["cum_bias"]
        assert _eq(b1, (w["ffn1_b2"] * 0.5).float())
        assert _eq(b2, (w["ffn1_b2"] * 0.5 + w["out_b"]).float())
        assert _eq(b4, (w["ffn1_b2"] * 0.5 + w["out_b"] + w["ffn2_b2"] * 0.5).float())
        assert p["final_ln"][0].dtype == torch.float32 and p["final_ln"][2] == w["final_ln"][2]


def test_pack_rejects_a_wrong_width(pkg):
    weights = encoder_weights(2, 1, seed=4)
    weights["heads"] = 4
    with pytest.raises(ValueError):
        pkg.encoder.pack_weights(weights)


def test_save_and_read_round_trip(pkg, tmp_path):
    packed = pkg.encoder.pack_weights(encoder_weights(2, 2, seed=5))
    path = tmp_path / "enc.safetensors"
    pkg.encoder.save_encoder(packed, max_batch=2, max_seconds=30.5, path=path)
    got, max_batch, max_seconds = pkg.encoder.read_encoder(path)
    assert (max_batch, max_seconds) == (2, 30.5)
    assert got["heads"] == packed["heads"] and len(got["layers"]) == len(packed["layers"])
    assert _eq(got["fp_w"], packed["fp_w"]) and got["fp_ln"][2] == packed["fp_ln"][2]
    for g, p in zip(got["layers"], packed["layers"]):
        assert set(g) == set(p)
        for key, val in p.items():
            if key == "cum_bias":
                assert all(_eq(a, b) for a, b in zip(g[key], val))
            elif isinstance(val, tuple):
                assert _eq(g[key][0], val[0]) and _eq(g[key][1], val[1]) and g[key][2] == val[2]
            else:
                assert _eq(g[key], val) and g[key].dtype == val.dtype, key


def test_read_rejects_other_files(pkg, tmp_path):
    from safetensors.torch import save_file

    path = tmp_path / "other.safetensors"
    save_file({"a": torch.zeros(2)}, str(path))
    with pytest.raises(ValueError):
        pkg.encoder.read_encoder(path)


@pytest.mark.parametrize("frames,bucket", [(2, 50), (50, 50), (51, 100), (1463, 1500), (1600, 1600), (1601, 1800),
                                           (4750, 4800), (4800, 4800)])
def test_bucket_rule(pkg, frames, bucket):
    # 1 s (50-frame) buckets up to 32 s, 4 s buckets above, capped at the
    # maximum (src/sidon_triton/runtime.py:366-372).
    assert pkg.runtime.bucket_frames(frames, 4800) == bucket


def test_bucket_cap(pkg):
    assert pkg.runtime.bucket_frames(4700, 4750) == 4750
    with pytest.raises(ValueError):
        pkg.runtime.bucket_frames(0, 4800)


def test_reads_the_reference_packed_file(pkg, tmp_path):
    # The reference's save_encoder writes {"packed": ..., "max_batch": ...,
    # "max_seconds": ...} with torch.save (src/sidon_triton/triton_encoder.py:514-518);
    # the packed layout is key for key the one pack_weights writes.
    packed = pkg.encoder.pack_weights(encoder_weights(2, 2, seed=6))
    path = tmp_path / "encoder_triton.pt"
    torch.save({"packed": packed, "max_batch": 1, "max_seconds": 96.0}, str(path))
    got, max_batch, max_seconds = pkg.encoder.read_triton_encoder(path)
    assert (max_batch, max_seconds) == (1, 96.0)
    for g, p in zip(got["layers"], packed["layers"]):
        for key, val in p.items():
            if key == "cum_bias":
                assert all(_eq(a, b) for a, b in zip(g[key], val))
            elif isinstance(val, tuple):
                assert _eq(g[key][0], val[0]) and g[key][2] == val[2]
            else:
                assert _eq(g[key], val), key


def test_reference_file_with_other_layout_is_rejected(pkg, tmp_path):
    packed = pkg.encoder.pack_weights(encoder_weights(2, 1, seed=6))
    del packed["layers"][0]["rel"]
    path = tmp_path / "bad.pt"
    torch.save({"packed": packed, "max_batch": 1, "max_seconds": 96.0}, str(path))
    with pytest.raises(ValueError):
        pkg.encoder.read_triton_encoder(path)


def test_load_encoder_reads_both_formats(pkg, tmp_path):
    packed = pkg.encoder.pack_weights(encoder_weights(2, 2, seed=7))
    ours = tmp_path / "enc.safetensors"
    theirs = tmp_path / "encoder_triton.pt"
    pkg.encoder.save_encoder(packed, max_batch=2, max_seconds=40.0, path=ours)
    torch.save({"packed": packed, "max_batch": 3, "max_seconds": 96.0}, str(theirs))
    a, ba, sa = pkg.encoder.load_encoder(ours, device="cpu")
    b, bb, sb = pkg.encoder.load_encoder(theirs, device="cpu")
    assert (ba, sa, bb, sb) == (2, 40.0, 3, 96.0)
    assert a.heads == b.heads == 2 and a.hidden == b.hidden == 128 and a.inter == b.inter == 256
    assert _eq(a.layers[1]["qkv_w"], b.layers[1]["qkv_w"])
