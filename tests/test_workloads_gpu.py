"""Oracle parity on the exact workloads bench.py measures and on the graphs
the runtime replays (needs an MI355X).

  * c3 as benched: ``bench.c3_workload`` (the residual chain h_{l+1} = h_l +
    ctx_l with q/k/v = qkv_of(h_l), per-layer tables) replayed through its
    captured graph; every layer on all 16 heads against the fp32 torch
    restatement of flexrel_triton.py:297-328 on the same fp16 inputs, plus
    the drift of the whole chain against an fp32-attention chain;
  * c4: every one of the 23 bucket graphs of ``bench.c4_workload`` replayed
    with a clip's valid length; layers 0 and 7 on two heads against the
    float64 closed form over the valid rows;
  * the encoder runtime (counterpart of runtime.py:366-401): ``run`` on a
    bucketed two-item batch and ``run_wave`` over several buckets in
    sequence, the earliest bucket replayed again last, against the float64
    front-end and encoder oracles at exact lengths on the valid rows.

Bars: the north star's SNR >= 60 dB and max |err| <= 2e-3 for the attention;
the encoder bars of tests/test_encoder_gpu.py for the runtime.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from make_encoder_golden import encoder_features, encoder_weights
import oracle.frontend_oracle as fo
from oracle.encoder_oracle import encoder_reference
from oracle.flexrel_oracle import errors, flexrel_reference, torch_core_chunked

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
H, D = 16, 64


def _heads(qkv, length):
    """Fused [L, 3*H*64] rows -> q, k, v [1, H, L, 64] views."""
    v = qkv.view(1, length, 3, H, D)
    return [v[:, :, i].permute(0, 2, 1, 3) for i in range(3)]


def _ctx_heads(out, length):
    """[L, H*64] context rows -> [1, H, L, 64]."""
    return out.view(1, length, H, D).permute(0, 2, 1, 3)


def test_c3_benched_chain_matches_oracle(sidon):
    import bench

    w = bench.c3_workload(torch, sidon, DEV)
    length = bench.L
    for o in w["outs"]:
        o.fill_(float("nan"))  # the replay must write every row
    w["graph"].replay()
    torch.cuda.synchronize()
    worst = 99.0
    for i in range(bench.LAYERS):
        q, k, v = _heads(w["qkv"][i], length)
        with torch.no_grad():
            ref = torch_core_chunked(q, k, v, w["rels_d"][i])
        got = _ctx_heads(w["outs"][i], length).float()
        err = errors(ref.double().cpu().numpy(), got.double().cpu().numpy())
        print(f"c3 layer {i}: snr={err['snr_db']:.2f} dB max_abs={err['max_abs']:.2e}")
        assert err["snr_db"] >= 60.0 and err["max_abs"] <= 2e-3, (i, err)
        worst = min(worst, err["snr_db"])
    # Chain drift: the same chain with fp32 attention (the oracle) in every
    # layer; the HIP chain's last-layer inputs and output against it.
    with torch.no_grad():
        h = w["h0"].to(DEV)
        for i in range(bench.LAYERS):
            qkv_ref = bench.qkv_of(torch, h, w["projs_d"][i])
            ctx = torch_core_chunked(*_heads(qkv_ref, length), w["rels_d"][i])
            h = h + ctx.permute(0, 2, 1, 3).reshape(length, H * D)
    torch.cuda.synchronize()
    drift_in = errors(qkv_ref.double().cpu().numpy(), w["qkv"][-1].double().cpu().numpy())
    drift_out = errors(ctx.double().cpu().numpy(), _ctx_heads(w["outs"][-1], length).double().cpu().numpy())
    print(f"c3 chain drift after {bench.LAYERS} layers: layer-7 q/k/v snr={drift_in['snr_db']:.2f} dB, "
          f"layer-7 output snr={drift_out['snr_db']:.2f} dB (worst per-layer snr {worst:.2f} dB)")
    assert drift_out["snr_db"] >= 40.0, drift_out


def test_c4_bucket_graphs_match_oracle(sidon):
    import bench

    clips, state, keep = bench.c4_workload(torch, sidon, DEV)
    rels = keep["rels"]
    assert len(state) == 23
    first = {}
    for length, lk in clips:
        first.setdefault(length, lk)
    for n, (length, lk) in enumerate(sorted(first.items())):
        qkv, outs, lens, graph = state[length]
        lens.fill_(lk)
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        heads = [n % H, (n + 7) % H]
        for layer in (0, bench.LAYERS - 1):
            q, k, v = (t[:, heads].float().cpu().numpy() for t in _heads(qkv[layer], length))
            ref = flexrel_reference(q, k, v, rels[layer].float().numpy(), [lk])
            got_all = _ctx_heads(outs[layer], length).float().cpu().numpy()
            assert np.isfinite(got_all).all(), (length, layer)
            err = errors(ref[:, :, :lk], got_all[:, heads, :lk])
            print(f"c4 L={length} LK={lk} layer {layer} heads {heads}: snr={err['snr_db']:.2f} dB "
                  f"max_abs={err['max_abs']:.2e}")
            assert err["snr_db"] >= 60.0 and err["max_abs"] <= 2e-3, (length, lk, layer, err)


def _encoder(sidon, weights):
    return sidon.encoder.HipEncoder(sidon.encoder.pack_weights(weights), DEV)


def _check_encoder_rows(got, want, label):
    err = errors(want, got)
    print(label, err)
    assert err["snr_db"] > 65 and err["max_abs"] < 5e-3, (label, err)  # the golden bar of test_encoder_gpu


def test_runtime_run_matches_encoder_oracle(sidon):
    """EncoderRuntime.run on a bucketed two-item batch, then a shorter batch
    in another bucket, then the first bucket again (a replay of its graph),
    each item's valid rows against the float64 oracle at its exact length."""
    weights = encoder_weights(2, 2, seed=9)
    rt = sidon.runtime.EncoderRuntime(_encoder(sidon, weights), max_batch=2, max_seconds=12)
    cases = [(480, [480, 301], 51), (123, [123, 97], 52), (480, [455, 480], 53)]
    for rep, (n, frames, seed) in enumerate(cases):
        feats = encoder_features(2, n, seed).float()
        got = rt.run(feats, frames).double().cpu().numpy()
        for b, f in enumerate(frames):
            want = encoder_reference(feats[b:b + 1, :f].double(), weights)[0].numpy()
            _check_encoder_rows(got[b, :f], want, f"run rep {rep} item {b} ({f} of {n} frames)")
    assert len(rt.graphs) == 2


def test_runtime_wave_matches_frontend_and_encoder_oracles(sidon):
    """EncoderRuntime.run_wave (front end + encoder in one graph per bucket)
    over three buckets in sequence and the earliest bucket again last; each
    item's valid rows against the float64 front-end oracle followed by the
    float64 encoder oracle at the item's exact length."""
    from make_fbank_golden import fbank_chunk

    weights = encoder_weights(2, 2, seed=9)
    fb = sidon.frontend.Fbank(DEV)
    rt = sidon.runtime.EncoderRuntime(_encoder(sidon, weights), max_batch=2, max_seconds=10, frontend=fb)
    sequence = [[30123, 17001], [52000], [8000, 12345], [31999, 30123]]
    buckets = []
    for rep, valid in enumerate(sequence):
        n = max(valid)
        wave = np.zeros((len(valid), n), np.float32)
        for b, v in enumerate(valid):
            wave[b, :v] = fbank_chunk(v, 70 + rep + b)
        got = rt.run_wave(torch.from_numpy(wave), valid).double().cpu().numpy()
        buckets.append(sidon.runtime.bucket_samples(n, rt.max_samples))
        for b, v in enumerate(valid):
            feats = fo.fbank_exact(wave[b, :v])
            rows = sidon.frontend.num_features(v)
            assert feats.shape[0] == rows
            want = encoder_reference(torch.from_numpy(feats)[None], weights)[0].numpy()
            _check_encoder_rows(got[b, :rows], want, f"run_wave rep {rep} item {b} ({v} samples)")
    assert buckets[0] == buckets[-1] and len(set(buckets)) == 3
