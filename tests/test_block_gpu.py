"""GPU tests of the encoder pieces around the attention: the residual
LayerNorm kernel (C ABI sidon_res_norm) and the conformer attention sub-block,
against torch fp32 / the float64 sub-block oracle."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from conftest import ROOT

sys.path.insert(0, str(ROOT / "tests" / "golden"))

from make_block_golden import block_input, block_layers  # noqa: E402
from oracle.encoder_block_oracle import attention_blocks_reference  # noqa: E402
from oracle.flexrel_oracle import errors  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ln_ref(x, norm):
    w, b, eps = norm
    return torch.nn.functional.layer_norm(x, (x.shape[-1],), w, b, eps)


@pytest.mark.parametrize("rows,cols", [(257, 1024), (33, 160), (5, 2048), (64, 4)])
@pytest.mark.parametrize("xn_fp16", [True, False])
def test_res_norm_matches_torch(sidon, rows, cols, xn_fp16):
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x0 = torch.randn(rows, cols, generator=g) * 3 + 0.5
    y = torch.randn(rows, cols, generator=g)
    bias = torch.randn(cols, generator=g) * 0.1
    n1 = (1 + 0.1 * torch.randn(cols, generator=g), 0.1 * torch.randn(cols, generator=g), 1e-5)
    n2 = (1 + 0.1 * torch.randn(cols, generator=g), 0.1 * torch.randn(cols, generator=g), 1e-6)
    u = _ln_ref(x0 + bias + y, n1)
    want_xn = _ln_ref(u, n2)
    x = x0.to(DEV)
    d = lambda t: t.to(DEV)  # noqa: E731
    xn = sidon.encoder_block.res_norm(x, y=d(y), norm1=(d(n1[0]), d(n1[1]), n1[2]), write_x=True,
                                      norm2=(d(n2[0]), d(n2[1]), n2[2]), bias=d(bias),
                                      xn_dtype=torch.float16 if xn_fp16 else torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_allclose(x.cpu().numpy(), u.numpy(), rtol=0, atol=2e-5)
    tol = 4e-3 if xn_fp16 else 2e-5
    np.testing.assert_allclose(xn.float().cpu().numpy(), want_xn.numpy(), rtol=0, atol=tol)


def test_res_norm_bias_only_leaves_x(sidon):
    g = torch.Generator().manual_seed(3)
    x0 = torch.randn(100, 1024, generator=g)
    bias = torch.randn(1024, generator=g)
    n2 = (torch.ones(1024), torch.zeros(1024), 1e-5)
    x = x0.to(DEV)
    xn = sidon.encoder_block.res_norm(x, norm2=tuple(t.to(DEV) if torch.is_tensor(t) else t for t in n2),
                                      bias=bias.to(DEV), write_x=False)
    torch.cuda.synchronize()
    assert torch.equal(x.cpu(), x0)  # write_x=False: the stream keeps no bias
    want = _ln_ref(x0 + bias, n2)
    np.testing.assert_allclose(xn.float().cpu().numpy(), want.numpy(), rtol=0, atol=4e-3)


def packed(layers, device):
    """fp16 / fp32 packed weights (triton_encoder.py:417-443) of oracle layers;
    also returns the oracle layers with the same fp16-rounded values."""
    cum = None
    out, ref = [], []
    for p in layers:
        h = {k: p[k].half() for k in ("qkv_w", "qkv_b", "rel", "out_w")}
        ob = p["out_b"].float()
        cum = ob.double() if cum is None else cum + ob.double()
        w, b, eps = p["attn_ln"]
        out.append({"attn_ln": (w.float().to(device), b.float().to(device), eps),
                    **{k: v.to(device) for k, v in h.items()},
                    "cum_bias": cum.float().to(device)})
        ref.append({"attn_ln": (w.float().double(), b.float().double(), eps),
                    **{k: v.double() for k, v in h.items()}, "out_b": ob.double()})
    return out, ref


@pytest.mark.parametrize("length,n_layers", [(300, 2), (1037, 1)])
def test_attention_blocks_match_oracle(sidon, length, n_layers):
    heads = 16
    layers, ref_layers = packed(block_layers(heads, n_layers, 40 + length), DEV)
    x0 = block_input(1, length, heads, 40 + length).float()
    want = attention_blocks_reference(x0.double(), ref_layers, heads)
    x = x0.reshape(length, -1).contiguous().to(DEV)
    lens = torch.full((1,), length, dtype=torch.int32, device=DEV)
    sidon.encoder_block.attention_blocks(x, layers, 1, heads, lens)
    torch.cuda.synchronize()
    got = x.cpu().double().reshape(1, length, -1)
    err = errors((want - x0.double()).numpy(), (got - x0.double()).numpy())
    print(f"blocks L={length} layers={n_layers}: update snr={err['snr_db']:.1f} dB max_abs={err['max_abs']:.2e}")
    # fp16 operands of the GEMMs and the attention: the update carries ~1e-3
    # relative error (the north star's 60 dB bar is for the attention alone)
    assert err["snr_db"] >= 50.0, err
    total = errors(want.numpy(), got.numpy())
    assert total["max_abs"] <= 2e-3 * float(np.abs(want.numpy()).max()), total


def test_attention_blocks_graph_replay_is_bit_exact(sidon):
    heads, length = 16, 260
    layers, _ = packed(block_layers(heads, 2, 9), DEV)
    x0 = block_input(1, length, heads, 9).float().reshape(length, -1).to(DEV)
    lens = torch.full((1,), 251, dtype=torch.int32, device=DEV)
    bufs = {"xn": torch.empty(length, 64 * heads, dtype=torch.float16, device=DEV),
            "qkv": torch.empty(length, 3 * 64 * heads, dtype=torch.float16, device=DEV),
            "ctx": torch.empty(length, 64 * heads, dtype=torch.float16, device=DEV)}
    eager = x0.clone()
    sidon.encoder_block.attention_blocks(eager, layers, 1, heads, lens, bufs)
    x = torch.empty_like(x0)
    graphs = sidon.graphs.BucketGraphs()

    def enqueue():
        x.copy_(x0)
        sidon.encoder_block.attention_blocks(x, layers, 1, heads, lens, bufs)
    graph = graphs.capture(("blocks", length), enqueue)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(x, eager)
        x.zero_()
        torch.cuda.synchronize()


def test_c5_chunk_matches_fp32_torch(sidon):
    """c5 at full size (bench.py's inputs): 8 sub-blocks at L=4800 against
    the fp32 torch sub-block (oracle) on the GPU."""
    import bench

    x0, raw = bench.c5_inputs(torch)
    cum = sidon.encoder_block.running_biases([p["out_b"] for p in raw])
    d = lambda t: t.to(DEV) if torch.is_tensor(t) else t  # noqa: E731
    layers = [{"attn_ln": tuple(d(t) for t in p["attn_ln"]), "qkv_w": d(p["qkv_w"]), "qkv_b": d(p["qkv_b"]),
               "rel": d(p["rel"]), "out_w": d(p["out_w"]), "cum_bias": d(c)} for p, c in zip(raw, cum)]
    ref_layers = [{"attn_ln": tuple(d(t) for t in p["attn_ln"]),
                   **{k: d(p[k]) for k in ("qkv_w", "qkv_b", "rel", "out_w", "out_b")}} for p in raw]
    length, hid = x0.shape
    x0_d = x0.to(DEV)
    x = x0_d.clone()
    lens = torch.full((1,), length, dtype=torch.int32, device=DEV)
    sidon.encoder_block.attention_blocks(x, layers, 1, 16, lens)
    with torch.no_grad():
        want = attention_blocks_reference(x0_d.view(1, length, hid), ref_layers, 16, dtype=torch.float32)
    torch.cuda.synchronize()
    err = errors((want.view(length, hid) - x0_d).double().cpu().numpy(), (x - x0_d).double().cpu().numpy())
    print(f"c5 chunk (8 sub-blocks, L={length}): update snr={err['snr_db']:.1f} dB max_abs={err['max_abs']:.2e}")
    assert err["snr_db"] >= 60.0, err
