"""CPU / torch oracle of the w2v-BERT conformer encoder -- TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module.  Only ``tests/`` and
``bench.py``'s check legs use it, as the checker.

The encoder (8 layers in Sidon) on fp32 features [B, L, F] (F = 160):

    x = LayerNorm_fp(features) W_fp^T + b_fp                      feature projection
    per layer:
      x = x + 0.5 * FFN1(LayerNorm(x))       FFN(u) = silu(u W1^T + b1) W2^T + b2
      x = x + SelfAttention(LayerNorm(x))    relative_key, 73 x 64 table per head
      x = x + ConvModule(x)
      x = x + 0.5 * FFN2(LayerNorm(x))
      x = LayerNorm_final(x)
    ConvModule(x) = silu(LN_dw(causal_dwconv_K(GLU(LN_conv(x) W_pw1^T)))) W_pw2^T

with the depthwise conv causal (K - 1 zero frames on the left) and no conv
biases.  Each batch item runs over its valid frames only (an exact-length
run); its rows past ``lens[b]`` are returned as zeros.

Sources restated here (read, not run):
  * transformers ``Wav2Vec2BertFeatureProjection``, ``Wav2Vec2BertFeedForward``,
    ``Wav2Vec2BertConvolutionModule``, ``Wav2Vec2BertEncoderLayer`` and
    ``Wav2Vec2BertEncoder`` (installed modeling_wav2vec2_bert.py, 5.15.0,
    lines 119-228 and 398-548; the reference pins 4.56.1 at pyproject.toml:16),
    with the configuration of tools/convert_torchscript.py:42-68 (hidden 1024,
    16 heads, FFN 4096, K = 31, relative_key 64 / 8, swish);
  * src/sidon_triton/triton_encoder.py:469-511, the same computation on the
    packed weights of :417-445 (FFN output weights pre-scaled by 0.5, biases of
    the accumulating GEMMs carried as running sums into the next norm) -- here
    every bias is added where the model adds it, so the equivalence of the
    packed form is what the GPU tests check.

Weights use the model's own layout (``model_weights`` of the package returns
the same dict from a transformers module): ``fp_ln`` (w, b, eps), ``fp_w``
[C, F], ``fp_b`` [C], and per layer ``ffn1_ln``, ``ffn1_w1`` [I, C],
``ffn1_b1`` [I], ``ffn1_w2`` [C, I], ``ffn1_b2`` [C], ``attn_ln``, ``q_w``,
``q_b``, ``k_w``, ``k_b``, ``v_w``, ``v_b``, ``rel`` [73, 64], ``out_w``,
``out_b``, ``conv_ln``, ``pw1_w`` [2C, C], ``dw_w`` [C, K], ``dw_ln``,
``pw2_w`` [C, C], ``ffn2_ln``, ``ffn2_w1``, ``ffn2_b1``, ``ffn2_w2``,
``ffn2_b2``, ``final_ln``.

Pinning: tests/test_encoder_oracle.py compares it with golden vectors written
by the installed transformers modules in float64
(tests/golden/make_encoder_golden.py), including a padded batch run with an
attention mask, with planted mistakes, and with a closed form (zero residual
branches leave only the final norms).
"""

from __future__ import annotations

from oracle.flexrel_oracle import HEAD_DIM, torch_core_chunked


def _ln(x, norm, dtype):
    import torch.nn.functional as F

    w, b, eps = norm
    return F.layer_norm(x, (x.shape[-1],), w.to(dtype), b.to(dtype), eps)


def _silu(x):
    import torch

    return x * torch.sigmoid(x)


def conv_module_reference(x, p, dtype):
    """ConvModule of one item x [n, C] (causal depthwise conv, no biases)."""
    import torch
    import torch.nn.functional as F

    hid = x.shape[-1]
    u = _ln(x, p["conv_ln"], dtype)
    h = u @ p["pw1_w"].to(dtype).t()
    g = h[:, :hid] * torch.sigmoid(h[:, hid:])
    taps = p["dw_w"].to(dtype)                       # [C, K]
    k = taps.shape[1]
    gp = F.pad(g.t()[None], (k - 1, 0))              # [1, C, n + K - 1]
    y = F.conv1d(gp, taps[:, None, :], groups=hid)[0].t()
    y = _silu(_ln(y, p["dw_ln"], dtype))
    return y @ p["pw2_w"].to(dtype).t()


def _ffn(u, p, which, dtype):
    h = _silu(u @ p[f"{which}_w1"].to(dtype).t() + p[f"{which}_b1"].to(dtype))
    return h @ p[f"{which}_w2"].to(dtype).t() + p[f"{which}_b2"].to(dtype)


def layer_reference(x, p, heads: int, dtype):
    """One conformer layer on one item x [n, C]."""
    import torch

    n, hid = x.shape
    x = x + 0.5 * _ffn(_ln(x, p["ffn1_ln"], dtype), p, "ffn1", dtype)
    u = _ln(x, p["attn_ln"], dtype)
    q, k, v = ((u @ p[f"{t}_w"].to(dtype).t() + p[f"{t}_b"].to(dtype)).reshape(1, n, heads, HEAD_DIM)
               .permute(0, 2, 1, 3) for t in "qkv")
    ctx = torch_core_chunked(q, k, v, p["rel"], None, dtype=dtype)
    ctx = ctx.permute(0, 2, 1, 3).reshape(n, hid)
    x = x + ctx @ p["out_w"].to(dtype).t() + p["out_b"].to(dtype)
    x = x + conv_module_reference(x, p, dtype)
    x = x + 0.5 * _ffn(_ln(x, p["ffn2_ln"], dtype), p, "ffn2", dtype)
    return _ln(x, p["final_ln"], dtype)


def encoder_reference(features, weights, lens=None, dtype=None):
    """features [B, L, F] torch tensor; weights as in the module docstring
    (``heads`` included); lens [B] valid frames or None.  Computes in
    ``dtype`` (default float64) on the features' device; returns [B, L, C]
    with zero rows past each item's valid length."""
    import torch

    dtype = torch.float64 if dtype is None else dtype
    batch, length, _ = features.shape
    heads = int(weights["heads"])
    hid = weights["fp_w"].shape[0]
    assert hid == heads * HEAD_DIM
    lens = [length] * batch if lens is None else [int(n) for n in lens]
    out = torch.zeros(batch, length, hid, dtype=dtype, device=features.device)
    for b, n in enumerate(lens):
        x = features[b, :n].to(dtype)
        x = _ln(x, weights["fp_ln"], dtype) @ weights["fp_w"].to(dtype).t() + weights["fp_b"].to(dtype)
        for p in weights["layers"]:
            x = layer_reference(x, p, heads, dtype)
        out[b, :n] = x
    return out
