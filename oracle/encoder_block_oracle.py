"""CPU / torch oracle of the conformer attention sub-block -- TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module.  Only ``tests/`` and
``bench.py``'s c5 check use it, as the checker.

Per layer, on the residual stream x [B, L, C] (C = 64 H):

    u   = LayerNorm(x)                              (w, b, eps)
    q|k|v = u W_qkv^T + b_qkv                        fused [3C, C]
    ctx = relative_key attention (flexrel_oracle)    per head, 73 x 64 table
    x   = x + ctx W_out^T + b_out

Sources restated here (read, not run):
  * transformers ``Wav2Vec2BertEncoderLayer.forward``, lines 436-447 of the
    installed modeling_wav2vec2_bert.py (5.15.0; the reference pins 4.56.1,
    pyproject.toml:16): residual, self_attn_layer_norm, self_attn, + residual;
    ``Wav2Vec2BertSelfAttention`` (linear_q/k/v with biases, relative_key,
    linear_out with bias);
  * src/sidon_triton/triton_encoder.py:491-503, the same sub-block on packed
    weights (``qkv_w = cat(Wq, Wk, Wv)``, :417-422), whose out-projection
    bias is carried as a running sum into the next norm (:438-443) -- here
    it is added directly, so the equivalence is what the GPU tests check.

Pinning: tests/test_block_oracle.py compares it with golden vectors written by
the installed transformers modules in float64 (tests/golden/make_block_golden.py)
and with a closed form (zero Q/K projections make every score equal, so the
context is the mean of the valid V rows).
"""

from __future__ import annotations

from oracle.flexrel_oracle import HEAD_DIM, torch_core_chunked


def attention_blocks_reference(x, layers, heads: int, lens=None, dtype=None):
    """x [B, L, C] torch tensor; layers: dicts with ``attn_ln`` (w, b, eps),
    ``qkv_w`` [3C, C], ``qkv_b`` [3C], ``rel`` [73, 64], ``out_w`` [C, C],
    ``out_b`` [C].  Computes in ``dtype`` (default float64) on x's device and
    returns the stream after all layers."""
    import torch
    import torch.nn.functional as F

    dtype = torch.float64 if dtype is None else dtype
    batch, length, hid = x.shape
    assert hid == heads * HEAD_DIM
    x = x.to(dtype)
    for p in layers:
        w, b, eps = p["attn_ln"]
        u = F.layer_norm(x, (hid,), w.to(dtype), b.to(dtype), eps)
        qkv = u @ p["qkv_w"].to(dtype).t() + p["qkv_b"].to(dtype)
        q, k, v = (qkv[..., i * hid:(i + 1) * hid].reshape(batch, length, heads, HEAD_DIM).permute(0, 2, 1, 3)
                   for i in range(3))
        ctx = torch_core_chunked(q, k, v, p["rel"], lens, dtype=dtype)
        ctx = ctx.permute(0, 2, 1, 3).reshape(batch, length, hid)
        x = x + ctx @ p["out_w"].to(dtype).t() + p["out_b"].to(dtype)
    return x
