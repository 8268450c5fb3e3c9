"""sidon-triton_amd: the Sidon-Triton encoder's relative_key flash attention,
rebuilt for MI355X (gfx950) as hand-written HIP behind a C ABI.

Entry points (same argument meaning as the reference):
  * ``flexrel.flexrel_attention(q, k, v, r, out=None, lens=None)`` --
    src/sidon_triton/flexrel_triton.py:249 ([B, H, L, 64] strided views);
  * ``encoder_attention.flexrel_attention(qkv, batch, heads, rel, lens)`` --
    src/sidon_triton/triton_encoder.py:346 (fused QKV rows);
  * ``graphs.BucketGraphs`` -- one HIP graph per length bucket
    (src/sidon_triton/runtime.py:374-401);
  * ``encoder_block.res_norm`` / ``encoder_block.attention_blocks`` -- the
    residual LayerNorm and the conformer attention sub-block around the
    attention (src/sidon_triton/triton_encoder.py:61-100, :491-503);
  * ``conformer.glu`` / ``conformer.causal_dw_norm`` / ``conformer.silu_`` --
    the conv module's and feed-forward's kernels (triton_encoder.py:113-181);
  * ``blas.gemm_nt`` -- the encoder's and the front end's plain library GEMMs
    on rocBLAS, kernel chosen per problem by timing (triton_encoder.py:491-492,
    :504; frontend.py:222);
  * ``encoder.pack_encoder`` / ``encoder.HipEncoder`` / ``encoder.save_encoder``
    / ``encoder.load_encoder`` -- the whole 8-layer conformer encoder
    (triton_encoder.py:392-525);
  * ``runtime.EncoderRuntime`` -- bucketed, graph-captured encoder calls on
    fixed max-size buffers (src/sidon_triton/runtime.py:74-186, :366-401);
  * ``frontend.Fbank`` -- the bucket-masked fbank front end that produces the
    encoder's features and valid frames (src/sidon_triton/frontend.py:175-246);
  * ``modeling.HipRelSelfAttention`` / ``modeling.replace_attention_with_hip``
    -- the module drop-in for transformers' relative_key self-attention
    (src/sidon_triton/modeling.py:40-131).

The package directory name is not a Python identifier; the repository's
entry scripts load it under the module name ``sidon_triton_amd``.
"""

from . import (_lib, blas, conformer, encoder, encoder_attention, encoder_block, flexrel, frontend, graphs,
               modeling, runtime)
from .flexrel import HEAD_DIM, LEFT, NUM_POS, RIGHT, flexrel_attention

__all__ = [
    "HEAD_DIM",
    "LEFT",
    "NUM_POS",
    "RIGHT",
    "blas",
    "conformer",
    "encoder",
    "encoder_attention",
    "encoder_block",
    "flexrel",
    "flexrel_attention",
    "frontend",
    "graphs",
    "modeling",
    "runtime",
    "_lib",
]
