"""Module drop-in for transformers' relative_key self-attention.

Mirrors ``FlexRelSelfAttention`` / ``replace_attention_with_flex`` of
src/sidon_triton/modeling.py:40-131: a module with the parameters of
``Wav2Vec2BertSelfAttention`` (``linear_q/k/v/out``, ``distance_embedding``;
its state dict loads strictly) whose forward runs this library's attention
kernel, and a helper that swaps it into every layer of a w2v-BERT encoder.

forward(hidden_states [B, L, C], attention_mask=None, ...) -> (out, None):
the projections run in the module's dtype; q / k / v go to the kernel as
fp16 [B, H, L, 64] views of the projection outputs (no copy when the module
is fp16), the table as fp16, and the context comes back to the module's
dtype for ``linear_out``.  Unlike the reference (which asserts the mask is
None, :95) a key-padding mask is accepted: transformers' additive
[B, 1, L, L] mask (0 for kept keys, a large negative number for padded
ones, the same row for every query) or a [B, L] 0/1 mask becomes the
kernel's per-item valid length; any other mask is rejected.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .flexrel import HEAD_DIM, LEFT, NUM_POS, RIGHT, flexrel_attention


def _lens_from_mask(mask: torch.Tensor, batch: int, length: int) -> torch.Tensor:
    """Valid keys per item of a right-padded key mask (int32 [B] on the
    mask's device)."""
    if mask.dim() == 2:
        keep = mask != 0
    elif mask.dim() == 4 and mask.shape[1] == 1:
        rows = mask[:, 0]
        if not torch.equal(rows, rows[:, :1].expand_as(rows)):
            raise ValueError("only key-padding masks (the same row for every query) are supported")
        keep = rows[:, 0] == 0
    else:
        raise ValueError(f"unsupported attention mask of shape {tuple(mask.shape)}")
    if tuple(keep.shape) != (batch, length):
        raise ValueError(f"mask covers {tuple(keep.shape)} keys, the input has {(batch, length)}")
    lens = keep.sum(dim=1)
    prefix = torch.arange(length, device=keep.device)[None, :] < lens[:, None]
    if not torch.equal(prefix, keep):
        raise ValueError("the kept keys must be a prefix of each row (right padding)")
    return lens.to(torch.int32).contiguous()


class HipRelSelfAttention(nn.Module):
    """relative_key self-attention (window -64..+8) on the MI355X kernel."""

    def __init__(self, hidden_size: int, num_heads: int, left_max_position: int = LEFT,
                 right_max_position: int = RIGHT) -> None:
        super().__init__()
        if hidden_size != num_heads * HEAD_DIM:
            raise ValueError(f"hidden size {hidden_size} must be {HEAD_DIM} x {num_heads} heads")
        if (left_max_position, right_max_position) != (LEFT, RIGHT):
            raise ValueError(f"the kernel's window is -{LEFT}..+{RIGHT}")
        self.num_heads = num_heads
        self.head_dim = HEAD_DIM
        self.left_max_position = left_max_position
        self.right_max_position = right_max_position
        self.linear_q = nn.Linear(hidden_size, hidden_size)
        self.linear_k = nn.Linear(hidden_size, hidden_size)
        self.linear_v = nn.Linear(hidden_size, hidden_size)
        self.linear_out = nn.Linear(hidden_size, hidden_size)
        self.distance_embedding = nn.Embedding(NUM_POS, HEAD_DIM)

    def forward(self, hidden_states: torch.Tensor, attention_mask: torch.Tensor | None = None,
                relative_position_embeddings: torch.Tensor | None = None, output_attentions: bool = False,
                **_: object) -> tuple[torch.Tensor, None]:
        batch, length, hidden = hidden_states.shape
        shape = (batch, length, self.num_heads, self.head_dim)
        q, k, v = (lin(hidden_states).to(torch.float16).view(shape).transpose(1, 2)
                   for lin in (self.linear_q, self.linear_k, self.linear_v))
        rel = self.distance_embedding.weight.to(torch.float16).contiguous()
        lens = None if attention_mask is None else _lens_from_mask(attention_mask, batch, length)
        context = flexrel_attention(q, k, v, rel, lens=lens)
        context = context.transpose(1, 2).reshape(batch, length, hidden).to(hidden_states.dtype)
        return self.linear_out(context), None


def replace_attention_with_hip(ssl_model: nn.Module) -> int:
    """Swap every self-attention of a w2v-BERT encoder (``ssl_model.encoder.layers``)
    for ``HipRelSelfAttention`` with the same weights; returns the count."""
    config = ssl_model.config
    count = 0
    for layer in ssl_model.encoder.layers:
        source = layer.self_attn
        hip = HipRelSelfAttention(int(config.hidden_size), int(config.num_attention_heads),
                                  int(config.left_max_position_embeddings),
                                  int(config.right_max_position_embeddings))
        hip = hip.to(source.linear_q.weight.device, source.linear_q.weight.dtype)
        hip.load_state_dict(source.state_dict(), strict=True)
        layer.self_attn = hip
        count += 1
    return count
