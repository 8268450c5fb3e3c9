"""Encoder-layout attention op: fused QKV rows in, context rows out.

Mirrors ``flexrel_attention(qkv, batch, heads, rel, lens)`` of
src/sidon_triton/triton_encoder.py:346-371: q / k / v are the three column
blocks of one fused QKV GEMM output, the context comes back as
[B*L, H*64] rows ready for the out-projection GEMM.  Same asserts
(head dim 64, rel [73, 64]); ``lens`` is the device int32 [B] vector of
valid keys per item.
"""

from __future__ import annotations

import torch

from . import _lib
from .flexrel import HEAD_DIM, NUM_POS, _check_device_tensor, _stream_handle


def flexrel_attention(qkv: torch.Tensor, batch: int, heads: int, rel: torch.Tensor,
                      lens: torch.Tensor | None, out: torch.Tensor | None = None) -> torch.Tensor:
    """qkv [B*L, 3*H*64] fp16 (q | k | v column blocks), rel [73, 64] fp16,
    lens int32 [B] valid keys -> context [B*L, H*64] fp16."""
    rows, width = qkv.shape
    hidden = width // 3
    dim = hidden // heads
    length = rows // batch
    assert dim == HEAD_DIM and tuple(rel.shape) == (NUM_POS, dim)
    assert width == 3 * heads * dim and rows == batch * length
    device = qkv.device
    _check_device_tensor("qkv", qkv, device)
    _check_device_tensor("rel", rel, device)
    if qkv.dtype != torch.float16 or rel.dtype != torch.float16:
        raise TypeError("qkv and rel must be float16")
    if not qkv.is_contiguous() or not rel.is_contiguous():
        raise ValueError("qkv and rel must be contiguous")
    if lens is not None:
        _check_device_tensor("lens", lens, device)
        if lens.dtype != torch.int32 or tuple(lens.shape) != (batch,) or not lens.is_contiguous():
            raise ValueError("lens must be a contiguous int32 tensor of shape [B]")
    if out is None:
        out = torch.empty(rows, hidden, device=device, dtype=qkv.dtype)
    elif out.dtype != torch.float16 or tuple(out.shape) != (rows, hidden) or not out.is_contiguous():
        raise ValueError("out must be a contiguous float16 [B*L, H*64] tensor")
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_flexrel_fwd_qkv(qkv.data_ptr(), rel.data_ptr(),
                                       None if lens is None else lens.data_ptr(),
                                       out.data_ptr(), batch, heads, length, _stream_handle(device))
    _lib.check("sidon_flexrel_fwd_qkv", rc)
    return out
