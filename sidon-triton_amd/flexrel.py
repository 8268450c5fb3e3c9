"""Strided [B, H, L, 64] relative_key attention on the HIP kernel.

Mirrors ``flexrel_attention(q, k, v, r, out=None)`` of
src/sidon_triton/flexrel_triton.py:249-278 (same argument meaning, same
asserts), plus the optional device ``lens`` of the encoder kernel
(src/sidon_triton/triton_encoder.py:219-226): keys j >= lens[b] weigh zero.
"""

from __future__ import annotations

import torch

from . import _lib

LEFT, RIGHT = 64, 8
NUM_POS = LEFT + RIGHT + 1  # 73
HEAD_DIM = 64


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check_device_tensor(name: str, t: torch.Tensor, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on a HIP device (got {t.device})")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, q is on {device}")


def flexrel_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, r: torch.Tensor,
                      out: torch.Tensor | None = None,
                      lens: torch.Tensor | None = None) -> torch.Tensor:
    """q, k, v: [B, H, L, 64] fp16 (last dim contiguous), r: [73, 64] fp16 contiguous.

    lens: optional int32 [B] on the same device (valid keys per item; None =
    L).  out: optional fp16 [B, H, L, 64] with a contiguous last dim;
    allocated contiguous when None.  Launches on the current stream of q's
    device and returns ``out``.
    """
    batch, heads, length, dim = q.shape
    assert dim == HEAD_DIM and tuple(r.shape) == (NUM_POS, dim), (q.shape, r.shape)
    assert q.stride(-1) == k.stride(-1) == v.stride(-1) == 1
    assert r.is_contiguous()
    device = q.device
    for name, t in (("q", q), ("k", k), ("v", v), ("r", r)):
        _check_device_tensor(name, t, device)
        if t.dtype != torch.float16:
            raise TypeError(f"{name} must be float16 (got {t.dtype})")
    if tuple(k.shape) != tuple(q.shape) or tuple(v.shape) != tuple(q.shape):
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} differ")
    if lens is not None:
        _check_device_tensor("lens", lens, device)
        if lens.dtype != torch.int32 or tuple(lens.shape) != (batch,) or not lens.is_contiguous():
            raise ValueError("lens must be a contiguous int32 tensor of shape [B]")
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    else:
        _check_device_tensor("out", out, device)
        if out.dtype != torch.float16 or tuple(out.shape) != tuple(q.shape) or out.stride(-1) != 1:
            raise ValueError("out must be float16 [B, H, L, 64] with a contiguous last dim")
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_flexrel_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), r.data_ptr(),
            None if lens is None else lens.data_ptr(), out.data_ptr(),
            batch, heads, length, dim,
            _lib.strides3(q.stride()[:3]), _lib.strides3(k.stride()[:3]),
            _lib.strides3(v.stride()[:3]), _lib.strides3(out.stride()[:3]),
            _stream_handle(device))
    _lib.check("sidon_flexrel_fwd", rc)
    return out
