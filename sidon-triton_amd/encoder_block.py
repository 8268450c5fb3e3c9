"""Conformer attention sub-block on the MI355X library.

Mirrors the attention part of ``TritonEncoder.__call__``
(src/sidon_triton/triton_encoder.py:491-503) on the packed weights of
:417-443:

    xn  = res_norm(x, bias=running bias, norm2=attn_ln, write_x=False)   # fp16
    qkv = xn W_qkv^T + b_qkv                     (hipBLASLt through torch)
    ctx = flexrel_attention(qkv, batch, heads, rel, lens)              # this library
    x  += ctx W_out^T                            (fp16 operands, fp32 output into the stream)

The out-projection bias is not added to x by the GEMM; like the reference,
the running sum of the biases of this and the earlier layers (``cum_bias``,
summed in float64, :438-443) is added inside the next norm, and once into x
after the last layer.

``res_norm`` is the HIP kernel of csrc/res_norm.hip (C ABI
``sidon_res_norm``, include/sidon_encoder.h), with the reference's argument
meaning (:84-100).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .encoder_attention import flexrel_attention
from .flexrel import _check_device_tensor, _stream_handle


def _ptr(t):
    return None if t is None else t.data_ptr()


def res_norm(x: torch.Tensor, y: torch.Tensor | None = None, norm1=None, write_x: bool = True, norm2=None,
             bias: torch.Tensor | None = None, xn_dtype=torch.float16, xn: torch.Tensor | None = None):
    """x [R, C] fp32 (in place): x += bias + y; x = LN1(x) (if norm1); stores x
    (if write_x); returns LN2(x) in ``xn_dtype`` (if norm2, else None).
    norm = (weight, bias, eps) with fp32 [C] tensors."""
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 [R, C] tensor")
    rows, cols = x.shape
    device = x.device
    _check_device_tensor("x", x, device)
    for name, t in (("y", y), ("bias", bias)):
        if t is not None:
            _check_device_tensor(name, t, device)
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float32 tensor")
    if y is not None and tuple(y.shape) != (rows, cols):
        raise ValueError("y must have x's shape")
    if bias is not None and tuple(bias.shape) != (cols,):
        raise ValueError("bias must be [C]")
    norms = []
    for norm in (norm1, norm2):
        if norm is None:
            norms.append((None, None, 0.0))
            continue
        w, b, eps = norm
        for t in (w, b):
            _check_device_tensor("norm weight", t, device)
            if t.dtype != torch.float32 or tuple(t.shape) != (cols,) or not t.is_contiguous():
                raise ValueError("norm weights must be contiguous float32 [C] tensors")
        norms.append((w, b, float(eps)))
    if norm2 is not None:
        if xn is None:
            xn = torch.empty(rows, cols, device=device, dtype=xn_dtype)
        elif xn.dtype != xn_dtype or tuple(xn.shape) != (rows, cols) or not xn.is_contiguous():
            raise ValueError("xn must be a contiguous [R, C] tensor of xn_dtype")
        if xn_dtype not in (torch.float16, torch.float32):
            raise TypeError("xn_dtype must be float16 or float32")
    else:
        xn = None
    lib = _lib.load()
    (n1w, n1b, e1), (n2w, n2b, e2) = norms
    with torch.cuda.device(device):
        rc = lib.sidon_res_norm(x.data_ptr(), _ptr(y), _ptr(bias), _ptr(n1w), _ptr(n1b), ctypes.c_float(e1),
                                int(bool(write_x)), _ptr(n2w), _ptr(n2b), ctypes.c_float(e2), _ptr(xn),
                                int(xn_dtype == torch.float16), rows, cols, _stream_handle(device))
    _lib.check("sidon_res_norm", rc)
    return xn


def running_biases(out_biases: list[torch.Tensor]) -> list[torch.Tensor]:
    """fp32 running sums of the layers' out-projection biases, summed in
    float64 (src/sidon_triton/triton_encoder.py:438-443)."""
    acc = None
    sums = []
    for b in out_biases:
        acc = b.double() if acc is None else acc + b.double()
        sums.append(acc.float().contiguous())
    return sums


def attention_blocks(x: torch.Tensor, layers: list[dict], batch: int, heads: int, lens: torch.Tensor | None,
                     buffers: dict | None = None) -> torch.Tensor:
    """Run the attention sub-block of every layer over the fp32 stream
    x [B*L, C] in place and return x (with the running bias added).

    layers: dicts with ``attn_ln`` (w, b, eps) fp32, ``qkv_w`` [3C, C] and
    ``qkv_b`` [3C] fp16, ``rel`` [73, 64] fp16, ``out_w`` [C, C] fp16 and
    ``cum_bias`` [C] fp32 (``running_biases`` of the out-projection biases).
    ``buffers`` (optional) holds preallocated ``xn`` [B*L, C] fp16, ``qkv``
    [B*L, 3C] fp16 and ``ctx`` [B*L, C] fp16, so the call allocates nothing and
    can be captured into a HIP graph."""
    rows, hid = x.shape
    buffers = buffers if buffers is not None else {}
    xn = buffers.get("xn")
    qkv = buffers.get("qkv")
    ctx = buffers.get("ctx")
    if qkv is None:
        qkv = torch.empty(rows, 3 * hid, device=x.device, dtype=torch.float16)
    xn = res_norm(x, norm2=layers[0]["attn_ln"], write_x=False, xn=xn)
    for i, p in enumerate(layers):
        torch.addmm(p["qkv_b"], xn, p["qkv_w"].t(), out=qkv)
        ctx = flexrel_attention(qkv, batch, heads, p["rel"], lens, out=ctx)
        torch.addmm(x, ctx, p["out_w"].t(), out_dtype=torch.float32, out=x)
        last = i + 1 == len(layers)
        xn = res_norm(x, bias=p["cum_bias"], norm2=None if last else layers[i + 1]["attn_ln"],
                      write_x=last, xn=None if last else xn)
    return x
