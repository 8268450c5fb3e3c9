"""The conformer layer's elementwise and convolution ops on the MI355X library.

Same names and argument meaning as src/sidon_triton/triton_encoder.py:

  * ``glu(h)`` (:127-133): h [R, 2C] fp16 -> h[:, :C] * sigmoid(h[:, C:]) fp16;
  * ``causal_dw_norm(g, batch, dwt, ln_w, ln_b, eps)`` (:163-181): g [B*T, C]
    fp16, dwt [K, C] fp32 -> silu(LN(causal depthwise conv)) fp16;
  * ``silu_(h)``: the in-place F.silu of the feed-forward modules (:498-499);
  * ``linear_silu(x, w, b)``: the feed-forward input projection and that SiLU
    in one kernel (``silu_(torch.addmm(b, x, w.t()))`` up to the GEMM's
    summation order; csrc/gemm.hip), for the shapes ``linear_silu_fits``
    accepts (N a multiple of 256, K of 64);

plus ``glu_causal_dw_norm(h, ...)``, the two fused: it reads the pointwise
conv's output h [B*T, 2C] and forms g on the fly (bit-identical to
``causal_dw_norm(glu(h), ...)``, without the g round trip through HBM).

All launch on the current stream of the tensors' device through the C ABI of
include/sidon_encoder.h (csrc/conformer_ops.hip) and allocate only their
outputs (none when ``out`` is given), so they can be captured into HIP graphs.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .flexrel import _check_device_tensor, _stream_handle


def _fp16_rows(name, t, device, cols=None):
    _check_device_tensor(name, t, device)
    if t.dtype != torch.float16 or t.dim() != 2 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float16 [R, C] tensor")
    if cols is not None and t.shape[1] != cols:
        raise ValueError(f"{name} must have {cols} columns (got {t.shape[1]})")


def glu(h: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    rows, c2 = h.shape
    if c2 % 2:
        raise ValueError("h must have an even number of columns")
    device = h.device
    _fp16_rows("h", h, device)
    c = c2 // 2
    if out is None:
        out = torch.empty(rows, c, device=device, dtype=h.dtype)
    else:
        _fp16_rows("out", out, device, c)
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_glu(h.data_ptr(), out.data_ptr(), rows, c, _stream_handle(device))
    _lib.check("sidon_glu", rc)
    return out


def silu_(h: torch.Tensor) -> torch.Tensor:
    """h = h * sigmoid(h) in place (fp16, any shape, contiguous)."""
    device = h.device
    _check_device_tensor("h", h, device)
    if h.dtype != torch.float16 or not h.is_contiguous():
        raise ValueError("h must be a contiguous float16 tensor")
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_silu(h.data_ptr(), h.numel(), _stream_handle(device))
    _lib.check("sidon_silu", rc)
    return h


def _dw(src, glu_input, batch, dwt, ln_w, ln_b, eps, out):
    rows, width = src.shape
    c = width // 2 if glu_input else width
    device = src.device
    _fp16_rows("h" if glu_input else "g", src, device)
    if rows % batch:
        raise ValueError(f"{rows} rows do not split into {batch} items")
    for name, t, shape in (("dwt", dwt, None), ("ln_w", ln_w, (c,)), ("ln_b", ln_b, (c,))):
        _check_device_tensor(name, t, device)
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 tensor")
        if shape is not None and tuple(t.shape) != shape:
            raise ValueError(f"{name} must be [{c}]")
    if dwt.dim() != 2 or dwt.shape[1] != c:
        raise ValueError(f"dwt must be [K, {c}]")
    if out is None:
        out = torch.empty(rows, c, device=device, dtype=torch.float16)
    else:
        _fp16_rows("out", out, device, c)
        if out.shape[0] != rows:
            raise ValueError("out must have the input's rows")
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_causal_dw_norm(src.data_ptr(), int(glu_input), dwt.data_ptr(), ln_w.data_ptr(),
                                      ln_b.data_ptr(), ctypes.c_float(float(eps)), out.data_ptr(), batch,
                                      rows // batch, c, dwt.shape[0], _stream_handle(device))
    _lib.check("sidon_causal_dw_norm", rc)
    return out


def causal_dw_norm(g: torch.Tensor, batch: int, dwt: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor,
                   eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """g [B*T, C] fp16 -> silu(LN(sum_k dwt[k] * g[t + k - (K-1)])) [B*T, C] fp16
    (zero left padding per item; dwt [K, C] fp32, ln_w / ln_b [C] fp32)."""
    return _dw(g, False, batch, dwt, ln_w, ln_b, eps, out)


def glu_causal_dw_norm(h: torch.Tensor, batch: int, dwt: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor,
                       eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """causal_dw_norm(glu(h), ...) in one pass: h [B*T, 2C] fp16."""
    return _dw(h, True, batch, dwt, ln_w, ln_b, eps, out)


def linear_silu_fits(x: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether ``linear_silu`` takes x [M, K] and w [N, K]."""
    return bool(_lib.load().sidon_gemm_bias_act_fits(x.shape[0], w.shape[0], w.shape[1])) and x.shape[1] == w.shape[1]


def linear_silu_preferred(rows: int, n: int, k: int, device=None) -> bool:
    """Whether ``linear_silu`` is expected to beat ``silu_(torch.addmm(...))``
    for x [rows, k], w [n, k] on ``device`` (its tiles fill >= 3/4 of the CUs
    in every round; at n = 4096, k = 1024 that is rows > 3840 on 256 CUs)."""
    with torch.cuda.device(device):
        return bool(_lib.load().sidon_gemm_bias_act_preferred(rows, n, k))


def _linear_args(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, out: torch.Tensor | None):
    device = x.device
    for name, t in (("x", x), ("w", w)):
        _check_device_tensor(name, t, device)
        if t.dtype != torch.float16 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"{name} must be a float16 [rows, K] tensor with K contiguous")
    rows, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"x has {k} columns, w {w.shape[1]}")
    if b is not None:
        _check_device_tensor("b", b, device)
        if b.dtype != torch.float16 or tuple(b.shape) != (n,) or not b.is_contiguous():
            raise ValueError(f"b must be a contiguous float16 [{n}] tensor")
    if out is None:
        out = torch.empty(rows, n, device=device, dtype=torch.float16)
    else:
        _check_device_tensor("out", out, device)
        if out.dtype != torch.float16 or tuple(out.shape) != (rows, n) or out.stride(1) != 1:
            raise ValueError(f"out must be a float16 [{rows}, {n}] tensor with rows contiguous")
    return rows, n, k, out


def linear_silu(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, out: torch.Tensor | None = None,
                act: bool = True) -> torch.Tensor:
    """silu(fp16(x . w^T + b)) [M, N] fp16 for x [M, K] and w [N, K] fp16
    (rows K-contiguous), b [N] fp16 or None; act=False leaves out the SiLU."""
    device = x.device
    rows, n, k, out = _linear_args(x, w, b, out)
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_gemm_bias_act(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                     None if b is None else b.data_ptr(), out.data_ptr(), out.stride(0), rows, n, k,
                                     1 if act else 0, _stream_handle(device))
    _lib.check("sidon_gemm_bias_act", rc)
    return out


def linear_silu_lt(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, out: torch.Tensor | None = None,
                   act: bool = True) -> torch.Tensor:
    """silu(x . w^T + b) [M, N] fp16 on hipBLASLt with the bias and SiLU in
    its epilogue (fp32 sum + bias, SiLU in fp32, one rounding to fp16), for
    x [M, K] and w [N, K] fp16 (rows K-contiguous), b [N] fp16 or None;
    act=False leaves out the SiLU.  The first call on a device must not run
    during stream capture."""
    device = x.device
    rows, n, k, out = _linear_args(x, w, b, out)
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_gemm_lt_act(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                                   None if b is None else b.data_ptr(), out.data_ptr(), out.stride(0), rows, n, k,
                                   1 if act else 0, _stream_handle(device))
    _lib.check("sidon_gemm_lt_act", rc)
    return out


def residual_gemm_fits(x: torch.Tensor, a: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether ``residual_gemm`` takes a [M, K], w [N, K] into x [M, N]."""
    return (bool(_lib.load().sidon_gemm_res_fits(a.shape[0], w.shape[0], w.shape[1])) and a.shape[1] == w.shape[1]
            and tuple(x.shape) == (a.shape[0], w.shape[0]))


def residual_gemm_preferred(rows: int, n: int, k: int, device=None) -> bool:
    """Whether ``residual_gemm`` is expected to beat torch.addmm for a
    [rows, k], w [n, k] on ``device`` (its 64 x 64 tiles fit one per compute
    unit: rows <= 1024 at n = 1024 on 256 CUs)."""
    with torch.cuda.device(device):
        return bool(_lib.load().sidon_gemm_res_preferred(rows, n, k))


def residual_gemm(x: torch.Tensor, a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x += a . w^T in place: x [M, N] fp32 (the residual stream), a [M, K]
    and w [N, K] fp16 with K contiguous -- the
    ``torch.addmm(x, a, w.t(), out_dtype=torch.float32, out=x)`` of the
    reference's res() (src/sidon_triton/triton_encoder.py:491-492)."""
    device = x.device
    for name, t in (("a", a), ("w", w)):
        _check_device_tensor(name, t, device)
        if t.dtype != torch.float16 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"{name} must be a float16 [rows, K] tensor with K contiguous")
    _check_device_tensor("x", x, device)
    rows, k = a.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"a has {k} columns, w {w.shape[1]}")
    if x.dtype != torch.float32 or tuple(x.shape) != (rows, n) or x.stride(1) != 1:
        raise ValueError(f"x must be a float32 [{rows}, {n}] tensor with rows contiguous")
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.sidon_gemm_res(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), x.data_ptr(), x.stride(0),
                                rows, n, k, _stream_handle(device))
    _lib.check("sidon_gemm_res", rc)
    return x
