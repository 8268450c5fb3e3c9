"""Plain GEMMs of the encoder and the front end on rocBLAS (csrc/blas.hip).

``gemm_nt(x, w, out, beta=0.0)`` computes ``out = x . w^T + beta * out`` for
row-major x [M, K] and w [N, K] (rows K-contiguous) with fp32 sums, in three
type combinations:

  * fp32 x, w, out -- the framing matmul of the front end
    (src/sidon_triton/frontend.py:222);
  * fp16 x, w, out (beta 0) -- the pointwise conv's first F.linear
    (src/sidon_triton/triton_encoder.py:504);
  * fp16 x, w and an fp32 out, beta 1 -- the form of the residual projections
    of res(), ``torch.addmm(x, a, W^T, out_dtype=float32, out=x)`` (:491-492).
    The encoder does not use rocBLAS for those: inside its graph rocBLAS's
    timed choice measured no faster (feed-forward output) or slower (the
    hidden -> hidden projections) than torch.addmm, which it keeps for long
    chunks, and short chunks take ``conformer.residual_gemm``.

The first call of a problem (shape, strides, types, beta != 0) on a device,
made while the stream is not capturing, times rocBLAS's kernels for it on
scratch tensors shaped like ``out`` and keeps the fastest one whose product
agrees with rocBLAS's default (``sidon_gemm_nt_tune``; the scratch lives only
for that call).  Later calls, and calls during capture, launch the kept
kernel, or rocBLAS's default before a problem is tuned.  Every candidate is
deterministic; any kernel may use the device's fixed rocBLAS workspace, so
calls on two streams of one device must not overlap.  SIDON_GEMM_TUNE=0 in
the environment keeps rocBLAS's default kernels.

The choice is made by timing, so two processes (or boxes) may keep different
kernels whose outputs differ in the last bits: results are not
bit-reproducible across processes while tuning is on.  ``chosen_kernels()``
returns the kernel kept per problem, and SIDON_GEMM_PIN=<file.json> (a map
from ``problem_name(key)`` to a rocBLAS solution index, e.g. written from
``chosen_kernels()`` of an earlier run) pins those problems to the given
kernels instead of timing them; a kernel rocBLAS does not list for the
problem is refused on its first call.
"""

from __future__ import annotations

import ctypes
import json
import os

import torch

from . import _lib
from .flexrel import _check_device_tensor, _stream_handle

# (operand dtype, output dtype) -> the C ABI's dtype code
_DTYPES = {
    (torch.float32, torch.float32): 0,
    (torch.float16, torch.float16): 1,
    (torch.float16, torch.float32): 2,
}
_tuned: set = set()
_chosen: dict = {}      # problem key -> rocBLAS solution index (INT_MIN: rocBLAS's default)
_pins = None            # SIDON_GEMM_PIN contents, read on first use


def problem_name(key) -> str:
    """'M,N,K,ldx,ldw,ldy,dtype,beta_nonzero' of a problem key (device omitted)."""
    return ",".join(str(int(v)) for v in key[1:])


def chosen_kernels() -> dict:
    """{problem_name: solution index} of the problems tuned or pinned in this process."""
    return {problem_name(k): v for k, v in _chosen.items()}


def _pinned(key):
    global _pins
    if _pins is None:
        path = os.environ.get("SIDON_GEMM_PIN")
        _pins = {}
        if path:
            with open(path) as f:
                _pins = {str(k): int(v) for k, v in json.load(f).items()}
    return _pins.get(problem_name(key))


def tuning_enabled() -> bool:
    return os.environ.get("SIDON_GEMM_TUNE", "1") != "0"


def gemm_nt(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor, beta: float = 0.0) -> torch.Tensor:
    """out = x . w^T + beta * out (in place); returns out."""
    device = x.device
    for name, t in (("x", x), ("w", w), ("out", out)):
        _check_device_tensor(name, t, device)
        if t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"{name} must be a 2-D tensor with contiguous rows")
    if w.dtype != x.dtype:
        raise ValueError(f"x is {x.dtype}, w {w.dtype}")
    dtype = _DTYPES.get((x.dtype, out.dtype))
    if dtype is None:
        raise ValueError(f"unsupported types: {x.dtype} operands with a {out.dtype} output")
    if dtype == 1 and beta != 0.0:
        raise ValueError("an fp16 output takes beta = 0 only")
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k or tuple(out.shape) != (m, n):
        raise ValueError(f"shapes x {tuple(x.shape)}, w {tuple(w.shape)}, out {tuple(out.shape)} do not match")
    lib = _lib.load()
    head = (x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0))
    key = (device.index, m, n, k, x.stride(0), w.stride(0), out.stride(0), dtype, beta != 0.0)
    with torch.cuda.device(device):
        stream = _stream_handle(device)
        pin = _pinned(key) if key not in _tuned else None
        if pin is not None:
            _lib.check("sidon_gemm_nt_pin", lib.sidon_gemm_nt_pin(m, n, k, x.stride(0), w.stride(0), out.stride(0),
                                                                  dtype, int(beta != 0.0), pin))
            _tuned.add(key)
            _chosen[key] = pin
        if key not in _tuned and tuning_enabled() and not torch.cuda.is_current_stream_capturing():
            scratch = torch.zeros(2, m, out.stride(0), device=device, dtype=out.dtype)
            solution = ctypes.c_int(0)
            rc = lib.sidon_gemm_nt_tune(*head, scratch[0].data_ptr(), scratch[1].data_ptr(), out.stride(0), m, n, k,
                                        dtype, float(beta), stream, ctypes.byref(solution))
            _lib.check("sidon_gemm_nt_tune", rc)
            _tuned.add(key)
            _chosen[key] = solution.value
        rc = lib.sidon_gemm_nt(*head, out.data_ptr(), out.stride(0), m, n, k, dtype, float(beta), stream)
    _lib.check("sidon_gemm_nt", rc)
    return out
