"""ctypes binding of libsidon_flexrel.so (the C ABI in include/sidon_flexrel.h and
include/sidon_encoder.h).

There is no fallback: if the library is missing or fails to load, every entry
point raises.  The library is built by ``build.py`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsidon_flexrel.so"

SIDON_OK = 0
ERROR_NAMES = {
    -1: "SIDON_E_NULL",
    -2: "SIDON_E_SHAPE",
    -3: "SIDON_E_STRIDE",
    -4: "SIDON_E_ALIGN",
    -5: "SIDON_E_LAUNCH",
    -6: "SIDON_E_DEVICE",
    -7: "SIDON_E_CONFIG",
}

# Every symbol include/*.h declares, with its ctypes signature.
_I64P = ctypes.POINTER(ctypes.c_int64)
_IP = ctypes.POINTER(ctypes.c_int)
_VP = ctypes.c_void_p
SIGNATURES = {
    "sidon_flexrel_fwd": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, _I64P, _I64P, _I64P, _I64P, _VP]),
    "sidon_flexrel_fwd_qkv": (ctypes.c_int, [_VP, _VP, _VP, _VP, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, _VP]),
    "sidon_flexrel_launch_shape": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int, _IP, _IP,
                                                  _IP, _IP]),
    "sidon_flexrel_debug_rerun_all": (None, [ctypes.c_int]),
    "sidon_res_norm": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, ctypes.c_float, ctypes.c_int, _VP, _VP,
                                      ctypes.c_float, _VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_glu": (ctypes.c_int, [_VP, _VP, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_silu": (ctypes.c_int, [_VP, ctypes.c_int64, _VP]),
    "sidon_gemm_bias_act_fits": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sidon_gemm_bias_act_preferred": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sidon_gemm_bias_act": (ctypes.c_int, [_VP, ctypes.c_int, _VP, ctypes.c_int, _VP, _VP, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_gemm_lt_act": (ctypes.c_int, [_VP, ctypes.c_int, _VP, ctypes.c_int, _VP, _VP, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_gemm_res_fits": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sidon_gemm_res_preferred": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "sidon_gemm_res": (ctypes.c_int, [_VP, ctypes.c_int, _VP, ctypes.c_int, _VP, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_gemm_nt": (ctypes.c_int, [_VP, ctypes.c_int, _VP, ctypes.c_int, _VP, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, _VP]),
    "sidon_gemm_nt_tune": (ctypes.c_int, [_VP, ctypes.c_int, _VP, ctypes.c_int, _VP, _VP, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, _VP,
                                          ctypes.POINTER(ctypes.c_int)]),
    "sidon_gemm_nt_pin": (ctypes.c_int, [ctypes.c_int] * 9),
    "sidon_causal_dw_norm": (ctypes.c_int, [_VP, ctypes.c_int, _VP, _VP, _VP, ctypes.c_float, _VP,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_fbank_frames": (ctypes.c_int, [_VP, _VP, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_fbank_logmel": (ctypes.c_int, [_VP, _VP, _VP, _VP, ctypes.c_int, _VP, ctypes.c_int, _VP]),
    "sidon_fbank_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_int]),
    "sidon_fbank_normalize": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_size_t, _VP, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_fbank_normalize_noalloc": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_int, ctypes.c_int, _VP]),
    "sidon_last_error": (ctypes.c_char_p, []),
    "sidon_version": (ctypes.c_char_p, []),
}

_lib = None


class SidonError(RuntimeError):
    """A nonzero return code of the C ABI."""

    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed with {ERROR_NAMES.get(code, code)}: {message}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load the HIP library once (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(func: str, code: int) -> None:
    if code != SIDON_OK:
        msg = load().sidon_last_error().decode(errors="replace")
        raise SidonError(func, code, msg)


def strides3(st) -> ctypes.Array:
    return (ctypes.c_int64 * 3)(*[int(x) for x in st])


def launch_shape(batch: int, heads: int, length: int) -> dict:
    """(queries per workgroup, key splits, workgroups, threads) the library uses."""
    lib = load()
    vals = [ctypes.c_int() for _ in range(4)]
    check("sidon_flexrel_launch_shape",
          lib.sidon_flexrel_launch_shape(batch, heads, length, *[ctypes.byref(x) for x in vals]))
    keys = ("queries_per_block", "key_splits", "workgroups", "threads_per_block")
    return {k: v.value for k, v in zip(keys, vals)}


def version() -> str:
    return load().sidon_version().decode()
