"""C ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and rejects bad arguments before launching."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "sidon_flexrel.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))


def header_functions() -> list[str]:
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(sidon_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def header_codes() -> dict[str, int]:
    return {m[0]: int(m[1]) for m in re.findall(r"#define\s+(SIDON_(?:OK|E_[A-Z]+))\s+\(?(-?\d+)\)?",
                                                 HEADER.read_text())}


def test_library_exports_every_header_function(sidon):
    lib = ctypes.CDLL(str(sidon._lib.LIB_PATH))
    names = header_functions()
    assert names == sorted(sidon._lib.SIGNATURES), names
    for name in names:
        assert hasattr(lib, name), name


def test_error_codes_match_header(sidon):
    codes = header_codes()
    assert codes["SIDON_OK"] == sidon._lib.SIDON_OK
    assert {v: k for k, v in codes.items() if k != "SIDON_OK"} == sidon._lib.ERROR_NAMES


def test_version(sidon):
    assert "gfx950" in sidon._lib.version()


@pytest.mark.parametrize("B,H,L", [(1, 16, 4800), (1, 16, 750), (1, 16, 1500), (4, 16, 100), (1, 1, 1)])
def test_launch_shape(sidon, B, H, L):
    s = sidon._lib.launch_shape(B, H, L)
    qpb = s["queries_per_block"]
    assert s["workgroups"] == B * H * -(-L // qpb)
    assert s["threads_per_block"] % 64 == 0
    assert s["key_splits"] >= 1


def _fwd(lib, **over):
    st = (ctypes.c_int64 * 3)(4800 * 64 * 16, 4800 * 64, 64)
    args = dict(q=16, k=16, v=16, rel=16, lens=None, out=16, B=1, H=16, L=4800, D=64,
                qs=st, ks=st, vs=st, os=st, stream=None)
    args.update(over)
    return lib.sidon_flexrel_fwd(args["q"], args["k"], args["v"], args["rel"], args["lens"],
                                 args["out"], args["B"], args["H"], args["L"], args["D"],
                                 args["qs"], args["ks"], args["vs"], args["os"], args["stream"])


@pytest.mark.parametrize("over,code", [
    (dict(q=None), -1),
    (dict(out=None), -1),
    (dict(rel=None), -1),
    (dict(D=128), -2),
    (dict(B=0), -2),
    (dict(L=0), -2),
    (dict(H=-1), -2),
    (dict(qs=(ctypes.c_int64 * 3)(0, 0, 60)), -3),
    (dict(os=(ctypes.c_int64 * 3)(-64, 0, 64)), -3),
    (dict(ks=(ctypes.c_int64 * 3)(0, 0, 1 << 26)), -3),
    (dict(qs=None), -1),
    (dict(q=24), -4),
    (dict(rel=8), -4),
])
def test_rejects_bad_arguments_before_launch(sidon, over, code):
    # fake (never dereferenced) 16-byte aligned addresses: validation returns
    # before any HIP call, so this runs without a GPU
    lib = sidon._lib.load()
    rc = _fwd(lib, **over)
    assert rc == code
    assert lib.sidon_last_error().decode()


def test_qkv_entry_rejects_bad_arguments(sidon):
    lib = sidon._lib.load()
    assert lib.sidon_flexrel_fwd_qkv(None, 16, None, 16, 1, 16, 100, None) == -1
    assert lib.sidon_flexrel_fwd_qkv(16, 16, None, 16, 1, 0, 100, None) == -2
    assert lib.sidon_flexrel_fwd_qkv(24, 16, None, 16, 1, 16, 100, None) == -4


def test_python_wrappers_reject_host_tensors(sidon):
    import torch

    q = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    rel = torch.zeros(73, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="HIP device"):
        sidon.flexrel.flexrel_attention(q, q, q, rel)
    with pytest.raises(AssertionError):
        sidon.flexrel.flexrel_attention(q[..., :32], q[..., :32], q[..., :32], rel[:, :32])
    qkv = torch.zeros(8, 3 * 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="HIP device"):
        sidon.encoder_attention.flexrel_attention(qkv, 1, 2, rel, None)
    with pytest.raises(AssertionError):
        sidon.encoder_attention.flexrel_attention(qkv, 1, 2, torch.zeros(72, 64, dtype=torch.float16), None)


def test_gemm_shape_support(sidon):
    lib = sidon._lib.load()
    assert lib.sidon_gemm_bias_act_fits(4800, 4096, 1024) == 1
    assert lib.sidon_gemm_bias_act_fits(1, 256, 64) == 1
    for m, n, k in ((0, 4096, 1024), (4800, 4000, 1024), (4800, 128, 1024), (4800, 4096, 1000), (4800, 4096, 32)):
        assert lib.sidon_gemm_bias_act_fits(m, n, k) == 0, (m, n, k)


@pytest.mark.parametrize("over,code", [
    (dict(x=None), -1),
    (dict(y=None), -1),
    (dict(N=4000), -2),
    (dict(K=1000), -2),
    (dict(M=0), -2),
    (dict(act=2), -2),
    (dict(ldx=1000), -3),
    (dict(ldy=4095), -3),
    (dict(x=24), -4),
    (dict(bias=12), -4),
])
def test_gemm_rejects_bad_arguments_before_launch(sidon, over, code):
    # fake aligned addresses, never dereferenced: validation returns before any HIP call
    lib = sidon._lib.load()
    args = dict(x=16, ldx=1024, w=16, ldw=1024, bias=16, y=16, ldy=4096, M=4800, N=4096, K=1024, act=1)
    args.update(over)
    rc = lib.sidon_gemm_bias_act(args["x"], args["ldx"], args["w"], args["ldw"], args["bias"], args["y"],
                                 args["ldy"], args["M"], args["N"], args["K"], args["act"], None)
    assert rc == code
    assert lib.sidon_last_error().decode()
