"""Build libsidon_flexrel.so (HIP, gfx950) in-tree with hipcc.

The library is compiled from csrc/*.hip into this package directory, where
``_lib.py`` loads it.  Every call recompiles (the build check of the repo);
the output is written to a temporary name and renamed, so a concurrent reader
never sees a half-written file.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
LIB_NAME = "libsidon_flexrel.so"
SOURCES = [PKG_DIR / "csrc" / name
           for name in ("flexrel_fwd.hip", "flexrel_w64.hip", "flexrel_w32.hip", "res_norm.hip", "conformer_ops.hip", "fbank.hip", "gemm.hip", "gemm_res.hip", "blas.hip", "blaslt.hip")]
# rocBLAS for the plain GEMMs of csrc/blas.hip.  Its soname is the one torch
# bundles, so inside a torch process the library shares torch's copy.
LIBS = ["-lrocblas", "-lhipblaslt"]
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the generated code.
# -amdgpu-mfma-vgpr-form: MFMA accumulators in ordinary VGPRs, so the softmax
# reads the scores without AGPR copies (one wavefront per SIMD uses all 512).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def generate(verbose: bool = False) -> None:
    """Writes csrc/flexrel_w64_step.inc (the hand-scheduled key-step loop of
    flexrel_w64.hip) from csrc/gen_w64_step.py, which also checks its wait
    states and load accounting."""
    for name in ("gen_w64_step.py",):
        gen = PKG_DIR / "csrc" / name
        proc = subprocess.run([sys.executable, str(gen)], capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"{gen.name} failed ({proc.returncode}):\n{proc.stdout}{proc.stderr}")
        if verbose:
            print(proc.stderr.strip(), flush=True)


def build(verbose: bool = False) -> Path:
    """Compile the HIP library; returns its path.  Raises on a compile error."""
    generate(verbose)
    out = PKG_DIR / LIB_NAME
    tmp = out.with_name(out.name + f".tmp{os.getpid()}")
    cmd = [hipcc(), *HIP_FLAGS, f"-I{REPO_DIR / 'include'}", "-o", str(tmp), *map(str, SOURCES), *LIBS]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only feature flag; drop that
    # one harmless warning and show everything else.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    log = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{log}")
    if verbose and log.strip():
        print(log, flush=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose=True)
    print(f"built {path}", file=sys.stderr)
