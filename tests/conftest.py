"""Shared fixtures.  Tests marked ``gpu`` need an MI355X; the rest run on CPU."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
for p in (str(ROOT), str(GOLDEN)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


@pytest.fixture(scope="session")
def sidon():
    """The package (loads the HIP library; raises if it was not built)."""
    from __graft_entry__ import load_package

    pkg = load_package()
    pkg._lib.load()
    return pkg


@pytest.fixture(scope="session")
def golden_cases():
    from make_golden import load_case

    return {p.stem: load_case(p) for p in sorted(GOLDEN.glob("hf_*.npz"))}


def seeded_inputs(batch, heads, length, seed, dtype=np.float16, scale=1.0, rel_std=0.02):
    """q, k, v ~ N(0, 1) * scale and rel ~ N(0, rel_std), one generator per role."""
    import torch

    def gen(role):
        return torch.Generator().manual_seed(seed * 16 + role)

    shape = (batch, heads, length, 64)
    q = torch.randn(shape, generator=gen(0)) * scale
    k = torch.randn(shape, generator=gen(1)) * scale
    v = torch.randn(shape, generator=gen(2)) * scale
    rel = torch.randn(73, 64, generator=gen(3)) * rel_std
    if dtype == np.float16:
        q, k, v, rel = (t.half() for t in (q, k, v, rel))
    return q, k, v, rel
