"""GPU parity of every attention kernel variant, not only the automatic
choice (needs an MI355X).

`SIDON_FLEXREL_VARIANT` (read by the library at every call) forces the
8-split kernel of flexrel_fwd.hip, the 64-row kernel of flexrel_w64.hip or
the 32-row kernel of flexrel_w32.hip; K and V rows of
different strides take the 8-split kernel
without being forced.  Each is checked against the float64 oracle at the
north-star bar on ragged and padded shapes, for the same results contract:
keys past the valid length (refilled with finite garbage, which sends the
loop's overflow check into its rerun) leave the valid rows bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import seeded_inputs
from oracle.flexrel_oracle import flexrel_reference
from test_flexrel_gpu import DEV, assert_parity, run

pytestmark = pytest.mark.gpu

VARIANTS = ["split8", "w64", "w32"]
SHAPES = [
    # (B, H, L, lens)
    (1, 2, 33, [20]),
    (1, 3, 127, [127]),
    (2, 2, 200, [200, 173]),
    (3, 2, 300, [300, 64, 129]),
    (1, 4, 513, [513]),
    (1, 16, 750, None),
]


@pytest.fixture
def variant(request, monkeypatch):
    monkeypatch.setenv("SIDON_FLEXREL_VARIANT", request.param)
    return request.param


@pytest.mark.parametrize("variant", VARIANTS, indirect=True)
@pytest.mark.parametrize("B,H,L,lens", SHAPES)
def test_variant_parity(sidon, variant, B, H, L, lens):
    q, k, v, rel = seeded_inputs(B, H, L, seed=1000 + L)
    got = run(sidon, q, k, v, rel, lens).float().cpu().numpy()
    lk = lens if lens is not None else [L] * B
    ref = np.zeros_like(got, dtype=np.float64)
    for b in range(B):
        if lk[b]:
            ref[b:b + 1, :, :lk[b]] = flexrel_reference(q.numpy()[b:b + 1, :, :lk[b]], k.numpy()[b:b + 1, :, :lk[b]],
                                                        v.numpy()[b:b + 1, :, :lk[b]], rel.numpy())
    assert_parity(ref, got, lk, f"{variant} B={B} H={H} L={L}")


@pytest.mark.parametrize("variant", VARIANTS, indirect=True)
def test_variant_padding_garbage_bit_identical(sidon, variant):
    """c2's bucket: L=1500, LK=1463; rows past LK refilled with +-60000."""
    L, LK = 1500, 1463
    q, k, v, rel = seeded_inputs(1, 16, L, seed=2)
    k[:, :, LK:] = 0
    v[:, :, LK:] = 0
    got = run(sidon, q, k, v, rel, [LK])
    ref = flexrel_reference(q.numpy()[:, :, :LK], k.numpy()[:, :, :LK], v.numpy()[:, :, :LK], rel.numpy())
    assert_parity(ref, got.float().cpu().numpy()[:, :, :LK], [LK], f"{variant} c2")
    gen = torch.Generator().manual_seed(22)
    k2, v2, q2 = k.clone(), v.clone(), q.clone()
    for t in (k2, v2, q2):
        t[:, :, LK:] = ((torch.rand(t[:, :, LK:].shape, generator=gen) * 2 - 1) * 60000).half()
    got2 = run(sidon, q2, k2, v2, rel, [LK])
    assert torch.equal(got[:, :, :LK], got2[:, :, :LK]), f"{variant}: keys past LK changed valid rows"


@pytest.mark.parametrize("variant", ["w64", "w32"], indirect=True)
def test_variant_c3_shape(sidon, variant):
    """L=4800, H=16: the grids of several rounds; 2 heads checked."""
    q, k, v, rel = seeded_inputs(1, 16, 4800, seed=3)
    got = run(sidon, q, k, v, rel).float().cpu().numpy()
    assert np.isfinite(got).all()
    heads = [0, 15]
    ref = flexrel_reference(q.numpy()[:, heads], k.numpy()[:, heads], v.numpy()[:, heads], rel.numpy())
    assert_parity(ref, got[:, heads], [4800], f"{variant} c3")


_FUSED_L3000 = {}


def _fused_l3000():
    """A 60 s chunk in the encoder's fused QKV layout: [L, 3 * 16 * 64] rows
    of unit-variance values, L = 3000 (the last key step straddles the
    length); the float64 oracle of all 16 heads, computed once."""
    if not _FUSED_L3000:
        L, H = 3000, 16
        gen = torch.Generator().manual_seed(L)
        qkv = torch.randn(L, 3 * H * 64, generator=gen).half()
        rel = (torch.randn(73, 64, generator=gen) * 0.02).half()
        x = qkv.view(L, 3, H, 64).permute(1, 2, 0, 3).numpy()  # [q|k|v, H, L, 64]
        ref = flexrel_reference(x[0][None], x[1][None], x[2][None], rel.numpy())[0]  # [H, L, 64]
        _FUSED_L3000.update(qkv=qkv, rel=rel, ref=ref, L=L, H=H)
    return _FUSED_L3000


@pytest.mark.parametrize("variant", ["w64", "w32"], indirect=True)
def test_variant_fused_layout_l3000(sidon, variant):
    c = _fused_l3000()
    L, H = c["L"], c["H"]
    lens = torch.tensor([L], dtype=torch.int32, device=DEV)
    out = sidon.encoder_attention.flexrel_attention(c["qkv"].to(DEV), 1, H, c["rel"].to(DEV), lens)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(L, H, 64).transpose(1, 0, 2)[None]
    assert_parity(c["ref"][None], got, [L], f"{variant} fused L=3000")


@pytest.mark.parametrize("variant", ["w64", "w32"], indirect=True)
def test_variant_repeated_launches_bit_identical(sidon, variant):
    """200 launches on the same inputs give the same bits.  Regression test:
    the hand-scheduled loops once returned with their last V^T operand reads
    still in flight, and the compiled PV products after the loop (moved by
    the compiler above the wait meant for them) read stale operands now and
    then -- one 32-row block's dims 0-31 wrong in ~3% of launches at
    L = 2990, never at 1500 or 4800."""
    L, H = 2990, 16
    gen = torch.Generator().manual_seed(L)
    qkv = torch.randn(L, 3 * H * 64, generator=gen).half().to(DEV)
    rel = (torch.randn(73, 64, generator=gen) * 0.02).half().to(DEV)
    lens = torch.tensor([L], dtype=torch.int32, device=DEV)
    out = torch.empty(L, H * 64, dtype=torch.float16, device=DEV)
    first = sidon.encoder_attention.flexrel_attention(qkv, 1, H, rel, lens).clone()
    bad = 0
    for _ in range(200):
        sidon.encoder_attention.flexrel_attention(qkv, 1, H, rel, lens, out=out)
        bad += int(not torch.equal(out, first))
    torch.cuda.synchronize()
    assert bad == 0, f"{variant}: {bad} of 200 launches differ from the first"


def test_different_kv_strides_take_the_8_split_kernel(sidon, monkeypatch):
    """K and V views of different row strides (V a slice of a wider buffer):
    the automatic choice falls back to the 8-split kernel; same results
    as contiguous copies of the same values."""
    monkeypatch.delenv("SIDON_FLEXREL_VARIANT", raising=False)
    B, H, L = 1, 4, 300
    q, k, v, rel = seeded_inputs(B, H, L, seed=61)
    wide = torch.zeros(B, H, L, 128, dtype=torch.float16)
    wide[..., 32:96] = v
    v_view = wide.to(DEV)[..., 32:96]          # row stride 128 elements, K's is 64
    out = sidon.flexrel.flexrel_attention(q.to(DEV), k.to(DEV), v_view, rel.to(DEV))
    torch.cuda.synchronize()
    ref = flexrel_reference(q.numpy(), k.numpy(), v.numpy(), rel.numpy())
    assert_parity(ref, out.float().cpu().numpy(), [L], "kv-strides")
    monkeypatch.setenv("SIDON_FLEXREL_VARIANT", "split8")
    out8 = run(sidon, q, k, v, rel)
    assert torch.equal(out, out8)


RERUN_SHAPES = [
    # (B, H, L, lens): plain, band, straddling and first-step paths; one 64-row
    # workgroup per CU and two; wavefronts with no step (L < 4 x 32)
    (1, 2, 33, [20]),
    (2, 2, 200, [200, 173]),
    (3, 2, 300, [300, 64, 129]),
    (2, 16, 600, [600, 517]),
    (1, 16, 1500, [1463]),
    (1, 16, 2990, None),
    (1, 16, 4800, None),
]


@pytest.mark.parametrize("B,H,L,lens", RERUN_SHAPES)
def test_w64_loop_matches_its_general_code_bit_for_bit(sidon, monkeypatch, B, H, L, lens):
    """The 64-row kernel's hand-scheduled key-step loop -- its plain steps and
    the scheduled block of every special-step path -- against the kernel's
    compiled general code, which a wavefront reruns when a probability leaves
    the fp16 range: with every wavefront forced onto that rerun
    (sidon_flexrel_debug_rerun_all), every output element, padded rows
    included, is bit-identical to the loop's."""
    monkeypatch.setenv("SIDON_FLEXREL_VARIANT", "w64")
    q, k, v, rel = seeded_inputs(B, H, L, seed=3000 + L)
    lib = sidon._lib.load()
    loop = run(sidon, q, k, v, rel, lens).cpu()
    lib.sidon_flexrel_debug_rerun_all(1)
    try:
        general = run(sidon, q, k, v, rel, lens).cpu()
    finally:
        lib.sidon_flexrel_debug_rerun_all(0)
    assert torch.equal(loop, general), int((loop != general).sum())


def test_rerun_hook_takes_the_general_code(sidon, monkeypatch):
    """The hook is live: with every wavefront on the compiled general code the
    c3 layer takes several times as long as the hand-scheduled loop (so the
    bit-identity above compares two different code paths)."""
    monkeypatch.setenv("SIDON_FLEXREL_VARIANT", "w64")
    L, H = 4800, 16
    gen = torch.Generator().manual_seed(L)
    qkv = torch.randn(L, 3 * H * 64, generator=gen).half().to(DEV)
    rel = (torch.randn(73, 64, generator=gen) * 0.02).half().to(DEV)
    lens = torch.tensor([L], dtype=torch.int32, device=DEV)
    out = torch.empty(L, H * 64, dtype=torch.float16, device=DEV)
    lib = sidon._lib.load()

    def ms():
        for _ in range(3):
            sidon.encoder_attention.flexrel_attention(qkv, 1, H, rel, lens, out=out)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            sidon.encoder_attention.flexrel_attention(qkv, 1, H, rel, lens, out=out)
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / 10

    fast = ms()
    lib.sidon_flexrel_debug_rerun_all(1)
    try:
        slow = ms()
    finally:
        lib.sidon_flexrel_debug_rerun_all(0)
    print(f"c3 layer: loop {fast:.3f} ms, every wavefront rerun {slow:.3f} ms", flush=True)
    assert slow > 1.5 * fast
