"""The allocation-free entry point sidon_fbank_normalize_noalloc (needs an
MI355X): through the C ABI, against the workspace entry point
sidon_fbank_normalize on the same inputs, bit for bit, on two calls in a
row -- the second with fewer items and frames, so it runs on what the first
left in the static scratch -- and oversize batches are refused.  Named to be
collected last (a failure here hides no other test)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _inputs(B, F, valid, seed):
    gen = torch.Generator().manual_seed(seed)
    logmel = (torch.randn(B, F, 80, generator=gen) * 3 - 5).to(DEV)
    return logmel, torch.tensor(valid, dtype=torch.int32, device=DEV)


def test_noalloc_normalize_matches_the_workspace_entry_point(sidon):
    lib = sidon._lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    # 96 s chunks (F = 9600 frames: 64 statistics tiles) then a shorter batch
    for B, F, valid, seed in ((3, 9600, [1536000, 1234567, 400001], 1), (2, 3000, [480000, 31999], 2)):
        logmel, vt = _inputs(B, F, valid, seed)
        nbytes = lib.sidon_fbank_workspace_bytes(B, F)
        ws = torch.empty(nbytes // 4, device=DEV)
        want = torch.full((B, F, 80), float("nan"), device=DEV)
        got = torch.full((B, F, 80), float("nan"), device=DEV)
        sidon._lib.check("sidon_fbank_normalize", lib.sidon_fbank_normalize(
            logmel.data_ptr(), vt.data_ptr(), ws.data_ptr(), nbytes, want.data_ptr(), B, F, stream))
        sidon._lib.check("sidon_fbank_normalize_noalloc", lib.sidon_fbank_normalize_noalloc(
            logmel.data_ptr(), vt.data_ptr(), got.data_ptr(), B, F, stream))
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), (B, F)


def test_noalloc_normalize_captured_in_a_graph(sidon):
    """After a first eager call on the device (which resolves the static
    array's address), the noalloc call captured into a HIP graph and replayed
    on new input contents matches the workspace entry point bit for bit on
    every replay, with eager work and synchronisations between replays."""
    lib = sidon._lib.load()
    B, F = 2, 4000
    valid = [640000, 301234]
    logmel, vt = _inputs(B, F, valid, 4)
    out = torch.empty(B, F, 80, device=DEV)
    nbytes = lib.sidon_fbank_workspace_bytes(B, F)
    ws = torch.empty(nbytes // 4, device=DEV)
    want = torch.empty(B, F, 80, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # eager first call (outside capture)
        sidon._lib.check("sidon_fbank_normalize_noalloc", lib.sidon_fbank_normalize_noalloc(
            logmel.data_ptr(), vt.data_ptr(), out.data_ptr(), B, F, side.cuda_stream))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sidon._lib.check("sidon_fbank_normalize_noalloc", lib.sidon_fbank_normalize_noalloc(
            logmel.data_ptr(), vt.data_ptr(), out.data_ptr(), B, F, torch.cuda.current_stream().cuda_stream))
    for seed in (5, 6, 7):
        fresh, _ = _inputs(B, F, valid, seed)
        logmel.copy_(fresh)
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        sidon._lib.check("sidon_fbank_normalize", lib.sidon_fbank_normalize(
            logmel.data_ptr(), vt.data_ptr(), ws.data_ptr(), nbytes, want.data_ptr(), B, F,
            torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(out, want), seed


def test_noalloc_normalize_refuses_more_items_than_its_scratch(sidon):
    lib = sidon._lib.load()
    logmel, vt = _inputs(33, 64, [20000] * 33, 3)
    out = torch.empty(33, 64, 80, device=DEV)
    rc = lib.sidon_fbank_normalize_noalloc(logmel.data_ptr(), vt.data_ptr(), out.data_ptr(), 33, 64,
                                           torch.cuda.current_stream().cuda_stream)
    assert rc == -2 and "32" in lib.sidon_last_error().decode()
