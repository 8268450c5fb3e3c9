"""HIP-graph capture of the attention sequence per length bucket (needs an MI355X).

Each bucket's graph is replayed several times with the program's own eager
work and synchronisations between the replays; every replay must equal the
eager result bit for bit.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def make_stack(batch, heads, max_len, layers, seed):
    gen = torch.Generator().manual_seed(seed)
    qkv = [torch.randn(batch * max_len, 3 * heads * 64, generator=gen).half().to(DEV) for _ in range(layers)]
    rel = [(torch.randn(73, 64, generator=gen) * 0.02).half().to(DEV) for _ in range(layers)]
    out = [torch.empty(batch * max_len, heads * 64, dtype=torch.float16, device=DEV) for _ in range(layers)]
    lens = torch.zeros(batch, dtype=torch.int32, device=DEV)
    return qkv, rel, out, lens


def test_graph_per_bucket_replays_match_eager(sidon):
    B, H, layers = 1, 16, 8
    max_len = 1250
    qkv, rel, out, lens = make_stack(B, H, max_len, layers, seed=5)
    graphs = sidon.graphs.BucketGraphs(max_graphs=4)

    def enqueue(length):
        rows = B * length
        for i in range(layers):
            sidon.encoder_attention.flexrel_attention(
                qkv[i][:rows], B, H, rel[i], lens, out=out[i][:rows])

    for length, valid in ((100, 93), (1250, 1250), (650, 601), (100, 57)):
        rows = B * length
        lens.fill_(valid)
        enqueue(length)
        torch.cuda.synchronize()
        eager = [o[:rows].clone() for o in out]
        for rep in range(3):
            for o in out:
                o.zero_()
            lens.fill_(valid)
            graphs.run(length, lambda: enqueue(length))
            torch.cuda.synchronize()
            for i in range(layers):
                assert torch.equal(out[i][:rows], eager[i]), (length, rep, i)
            _ = (qkv[0][:rows].float() * 2).sum().item()  # unrelated eager work
    assert len(graphs) == 3


def test_graph_keeps_the_tensors_its_work_reads_alive(sidon):
    """Tensors referenced only by the captured callable (here: the tables
    and inputs, made inside a helper and never returned) must outlive the
    capture: later allocations of the same sizes, filled with garbage, must
    not change what a replay computes.  The result is checked against the
    float64 oracle, not against another run of the same path."""
    import numpy as np

    from oracle.flexrel_oracle import errors, flexrel_reference

    H, L, lk = 4, 200, 162
    gen = torch.Generator().manual_seed(31)
    q_host = torch.randn(L, 3 * H * 64, generator=gen).half()
    rel_host = (torch.randn(73, 64, generator=gen) * 0.02).half()
    out = torch.empty(L, H * 64, dtype=torch.float16, device=DEV)
    lens = torch.full((1,), lk, dtype=torch.int32, device=DEV)
    graphs = sidon.graphs.BucketGraphs()

    def capture():
        qkv, rel = q_host.to(DEV), rel_host.to(DEV)  # held only by the closure

        def enqueue():
            sidon.encoder_attention.flexrel_attention(qkv, 1, H, rel, lens, out=out)
        graphs.capture("only-closure", enqueue)

    capture()
    junk = [torch.full((n,), float("nan"), dtype=torch.float16, device=DEV)
            for n in (73 * 64, L * 3 * H * 64) for _ in range(8)]
    out.fill_(float("nan"))
    graphs.run("only-closure", lambda: None)
    torch.cuda.synchronize()
    v = q_host.view(1, L, 3, H, 64).float()
    q, k, vv = (v[:, :, i].permute(0, 2, 1, 3).numpy() for i in range(3))
    ref = flexrel_reference(q, k, vv, rel_host.float().numpy(), [lk])
    got = out.view(1, L, H, 64).permute(0, 2, 1, 3).float().cpu().numpy()
    err = errors(ref[:, :, :lk], got[:, :, :lk])
    assert np.isfinite(got).all() and err["snr_db"] >= 60.0 and err["max_abs"] <= 2e-3, err
    del junk
