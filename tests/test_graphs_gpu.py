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
