"""One captured HIP graph per length bucket, replayed on the current stream.

Mirrors the bucketed graph execution of src/sidon_triton/runtime.py:374-401:
the first call for a key warms the work up on a side stream, then captures it
into a ``torch.cuda.CUDAGraph`` that draws from one memory pool shared by all
graphs (only one graph replays at a time); later calls replay it.  At most
``max_graphs`` graphs are kept (least recently used evicted), as runtime.py's
LRU of 128.

The attention entry points are capture-safe: they launch on the current
stream, allocate nothing inside the library and never read device data on the
host, so a whole sequence of layers is one graph per bucket.

A graph holds raw device addresses of every tensor its work touched.  Each
graph is therefore kept together with the ``enqueue`` callable it was
captured from: whatever that callable references (its tensors, directly or
through a closure) stays alive exactly as long as the graph, and is never
freed and reused under a later replay.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Callable, Hashable

import torch


class BucketGraphs:
    def __init__(self, max_graphs: int = 128):
        self.max_graphs = max_graphs
        self._graphs: OrderedDict = OrderedDict()
        self._pool = None

    def __len__(self) -> int:
        return len(self._graphs)

    def capture(self, key: Hashable, enqueue: Callable[[], None]) -> torch.cuda.CUDAGraph:
        entry = self._graphs.get(key)
        if entry is not None:
            self._graphs.move_to_end(key)
            return entry[0]
        current = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(current)
        with torch.cuda.stream(side):
            enqueue()
        current.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        if self._pool is None:
            self._pool = torch.cuda.graph_pool_handle()
        with torch.cuda.graph(graph, pool=self._pool):
            enqueue()
        self._graphs[key] = (graph, enqueue)
        while len(self._graphs) > self.max_graphs:
            self._graphs.popitem(last=False)
        return graph

    def run(self, key: Hashable, enqueue: Callable[[], None]) -> None:
        """Replay the graph of ``key`` (capturing ``enqueue`` the first time)."""
        self.capture(key, enqueue).replay()
