"""HIP-graph capture and replay of a fixed-topology step.

The reference records a ttnn trace of its device step once per topology and replays it per MD
step (trace.py:83-215).  The MI355X counterpart is a HIP graph: the step's kernels (all of them
launched by this package on the current stream, with preallocated buffers and no host
synchronisation, allocation or memset inside) are captured once per (engine, variant) and
replayed with one launch.  Inputs are copied into the engine's static buffers before a replay;
outputs are read from its static buffers after.
"""
from __future__ import annotations

import torch


class StepGraphs:
    """``graphs = StepGraphs(fn)``; ``graphs.run(key)`` runs ``fn(key)``: eagerly on the first
    call for that key, through a graph captured on the second, by replay afterwards.  An engine
    used once (a topology that changes every step) thus never pays for a capture."""

    def __init__(self, fn):
        self._fn = fn
        self._graphs = {}
        self._seen = set()

    def run(self, key):
        g = self._graphs.get(key)
        if g is None:
            if key not in self._seen:
                self._seen.add(key)
                self._fn(key)
                return
            torch.cuda.current_stream().synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._fn(key)
            self._graphs[key] = g
        g.replay()

    def reset(self):
        self._graphs.clear()
        self._seen.clear()
