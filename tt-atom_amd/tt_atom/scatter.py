"""Per-op entry points of the reference's scatter module (scatter.py:35-89): the fixed-width
gather table of an edge -> node sum and the sum itself, over fp32 torch tensors on the device
(csrc/pattern.hip, tta_segment_sum_table).

``build_gather`` writes the reference's table format: row n of ``[N, Dmax]`` lists, in edge
order, the edges whose node is n, and the padding slots hold a sentinel (the index of the zero
row the reference appends to the messages).  ``segment_sum`` takes the reference's arguments; its
``ttnn`` argument is accepted and not used, and a sentinel (any index outside the message rows)
adds nothing instead of reading an appended zero row.  The fused step (tt_atom.trace) sums over
destination CSR offsets instead (tta_rotate_env_segsum, tta_node_gather_sum), which needs no
padding.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _native as nat

__all__ = ["build_gather", "segment_sum"]


def build_gather(idx: torch.Tensor, num_nodes: int, E: int, sentinel=None, min_width: int = 0):
    """``idx`` ``[E]`` (each edge's node) -> (``gather_flat`` ``[num_nodes * Dmax]`` int32, ``Dmax``)
    with Dmax = max(largest degree, ``min_width``) (1 for an empty graph) and the padding slots
    set to ``sentinel`` (default ``E``) (scatter.py:35-59)."""
    nodes = np.asarray(idx.detach().cpu() if isinstance(idx, torch.Tensor) else idx,
                       dtype=np.int64).reshape(-1)[:E]
    if nodes.size and (nodes.min() < 0 or nodes.max() >= num_nodes):
        raise ValueError("build_gather: node index out of range")
    deg = np.bincount(nodes, minlength=num_nodes)
    width = max(int(deg.max()) if nodes.size else 1, int(min_width))
    table = np.full((num_nodes, width), E if sentinel is None else sentinel, dtype=np.int64)
    edges = np.argsort(nodes, kind="stable")          # edge ids grouped by node, in edge order
    first = np.concatenate([[0], np.cumsum(deg)[:-1]])
    sorted_nodes = nodes[edges]
    table[sorted_nodes, np.arange(nodes.size) - first[sorted_nodes]] = edges
    return table.reshape(-1).astype(np.int32), width


def segment_sum(ttnn, msg, gather_dev, Dmax, N, W):
    """``msg`` ``[E, W]`` -> ``[N, W]``: row n sums the message rows the table lists for node n,
    in table order (scatter.py:62-89).  ``gather_dev``: the ``[N * Dmax]`` table (any integer
    tensor or array; moved to the messages' device as int32)."""
    if msg.dim() != 2 or msg.shape[1] != W:
        raise RuntimeError(f"segment_sum: msg must be [E, {W}], got {tuple(msg.shape)}")
    g = torch.as_tensor(gather_dev)
    if g.numel() != N * Dmax:
        raise RuntimeError(f"segment_sum: the table has {g.numel()} entries, expected {N * Dmax}")
    g = g.to(device=msg.device, dtype=torch.int32).contiguous()
    out = torch.empty(N, W, device=msg.device, dtype=torch.float32)
    nat.segment_sum_table(msg.contiguous(), g, out, N=N, Dmax=Dmax, W=W)
    return out
