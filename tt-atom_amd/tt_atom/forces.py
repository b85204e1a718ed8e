"""Conservative energy + analytic forces (+ virial) for one system (reference forces.py:592-613).

``energy_and_forces(bb, geo, pos, atomic_numbers, edge_index, sys_node_embedding,
edge_cell_shift=None, compute_stress=False)`` keeps the reference signature and return values:
``(E, F)`` or ``(E, F, virial)`` with ``virial = dE/dstrain`` (the caller divides by the cell
volume for the stress).  The whole pass -- geometry, backbone, reverse pass, geometric VJP --
runs on the GPU (``trace.TracedEngine``); this one-shot form builds the engine for the given
topology and runs it once."""
from __future__ import annotations

from .trace import TracedEngine


def energy_and_forces(bb, geo, pos, atomic_numbers, edge_index, sys_node_embedding,
                      edge_cell_shift=None, compute_stress=False):
    # one step per engine: launched eagerly (a graph pays off from the second step on)
    eng = TracedEngine(bb, geo, atomic_numbers, edge_index, sys_node_embedding,
                       edge_cell_shift=edge_cell_shift, use_graph=False)
    return eng(pos, compute_stress=compute_stress)
