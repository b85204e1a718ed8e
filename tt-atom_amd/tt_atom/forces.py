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


def energy_and_forces_batch(bb, geo, bg, *, compute_forces=True):
    """Disjoint-union batch (forces.py:616-637): one step over the block-diagonal graph ``bg``
    (``disjoint.BatchedGraph``); raw per-system energies [K] from per-system node sums and the
    forces of the one shared reverse pass (block-diagonal, so each atom's own system's force)."""
    eng = TracedEngine(bb, geo, bg.Z, bg.edge_index, bg.sys_emb, edge_cell_shift=bg.cell_shift,
                       use_graph=False)
    eng.run(bg.pos)
    E = eng.segment_energies(bg.natoms).cpu()
    F = eng.forces.detach().cpu().clone() if compute_forces else None
    return E, F
