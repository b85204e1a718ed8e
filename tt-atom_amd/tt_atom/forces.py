"""Conservative energy + analytic forces (+ virial) for one system (reference forces.py:592-613).

``energy_and_forces(bb, geo, pos, atomic_numbers, edge_index, sys_node_embedding,
edge_cell_shift=None, compute_stress=False)`` keeps the reference signature and return values:
``(E, F)`` or ``(E, F, virial)`` with ``virial = dE/dstrain`` (the caller divides by the cell
volume for the stress).  The whole pass -- geometry, backbone, reverse pass, geometric VJP --
runs on the GPU (``trace.TracedEngine``).  The engine of the last topology is kept on the
backbone (``engine_cache``): an MD loop that calls this function with new positions and the same
neighbour list replays the captured step instead of rebuilding the engine."""
from __future__ import annotations

from .engine_cache import cached_engine
from .trace import TracedEngine


def energy_and_forces(bb, geo, pos, atomic_numbers, edge_index, sys_node_embedding,
                      edge_cell_shift=None, compute_stress=False):
    key = (geo, atomic_numbers, edge_index, sys_node_embedding, edge_cell_shift)
    eng = cached_engine(bb, "energy_and_forces", key, lambda: TracedEngine(
        bb, geo, atomic_numbers, edge_index, sys_node_embedding,
        edge_cell_shift=edge_cell_shift))
    return eng(pos, compute_stress=compute_stress)


def energy_and_forces_batch(bb, geo, bg, *, compute_forces=True):
    """Disjoint-union batch (forces.py:616-637): one step over the block-diagonal graph ``bg``
    (``disjoint.BatchedGraph``); raw per-system energies [K] from per-system node sums and the
    forces of the one shared reverse pass (block-diagonal, so each atom's own system's force)."""
    key = (geo, bg.Z, bg.edge_index, bg.sys_emb, bg.cell_shift, tuple(bg.natoms))
    eng = cached_engine(bb, "energy_and_forces_batch", key, lambda: TracedEngine(
        bb, geo, bg.Z, bg.edge_index, bg.sys_emb, edge_cell_shift=bg.cell_shift))
    eng.run(bg.pos)
    E = eng.segment_energies(bg.natoms).cpu()
    F = eng.forces.detach().cpu().clone() if compute_forces else None
    return E, F
