"""Disjoint-union batching of independent systems (reference disjoint.py:123-218).

``assemble`` builds the block-diagonal eSCN-MD graph of K systems: each system's neighbour list
on its own, edges offset by the running node count, per-node system embeddings from each
system's charge / spin.  ``assemble_orb`` (Orb's convention) lives in ``tt_atom.orb`` and is
re-exported here under the reference's module path."""
from __future__ import annotations

import numpy as np
import torch

from .geometry import csd_embedding, system_graphs
from .orb import OrbBatchedGraph, _fields, assemble_orb

__all__ = ["BatchedGraph", "assemble", "assemble_orb", "OrbBatchedGraph"]


class BatchedGraph:
    """Block-diagonal union of K systems (disjoint.py:49-120)."""

    def __init__(self, pos, Z, edge_index, cell_shift, batch, natoms, sys_emb):
        self.pos, self.Z, self.edge_index, self.cell_shift = pos, Z, edge_index, cell_shift
        self.batch, self.natoms, self.sys_emb = batch, list(natoms), sys_emb

    @property
    def K(self):
        return len(self.natoms)

    def segment_matrix(self):
        """[K, Ntot] one-hot system membership (disjoint.py:109-120)."""
        seg = torch.zeros(self.K, self.pos.shape[0])
        seg[self.batch, torch.arange(self.pos.shape[0])] = 1.0
        return seg


def assemble(systems, cutoff, weights, sphere_channels, task="omol", max_neighbors=None,
             neighbor_list="host"):
    """K systems (ASE Atoms, dicts or (pos, Z[, cell, pbc]) tuples) -> ``BatchedGraph``; raises
    if a system has no edge within ``cutoff``.  ``max_neighbors`` applies the per-receiver cap;
    ``neighbor_list="device"`` builds the same graphs on the GPU."""
    if len(systems) == 0:
        raise ValueError("empty batch")
    fields = []
    for system in systems:
        pos, Z, cell, pbc, charge, spin = _fields(system)
        fields.append((torch.as_tensor(np.asarray(pos), dtype=torch.float32),
                       torch.as_tensor(np.asarray(Z), dtype=torch.int64), cell, pbc,
                       float(charge), float(spin)))
    graphs = system_graphs([(f[0], f[2], f[3]) for f in fields], cutoff, max_neighbors,
                           neighbor_list)
    pos_all, Z_all, ei_all, sh_all, b_all, se_all, natoms = ([] for _ in range(7))
    off = 0
    for k, (pos, Z, cell, pbc, charge, spin) in enumerate(fields):
        ei, shift = graphs[k]
        if ei.shape[1] == 0:
            raise ValueError(f"system {k} has no edges within cutoff -- too sparse for this model")
        n = Z.shape[0]
        pos_all.append(pos)
        Z_all.append(Z)
        ei_all.append(ei + off)
        sh_all.append(shift.float())
        b_all.append(torch.full((n,), k, dtype=torch.long))
        se = csd_embedding(weights, torch.tensor([charge]), torch.tensor([spin]),
                           sphere_channels, dataset=task)
        se_all.append(se.expand(n, -1))
        natoms.append(n)
        off += n
    return BatchedGraph(torch.cat(pos_all), torch.cat(Z_all), torch.cat(ei_all, 1),
                        torch.cat(sh_all), torch.cat(b_all), natoms, torch.cat(se_all))
