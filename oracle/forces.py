"""Oracle: conservative energy, forces and virial of the UMA path via torch autograd (CPU).

Test infrastructure only (see ``oracle/__init__.py``).  Follows ``tt_atom/forces.py:501-613`` of
the reference: a strain leaf applied to the edge vectors as ``r' = r + r @ sym(strain)``, the host
geometry, the backbone and the energy head, then ``torch.autograd.grad`` to positions (and to
the strain for the virial).  ``calculator.py:155-165`` then scales by the energy normalizer and
divides the virial by the cell volume.
"""
from __future__ import annotations

import torch

from . import uma
from .geometry import HostGeometry


class Model:
    """Weights + fixed buffers of one bundle (the ``.npz`` layout of weights.py:19-136)."""

    def __init__(self, w, cfg, bufs, gamma=0.0):
        self.w, self.cfg, self.bufs, self.gamma = w, cfg, bufs, gamma
        self.geo = HostGeometry(w, cfg, bufs["to_m"], bufs["gauss_offset"], bufs["gauss_coeff"],
                                gamma=gamma)
        self.to_grid = bufs.get("to_grid_mat")
        self.from_grid = bufs.get("from_grid_mat")

    def to(self, dtype):
        """Copy of the model in another float dtype (fp64 for finite-difference checks)."""
        def cast(d):
            return {k: (v.to(dtype) if torch.is_tensor(v) and torch.is_floating_point(v) else v)
                    for k, v in d.items()}
        return Model(cast(self.w), self.cfg, cast(self.bufs), self.gamma)


def forward_energy(model, pos, Z, edge_index, sys_emb, edge_cell_shift=None, strain=None):
    """Energy (scalar tensor) as a differentiable function of pos (and strain)."""
    edge_vec = None
    if strain is not None:
        src, tgt = edge_index[0], edge_index[1]
        ev = pos[src] - pos[tgt]
        if edge_cell_shift is not None:
            ev = ev + edge_cell_shift
        sym = 0.5 * (strain + strain.transpose(0, 1))
        edge_vec = ev + ev @ sym                                  # forces.py:516-524
    t = model.geo(pos, Z, edge_index, sys_emb, edge_vec=edge_vec, edge_cell_shift=edge_cell_shift)
    ne = uma.backbone(model.w, model.cfg, t["x_init"], t["wigner"], t["wigner_inv"], t["x_edge"],
                      t["edge_envelope"], sys_emb, edge_index, model.to_grid, model.from_grid)
    return uma.energy(ne, model.w), ne, t


def energy_and_forces(model, pos, Z, edge_index, sys_emb, edge_cell_shift=None,
                      compute_stress=False):
    """Returns (E float, F [N,3]) or (E, F, virial [3,3]) -- forces.py:592-613."""
    pos = pos.detach().clone().requires_grad_(True)
    strain = None
    if compute_stress:
        strain = torch.zeros(3, 3, dtype=pos.dtype, requires_grad=True)
    E, _, _ = forward_energy(model, pos, Z, edge_index, sys_emb, edge_cell_shift, strain)
    inputs = [pos] if strain is None else [pos, strain]
    grads = torch.autograd.grad(E, inputs)
    if strain is None:
        return float(E.detach()), -grads[0]
    return float(E.detach()), -grads[0], grads[1]
