"""Orb-v3 conservative energy + forces under the reference's signatures (orb_forces.py:257-378).

``energy_and_forces(encoder, layers, ehead, device, *, pos, senders, receivers, atomic_numbers,
node_feat, ...)`` and ``energy_and_forces_batch(..., seg_mean, seg_mean_T, ...)`` take the module
objects of ``tt_atom.orb_model`` (built with the reference's constructors) and return what the
reference returns: the raw (normalised-space) energy -- a float, or a [K] fp64 tensor for a
batch -- and ``F = -dE/dpos`` [N, 3] (plus the raw virial dE/dstrain [3, 3] with
``compute_stress``).  The reference runs a ttnn forward, a ttnn reverse pass over cached
activations and a host ``torch.autograd`` finish through the edge geometry; here the modules are
assembled into one ``tt_atom.orb.OrbEngine`` step whose forward, analytic backward, edge-geometry
VJP and force / virial reductions are all HIP kernels on the GPU.

``bucketing`` / ``max_num_neighbors`` only shape the reference's compiled programs (the result
is the same); the kernels here take any edge count, so they are accepted and have no effect.
"""
from __future__ import annotations

import torch

from . import orb as _orb
from .engine_cache import cached_engine

__all__ = ["energy_and_forces", "energy_and_forces_batch"]


def _model(encoder, layers, ehead, device, r_max, num_bases):
    """The OrbModel view of the modules, built once per (modules, r_max, num_bases) and kept on
    the energy head."""
    key = (id(encoder), tuple(id(l) for l in layers), float(r_max), int(num_bases), str(device))
    cache = ehead.__dict__.setdefault("_orb_models", {})
    if key in cache:
        return cache[key][0]
    precs = {encoder.precision} | {l.precision for l in layers}
    if len(precs) != 1:
        raise ValueError(f"encoder and layers must share one precision, got {sorted(precs)}")
    if encoder.edge_in != 16 * int(num_bases):
        raise ValueError(f"encoder edge input is {encoder.edge_in}, expected 16 * num_bases = "
                         f"{16 * int(num_bases)}")
    cfg = {"latent_dim": encoder.latent_dim, "num_bases": int(num_bases), "cutoff": float(r_max)}
    dev = torch.device("cuda") if device is None or str(device) in ("", "None") \
        else torch.device(device)
    m = _orb.OrbModel.from_parts((encoder.node_fn._p, encoder.edge_fn._p),
                                 [l._p for l in layers], (ehead._p, None, None), cfg=cfg,
                                 device=dev, precision=precs.pop())
    cache[key] = (m, encoder, tuple(layers))      # the modules stay alive with their model
    return m


def _engine(m, pos, senders, receivers, atomic_numbers, node_feat, cell_shift, natoms,
            cond_nodes, slot):
    """The step engine of this topology, kept on the OrbModel between calls with the same
    senders, receivers, species, node features, cell shifts, system sizes and conditioning
    (``engine_cache``: a fixed-topology MD loop replays the captured step)."""
    N = int(torch.as_tensor(atomic_numbers).shape[0])
    cond = cond_nodes if (cond_nodes is not None and any(
        l.cond_w_t is not None for l in m.layers)) else None

    def build():
        graph = _orb.OrbGraph(m.device, senders=senders, receivers=receivers, num_nodes=N,
                              atomic_numbers=atomic_numbers, cell_shift=cell_shift,
                              natoms=natoms)
        return _orb.OrbEngine(m, graph, cond,
                              node_feat=torch.as_tensor(node_feat, dtype=torch.float32))

    key = (senders, receivers, atomic_numbers, torch.as_tensor(node_feat), cell_shift,
           None if natoms is None else tuple(int(n) for n in natoms), cond)
    eng = cached_engine(m, slot, key, build)
    p = torch.as_tensor(pos).to(m.device, torch.float32).contiguous()
    return eng, p


def energy_and_forces(encoder, layers, ehead, device, *, pos, senders, receivers,
                      atomic_numbers, node_feat, cell_shift=None, r_max=6.0, num_bases=8,
                      compute_stress=False, cond_nodes=None, bucketing=False,
                      max_num_neighbors=0):
    """One system (orb_forces.py:307-378): ``(energy_raw: float, forces [N, 3])`` and, with
    ``compute_stress``, the raw virial ``dE/dstrain`` [3, 3]; forces / virial on the host in
    ``pos``'s floating dtype."""
    m = _model(encoder, layers, ehead, device, r_max, num_bases)
    eng, p = _engine(m, pos, senders, receivers, atomic_numbers, node_feat, cell_shift, None,
                     cond_nodes, "energy_and_forces")
    raw, F, vir = eng.run(p, compute_stress)
    dt = pos.dtype if torch.is_tensor(pos) and pos.is_floating_point() else torch.float32
    out = (float(raw[0]), F.detach().to("cpu", dt))
    return out if not compute_stress else out + (vir.detach().to("cpu", dt),)


def _natoms_from_seg_mean(seg_mean, n):
    """System sizes of a row-normalised segment matrix [K, Ntot]; the systems must be contiguous
    node ranges in order (as assemble_orb builds them)."""
    sm = torch.as_tensor(seg_mean)
    if sm.dim() != 2 or sm.shape[1] != n:
        raise ValueError(f"seg_mean must be [K, {n}]")
    nz = sm != 0
    if not bool((nz.sum(0) == 1).all()):
        raise ValueError("every node must belong to exactly one system of seg_mean")
    batch = nz.to(torch.int64).argmax(0)
    if n and not bool((batch[1:] >= batch[:-1]).all()):
        raise ValueError("the systems of seg_mean must be contiguous node ranges in order")
    natoms = torch.bincount(batch, minlength=sm.shape[0]).tolist()
    if min(natoms) == 0:
        raise ValueError("seg_mean has a system without nodes")
    return natoms


def energy_and_forces_batch(encoder, layers, ehead, device, *, pos, senders, receivers,
                            atomic_numbers, node_feat, cell_shift, seg_mean, seg_mean_T,
                            r_max=6.0, num_bases=8, cond_nodes=None):
    """Disjoint-union batch (orb_forces.py:257-304): ``(energy_raw [K] fp64, forces [Ntot, 3])``;
    ``seg_mean`` [K, Ntot] is the row-normalised membership matrix (its transpose ``seg_mean_T``
    is accepted for the reference's signature)."""
    n = int(torch.as_tensor(atomic_numbers).shape[0])
    natoms = _natoms_from_seg_mean(seg_mean, n)
    if seg_mean_T is not None and tuple(torch.as_tensor(seg_mean_T).shape) != (n, len(natoms)):
        raise ValueError("seg_mean_T must be the transpose of seg_mean")
    m = _model(encoder, layers, ehead, device, r_max, num_bases)
    eng, p = _engine(m, pos, senders, receivers, atomic_numbers, node_feat, cell_shift, natoms,
                     cond_nodes, "energy_and_forces_batch")
    raw, F, _ = eng.run(p, False)
    dt = pos.dtype if torch.is_tensor(pos) and pos.is_floating_point() else torch.float32
    return raw, F.detach().to("cpu", dt)
