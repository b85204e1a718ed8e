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

from . import _native as nat
from . import orb as _orb
from .engine_cache import cached_engine

__all__ = ["energy_and_forces", "energy_and_forces_batch", "rmsnorm_bw", "mlpnorm_bw",
           "attn_layer_bw", "energy_bw", "energy_bw_batch", "backbone_bw", "backbone_bw_batch"]


# ----------------------------------------------------------------------------- per-module reverse
# The VJPs of the modules called one by one (orb_forces.py:67-254), over the activations the
# modules' __call__ kept; the same kernels as the engine's reverse pass, launched per module.
def _empty(*shape, like):
    return torch.empty(*shape, device=like.device, dtype=torch.float32)


def rmsnorm_bw(norm, g_out):
    """Adjoint of ``RMSNorm.__call__``'s input (orb_forces.py:67-79)."""
    x, inv = norm._cache_x, norm._cache_inv
    g = g_out.to(device=x.device, dtype=torch.float32).contiguous()
    g_x = torch.empty_like(x)
    nat.rms_bwd(g, x, norm.w, inv, g_x)
    return g_x


def mlpnorm_bw(mlp, g_out):
    """Adjoint of ``MLPNorm.__call__``'s input (orb_forces.py:82-91): the RMSNorm adjoint, then
    each linear's transpose with the SiLU derivative of the kept pre-activation in its epilogue."""
    p = mlp._p
    g_h2 = rmsnorm_bw(mlp.norm, g_out)
    R = g_h2.shape[0]
    g_a1 = _empty(R, p.hidden, like=g_h2)
    g_a0 = _empty(R, p.hidden, like=g_h2)
    nat.linear(g_h2, p.w[2], out=g_a1, epilogue=nat.EPI_SILU_GRAD, aux=mlp._cache_a1)
    nat.linear(g_a1, p.w[1], out=g_a0, epilogue=nat.EPI_SILU_GRAD, aux=mlp._cache_a0)
    return nat.linear(g_a0, p.w[0])


def attn_layer_bw(layer, graph, g_nodes_out, g_edges_out):
    """Adjoints (nodes, edges, cutoff [E, 1]) of ``AttentionInteractionLayer.__call__``'s inputs
    from those of its outputs (orb_forces.py:94-148), edges in the graph's edge order."""
    c, p, C = layer._cache, layer._p, layer.C
    t = graph._module_topology()
    N, E, H = graph.N, graph.E, p.edge.hidden
    dev = t.send.device
    g_n = g_nodes_out.to(device=dev, dtype=torch.float32).clone()
    g_e = g_edges_out.to(device=dev, dtype=torch.float32)[t.order].contiguous()
    g_cut = torch.zeros(E, device=dev, dtype=torch.float32)
    Hn = p.node.hidden
    g_hn2, g_an1, g_an0 = _empty(N, C, like=g_n), _empty(N, Hn, like=g_n), _empty(N, Hn, like=g_n)
    nat.rms_bwd(g_n, c["hn2"], p.node.norm, c["ninv"], g_hn2)
    nat.linear(g_hn2, p.node.w[2], out=g_an1, epilogue=nat.EPI_SILU_GRAD, aux=c["an1"])
    nat.linear(g_an1, p.node.w[1], out=g_an0, epilogue=nat.EPI_SILU_GRAD, aux=c["an0"])
    g_node_in = nat.linear(g_an0, p.node.w[0])                          # [N, 3C]
    g_h2 = _empty(E, C, like=g_n)
    nat.orb_edge_bwd(g_e, g_node_in, c["ue"], c["sig"], t.cut, c["h2"], c["inv"], p.edge.norm,
                     p.attn_w, t.send, t.recv, g_h2, g_cut)
    g_a1, g_a0 = _empty(E, H, like=g_n), _empty(E, H, like=g_n)
    nat.linear(g_h2, p.edge.w[2], out=g_a1, epilogue=nat.EPI_SILU_GRAD, aux=c["a1"])
    nat.linear(g_a1, p.edge.w[1], out=g_a0, epilogue=nat.EPI_SILU_GRAD, aux=c["a0"])
    G = _empty(N, 2 * H, like=g_n)
    nat.orb_node_segsum2(g_a0, t.send_ptr, t.recv_ptr, t.recv_perm, G)
    nat.add_rows(g_node_in[:, :C], g_n)
    nat.linear_group([(g_a0, p.we, None, g_e, nat.EPI_ACCUM),
                      (G, p.wsr, None, g_n, nat.EPI_ACCUM)])
    return g_n, g_e[t.inv_order], g_cut[t.inv_order].reshape(E, 1)


def energy_bw(ehead):
    """Adjoint [N, C] of ``EnergyHead.__call__``'s node features for dE/dE = 1
    (orb_forces.py:151-172): every row is the mean's adjoint over N."""
    p = ehead._p
    a0, N = ehead._cache_a0, ehead._cache_N
    ones = torch.ones(1, 1, device=a0.device, dtype=torch.float32)
    g_a0 = _empty(1, p.hidden, like=a0)
    nat.linear(ones, p.w[1], out=g_a0, epilogue=nat.EPI_SILU_GRAD, aux=a0)
    g_mean = nat.linear(g_a0, p.w[0])                                   # [1, C]
    out = _empty(N, g_mean.shape[1], like=a0)
    nat.segment_mean_bwd(g_mean, torch.zeros(N, dtype=torch.int32, device=a0.device),
                         torch.tensor([0, N], dtype=torch.int32, device=a0.device), out)
    return out


def energy_bw_batch(ehead, seg_mean_T):
    """Adjoint [N, C] of ``EnergyHead.batch``'s node features for the summed energies, with
    ``seg_mean_T`` [N, K] the transposed row-normalised segment matrix (orb_forces.py:207-229)."""
    p = ehead._p
    a0 = ehead._cache_a0
    K = a0.shape[0]
    ones = torch.ones(K, 1, device=a0.device, dtype=torch.float32)
    g_a0 = _empty(K, p.hidden, like=a0)
    nat.linear(ones, p.w[1], out=g_a0, epilogue=nat.EPI_SILU_GRAD, aux=a0)
    g_mean = nat.linear(g_a0, p.w[0])                                   # [K, C]
    smt = seg_mean_T.to(device=a0.device, dtype=torch.float32).contiguous()
    return nat.linear(smt, g_mean)


def _backbone_bw(encoder, layers, g_nodes, graph):
    g_edges = torch.zeros(graph.E, layers[0].C if layers else encoder.latent_dim,
                          device=g_nodes.device, dtype=torch.float32)
    g_cutoff = None
    for layer in reversed(layers):
        g_nodes, g_edges, g_c = attn_layer_bw(layer, graph, g_nodes, g_edges)
        g_cutoff = g_c if g_cutoff is None else g_cutoff + g_c
    return mlpnorm_bw(encoder.edge_fn, g_edges), g_cutoff


def backbone_bw(encoder, layers, ehead, graph, e_true=None):
    """Reverse pass from the energy head through every layer to the encoder's edge input:
    (adjoint of the edge features, adjoint of the cutoff) (orb_forces.py:175-204).  ``e_true``
    (the reference's bucketed edge count) must be None or the true count: graphs are not padded
    here."""
    if e_true is not None and int(e_true) != graph.E:
        raise ValueError("padded (bucketed) graphs are not used by this build")
    return _backbone_bw(encoder, layers, energy_bw(ehead), graph)


def backbone_bw_batch(encoder, layers, ehead, graph, seg_mean_T):
    """``backbone_bw`` for a disjoint-union batch (orb_forces.py:232-254)."""
    return _backbone_bw(encoder, layers, energy_bw_batch(ehead, seg_mean_T), graph)


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
