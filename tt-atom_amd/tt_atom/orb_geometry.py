"""Orb-v3 edge descriptor under the reference's names (orb_geometry.py:65-139).

``host_edge_features`` and ``host_edge_features_vjp`` keep the reference's signatures and
results, but the arithmetic runs in the HIP kernels of ``libttatom_hip.so``
(``tta_orb_edge_features``: Bessel(num_bases) x real SH(l <= 3) x polynomial cutoff;
``tta_orb_edge_features_bwd``: their closed-form VJP; ``tta_node_forces``: the deterministic
per-node reduction).  ``host_edge_features`` is differentiable with respect to ``pos`` and
``strain`` (a ``torch.autograd.Function`` whose backward is the VJP kernel), so a caller that
finishes forces with ``torch.autograd.grad`` as orb_forces.py:303 / 374 does keeps working.
Tensors may live on the host or on the GPU; results come back on the device of ``pos``.
"""
from __future__ import annotations

import torch

from . import _native as nat
from .orb import OrbGraph

__all__ = ["host_edge_features", "host_edge_features_vjp"]


def _device():
    nat.load()
    return torch.device("cuda", torch.cuda.current_device())


def _check_nb(num_bases):
    nb = int(num_bases)
    if nb < 1 or nb > 64 or nb & (nb - 1):
        raise ValueError("num_bases must be a power of two <= 64")
    return nb


def _node_reduce(g_vec, senders, receivers, num_nodes, dev):
    """-dE/dpos from the edge-vector adjoint g_vec (vec = pos[recv] - pos[send]): the sums over
    each node's sender and receiver edges, in a fixed order (tta_node_forces)."""
    g = OrbGraph(dev, senders=senders, receivers=receivers, num_nodes=num_nodes,
                 atomic_numbers=torch.zeros(num_nodes, dtype=torch.int64))
    forces = torch.empty(num_nodes, 3, device=dev, dtype=torch.float32)
    nat.node_forces(g_vec[g.order].contiguous(), g.recv_ptr, g.recv_perm, g.send_ptr, forces)
    return forces


class _EdgeFeatures(torch.autograd.Function):
    """(pos [N, 3], shift [E, 3] or None) -> (edge_feat [E, nb*16], cutoff [E], vectors [E, 3])
    on the GPU, with the closed-form VJP as its backward."""

    @staticmethod
    def forward(ctx, pos, shift, send, recv, r_max, nb):
        E = send.numel()
        f = lambda *s: torch.empty(*s, device=pos.device, dtype=torch.float32)
        vec, feat, cut = f(E, 3), f(E, nb * 16), f(E)
        nat.orb_edge_features(pos, send, recv, shift, r_max, nb, vec, feat, cut)
        ctx.save_for_backward(vec, send, recv)
        ctx.r_max, ctx.nb, ctx.N, ctx.has_shift = r_max, nb, pos.shape[0], shift is not None
        return feat, cut, vec

    @staticmethod
    def backward(ctx, g_feat, g_cut, g_vec_in):
        vec, send, recv = ctx.saved_tensors
        E = vec.shape[0]
        z = lambda *s: torch.zeros(*s, device=vec.device, dtype=torch.float32)
        g_feat = z(E, ctx.nb * 16) if g_feat is None else g_feat.float().contiguous()
        g_cut = z(E) if g_cut is None else g_cut.float().reshape(E).contiguous()
        g_vec = torch.empty(E, 3, device=vec.device, dtype=torch.float32)
        nat.orb_edge_features_bwd(vec, g_feat, g_cut, ctx.r_max, ctx.nb, g_vec)
        if g_vec_in is not None:
            g_vec = g_vec + g_vec_in
        g_pos = -_node_reduce(g_vec, send, recv, ctx.N, vec.device)
        return g_pos, (g_vec if ctx.has_shift else None), None, None, None, None


def host_edge_features(pos, senders, receivers, cell_shift, *, r_max=6.0, num_bases=8,
                       strain=None):
    """Differentiable ``pos -> (edge_feat [E, num_bases*16], cutoff [E, 1], vectors [E, 3])``
    (orb_geometry.py:65-97): ``vectors = pos[receivers] - pos[senders] (+ cell_shift)``, scaled
    by ``I + sym(strain)`` when a strain is given; ``edge_feat = cutoff * (rbf (x) sh)``."""
    nb = _check_nb(num_bases)
    out_dev = pos.device
    dev = _device()
    p = pos.to(dev, torch.float32)
    sh = None if cell_shift is None else torch.as_tensor(cell_shift).to(dev, torch.float32)
    if strain is not None:
        # vec (I + sym) = pos' [recv] - pos' [send] + shift' with pos' = pos (I + sym), shift'
        # likewise: the strain enters through torch ops, so autograd reaches it
        m = torch.eye(3, device=dev) + 0.5 * (strain + strain.transpose(0, 1)).to(dev, torch.float32)
        p = p @ m
        sh = None if sh is None else sh @ m
    send = torch.as_tensor(senders).to(dev, torch.int32).contiguous()
    recv = torch.as_tensor(receivers).to(dev, torch.int32).contiguous()
    n = p.shape[0]
    if send.numel() != recv.numel():
        raise ValueError("senders / receivers length mismatch")
    if send.numel() and not bool(((send >= 0) & (send < n) & (recv >= 0) & (recv < n)).all()):
        raise ValueError("edge index out of range")
    feat, cut, vec = _EdgeFeatures.apply(p.contiguous(), None if sh is None else sh.contiguous(),
                                         send, recv, float(r_max), nb)
    return feat.to(out_dev), cut.reshape(-1, 1).to(out_dev), vec.to(out_dev)


def host_edge_features_vjp(vectors, senders, receivers, num_nodes, g_edge_feat, g_cutoff, *,
                           r_max=6.0, num_bases=8):
    """Closed-form VJP of :func:`host_edge_features` returning ``-dE/dpos`` [num_nodes, 3]
    (orb_geometry.py:100-139), on the device of ``vectors``."""
    nb = _check_nb(num_bases)
    out_dev = vectors.device
    dev = _device()
    vec = vectors.to(dev, torch.float32).contiguous()
    E = vec.shape[0]
    g_feat = torch.as_tensor(g_edge_feat).to(dev, torch.float32).reshape(E, nb * 16).contiguous()
    g_cut = torch.as_tensor(g_cutoff).to(dev, torch.float32).reshape(E).contiguous()
    g_vec = torch.empty(E, 3, device=dev, dtype=torch.float32)
    nat.orb_edge_features_bwd(vec, g_feat, g_cut, float(r_max), nb, g_vec)
    forces = _node_reduce(g_vec, torch.as_tensor(senders), torch.as_tensor(receivers),
                          int(num_nodes), dev)
    return forces.to(out_dev)
