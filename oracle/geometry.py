"""Oracle: host geometry of the UMA path (neighbour list, Wigner-D, x_edge, envelope, node init).

Test infrastructure only (see ``oracle/__init__.py``).  A torch-CPU restatement of
``tt_atom/geometry.py`` of the reference; the same fp32 torch operations in the same order so the
neighbour list and every geometric term agree with the reference CPU path.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

EPS = 1e-7  # geometry.py:20


def csd_embedding(w, charge, spin, dataset="omat"):
    """System embedding [nsys, C]; geometry.py:23-45 (rand_emb and pos_emb encodings)."""
    if "charge_embedding.rand_emb.weight" in w:
        chg = F.embedding(charge.long() + 100, w["charge_embedding.rand_emb.weight"])
        sp = F.embedding(spin.long(), w["spin_embedding.rand_emb.weight"])
    else:
        def enc(x, W, is_spin):
            xp = x[:, None] * W[None, :] * 2 * math.pi
            emb = torch.cat([torch.sin(xp), torch.cos(xp)], dim=-1)
            if is_spin:
                emb = emb.clone()
                emb[torch.where(x == 0)[0]] = 0
            return emb
        chg = enc(charge, w["charge_embedding.W"], False)
        sp = enc(spin, w["spin_embedding.W"], True)
    ds = w[f"dataset_embedding.dataset_emb_dict.{dataset}.weight"][0].expand(charge.shape[0], -1)
    return F.silu(F.linear(torch.cat([chg, sp, ds], dim=1), w["mix_csd.weight"], w["mix_csd.bias"]))


def radius_graph(pos, cutoff, cell=None, pbc=None):
    """Brute-force neighbour list; geometry.py:48-81.

    Aperiodic: ``d = ||pos_i - pos_j||``, keep ``0 < d < cutoff``, order src-major
    (``torch.where`` over [src, tgt]).  Periodic: image cells ``ceil(cutoff * ||b_k||)`` per
    axis, keep ``1e-8 < d^2 <= cutoff^2``, order (tgt, src, cell), ``edge_index = [src, tgt]``.
    Returns ``(edge_index [2,E] int64, cell_shift [E,3], cell_id [E] int64)``; ``cell_id`` is the
    index of the image cell in the cartesian-product order (0 when aperiodic) and is only used by
    the max-neighbour cap below."""
    periodic = cell is not None and pbc is not None and bool(torch.as_tensor(pbc).any())
    if not periodic:
        d = torch.linalg.norm(pos[:, None, :] - pos[None, :, :], dim=-1)
        mask = (d < cutoff) & (d > 0)
        src, tgt = torch.where(mask)
        E = int(mask.sum())
        return torch.stack([src, tgt], 0), pos.new_zeros(E, 3), torch.zeros(E, dtype=torch.long)
    cell = torch.as_tensor(cell, dtype=pos.dtype).reshape(3, 3)
    pbc = torch.as_tensor(pbc, dtype=torch.bool).reshape(-1).expand(3)
    recip = torch.linalg.inv(cell).transpose(0, 1)
    reps = [int(math.ceil(float(cutoff * torch.linalg.norm(recip[k])))) if bool(pbc[k]) else 0
            for k in range(3)]
    ranges = [torch.arange(-r, r + 1, dtype=pos.dtype) for r in reps]
    cells = torch.cartesian_prod(*ranges).reshape(-1, 3)
    shifts = cells @ cell
    disp = pos[:, None, None, :] - (pos[None, :, None, :] + shifts[None, None, :, :])
    d2 = (disp ** 2).sum(-1)
    mask = (d2 <= cutoff * cutoff) & (d2 > 1e-8)
    i, j, c = torch.where(mask)
    return torch.stack([j, i], 0), shifts[c], c


def cap_neighbors(pos, edge_index, cell_shift, max_neighbors):
    """Max-neighbour cap (builder decision D3; the reference has no cap for UMA).

    Per receiver (tgt) keep the ``max_neighbors`` nearest sources, ordered by
    ``(d2, src, cell)`` ascending where ``d2 = sum((pos[src] - pos[tgt] + shift)^2)`` in fp32;
    then emit the surviving edges in the reference order of the uncapped graph.  Because the
    uncapped order within a receiver is already (src, cell) ascending, a stable sort on d2
    within each receiver realises the tie-break.  Returns a bool keep-mask over the edges."""
    E = edge_index.shape[1]
    keep = torch.zeros(E, dtype=torch.bool)
    if E == 0:
        return keep
    src, tgt = edge_index[0], edge_index[1]
    ev = pos[src] - pos[tgt] + cell_shift
    d2 = (ev[:, 0] * ev[:, 0] + ev[:, 1] * ev[:, 1]) + ev[:, 2] * ev[:, 2]
    order_t = torch.argsort(tgt, stable=True)                 # group by receiver, keep edge order
    d2_t = d2[order_t]
    tg = tgt[order_t]
    # stable sort by d2 inside each receiver group: sort by (tgt, d2) lexicographically
    o2 = torch.argsort(d2_t, stable=True)
    o3 = torch.argsort(tg[o2], stable=True)
    ranked = order_t[o2[o3]]                                  # edges grouped by tgt, d2-ascending
    tg_r = tgt[ranked]
    counts = torch.bincount(tg_r, minlength=int(pos.shape[0]))
    starts = torch.cumsum(counts, 0) - counts
    rank = torch.arange(E) - starts[tg_r]
    keep[ranked[rank < max_neighbors]] = True
    return keep


def neighbor_list(pos, cutoff, cell=None, pbc=None, max_neighbors=None):
    """radius_graph followed by the optional cap; returns (edge_index, cell_shift)."""
    ei, shift, _ = radius_graph(pos, cutoff, cell, pbc)
    if max_neighbors is not None:
        keep = cap_neighbors(pos, ei, shift, max_neighbors)
        ei, shift = ei[:, keep], shift[keep]
    return ei, shift


class SafeAcos(torch.autograd.Function):
    """acos with the regularised gradient of geometry.py:87-96."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x.clamp(-1 + EPS, 1 - EPS))
        return torch.acos(x)

    @staticmethod
    def backward(ctx, g):
        (xc,) = ctx.saved_tensors
        return -g / torch.sqrt(1 - xc.pow(2)).clamp(min=EPS)


class SafeAtan2(torch.autograd.Function):
    """atan2 with the regularised gradient of geometry.py:99-109."""

    @staticmethod
    def forward(ctx, y, x):
        ctx.save_for_backward(y, x)
        return torch.atan2(y, x)

    @staticmethod
    def backward(ctx, g):
        y, x = ctx.saved_tensors
        denom = (x.pow(2) + y.pow(2)).clamp(min=EPS)
        return g * x / denom, -g * y / denom


def euler_angles(edge_vec, gamma_val=0.0):
    """geometry.py:112-118: returns the (alpha, beta, gamma) triple fed to the Wigner build."""
    xyz = F.normalize(edge_vec).clamp(-1.0, 1.0)
    x, y, z = torch.split(xyz, 1, dim=1)
    beta = SafeAcos.apply(y.squeeze(-1))
    alpha = SafeAtan2.apply(x.squeeze(-1), z.squeeze(-1))
    gamma = torch.full_like(alpha, gamma_val)
    return -gamma, -beta, -alpha


def z_rot_mat(angle, lv):
    """geometry.py:124-136: cos on the diagonal, sin on the anti-diagonal, freqs l..-l."""
    freqs = torch.arange(lv, -lv - 1, -1, dtype=angle.dtype)
    fa = freqs * angle[..., None]
    return torch.diag_embed(torch.cos(fa)) + torch.diag_embed(torch.sin(fa)).flip(-1)


def wigner_D(lv, alpha, beta, gamma, Jd):
    """geometry.py:139-142: D_l = Z(alpha) J Z(beta) J Z(gamma)."""
    alpha, beta, gamma = torch.broadcast_tensors(alpha, beta, gamma)
    J = Jd[lv]
    return z_rot_mat(alpha, lv) @ J @ z_rot_mat(beta, lv) @ J @ z_rot_mat(gamma, lv)


def eulers_to_wigner(eulers, lmax, Jd):
    """geometry.py:145-155: block-diagonal [E, nsph, nsph]."""
    alpha, beta, gamma = eulers
    size = (lmax + 1) ** 2
    wig = torch.zeros(len(alpha), size, size, dtype=alpha.dtype)
    start = 0
    for lv in range(lmax + 1):
        blk = wigner_D(lv, alpha, beta, gamma, Jd)
        end = start + blk.shape[1]
        wig[:, start:end, start:end] = blk
        start = end
    return wig


def radial_mlp(x, w, p):
    """geometry.py:161-168 / mirror.py:21-28."""
    x = F.linear(x, w[f"{p}.net.0.weight"], w[f"{p}.net.0.bias"])
    x = F.layer_norm(x, (x.shape[-1],), w[f"{p}.net.1.weight"], w[f"{p}.net.1.bias"], 1e-5)
    x = F.silu(x)
    x = F.linear(x, w[f"{p}.net.3.weight"], w[f"{p}.net.3.bias"])
    x = F.layer_norm(x, (x.shape[-1],), w[f"{p}.net.4.weight"], w[f"{p}.net.4.bias"], 1e-5)
    x = F.silu(x)
    return F.linear(x, w[f"{p}.net.6.weight"], w[f"{p}.net.6.bias"])


class HostGeometry:
    """geometry.py:174-280 (mmax == lmax, permutation ``to_m``; the uma-s case)."""

    def __init__(self, w, cfg, to_m, gauss_offset, gauss_coeff, gamma=0.0):
        self.w, self.cfg = w, cfg
        self.lmax = cfg["lmax"]
        self.C = cfg["sphere_channels"]
        self.cutoff = cfg["cutoff"]
        self.gamma = gamma
        self.Jd = [w[f"Jd_{l}"] for l in range(self.lmax + 1)]
        tm = torch.as_tensor(to_m)
        self.perm = tm.abs().argmax(dim=1).long()                 # geometry.py:186-193
        self.offset = gauss_offset
        self.coeff = float(gauss_coeff.reshape(-1)[0])
        p = 5.0                                                   # geometry.py:202-207
        self.env_a = -(p + 1) * (p + 2) / 2
        self.env_b = p * (p + 2)
        self.env_c = -p * (p + 1) / 2
        self.env_p = p
        self.rescale = 5.0

    def wigner(self, edge_vec):
        """geometry.py:209-224 (permutation branch)."""
        wig = eulers_to_wigner(euler_angles(edge_vec, self.gamma), self.lmax, self.Jd)
        wig_inv = torch.transpose(wig, 1, 2).contiguous()
        return wig.index_select(1, self.perm), wig_inv.index_select(2, self.perm)

    def __call__(self, pos, Z, edge_index, sys_node_embedding, edge_vec=None,
                 edge_cell_shift=None):
        """geometry.py:226-280 (host edge-degree branch)."""
        w, C, lmax = self.w, self.C, self.lmax
        src, tgt = edge_index[0], edge_index[1]
        if edge_vec is None:
            edge_vec = pos[src] - pos[tgt]
            if edge_cell_shift is not None:
                edge_vec = edge_vec + edge_cell_shift
        dist = torch.linalg.norm(edge_vec, dim=1)
        wig_M, wig_M_inv = self.wigner(edge_vec)
        gauss = torch.exp(self.coeff * (dist.view(-1, 1) - self.offset.view(1, -1)) ** 2)
        se = F.embedding(Z[src], w["source_embedding.weight"])
        te = F.embedding(Z[tgt], w["target_embedding.weight"])
        x_edge = torch.cat([gauss, se, te], dim=1)
        ds = dist / self.cutoff
        env_val = 1 + (ds ** self.env_p) * (self.env_a + ds * (self.env_b + self.env_c * ds))
        envelope = torch.where(ds < 1, env_val, torch.zeros_like(env_val)).reshape(-1, 1, 1)
        N = Z.shape[0]
        nsph = (lmax + 1) ** 2
        l0 = F.embedding(Z, w["sphere_embedding.weight"]) + sys_node_embedding
        l0 = F.pad(l0.unsqueeze(1), (0, 0, 0, nsph - 1))
        edm = radial_mlp(x_edge, w, "edge_degree_embedding.rad_func").reshape(-1, lmax + 1, C)
        edm = F.pad(edm, (0, 0, 0, nsph - (lmax + 1)))
        edm = torch.bmm(wig_M_inv, edm) * envelope
        node = torch.zeros(N, nsph, C, dtype=pos.dtype)
        node = node.index_add(0, tgt, edm / self.rescale)
        return dict(x_init=node + l0, l0=l0, wigner=wig_M, wigner_inv=wig_M_inv, x_edge=x_edge,
                    edge_envelope=envelope, edge_distance=dist, edge_distance_vec=edge_vec)
