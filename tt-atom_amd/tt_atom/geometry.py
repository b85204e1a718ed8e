"""Geometry front end: neighbour list, system embedding and the device-side geometric constants.

``radius_graph`` restates the reference's brute-force neighbour list (tt_atom/geometry.py:48-81)
with the same fp32 comparisons and edge order, plus the optional per-receiver max-neighbour cap
(builder decision D3).  It runs on the host once per topology, as in the reference.
``HostGeometry`` keeps the reference class name and constructor (geometry.py:174-207) but holds
the device constants of the per-step geometry kernels (Wigner ``Jd`` blocks, gaussian basis,
envelope cutoff); the per-edge terms are computed on the GPU by the step engine.
"""
from __future__ import annotations

import math

import numpy as np

import torch
import torch.nn.functional as F

from .model import TO_M_PERM, _UNSUPPORTED


def csd_embedding(w, charge, spin, sphere_channels=None, dataset="omat"):
    """System (charge / spin / dataset) embedding -> [nsys, C] (geometry.py:23-45)."""
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
        chg = enc(charge.float(), w["charge_embedding.W"], False)
        sp = enc(spin.float(), w["spin_embedding.W"], True)
    ds = w[f"dataset_embedding.dataset_emb_dict.{dataset}.weight"][0].expand(charge.shape[0], -1)
    return F.silu(F.linear(torch.cat([chg, sp, ds], dim=1), w["mix_csd.weight"], w["mix_csd.bias"]))


def radius_graph(pos, cutoff, cell=None, pbc=None, max_neighbors=None):
    """Neighbour list ``(edge_index [2,E] int64, cell_shift [E,3])`` on the host.

    Aperiodic: keep ``0 < |pos_i - pos_j| < cutoff``, src-major order.  Periodic: image cells
    ``ceil(cutoff * |b_k|)`` per periodic axis, keep ``1e-8 < d^2 <= cutoff^2``, order
    (tgt, src, cell), ``edge_vec = pos[src] - pos[tgt] + cell_shift``.  With ``max_neighbors``
    each receiver keeps its nearest sources by ``(d^2, src, cell)`` and the surviving edges keep
    the uncapped order."""
    pos = torch.as_tensor(pos, dtype=torch.float32).cpu()
    periodic = cell is not None and pbc is not None and bool(torch.as_tensor(pbc).any())
    if not periodic:
        d = torch.linalg.norm(pos[:, None, :] - pos[None, :, :], dim=-1)
        mask = (d < cutoff) & (d > 0)
        src, tgt = torch.where(mask)
        ei = torch.stack([src, tgt], 0)
        shift = pos.new_zeros(ei.shape[1], 3)
    else:
        cell = torch.as_tensor(cell, dtype=pos.dtype).reshape(3, 3)
        pbc = torch.as_tensor(pbc, dtype=torch.bool).reshape(-1).expand(3)
        recip = torch.linalg.inv(cell).transpose(0, 1)
        reps = [int(math.ceil(float(cutoff * torch.linalg.norm(recip[k])))) if bool(pbc[k]) else 0
                for k in range(3)]
        cells = torch.cartesian_prod(*[torch.arange(-r, r + 1, dtype=pos.dtype) for r in reps])
        shifts = cells.reshape(-1, 3) @ cell
        ei_parts, sh_parts = [], []
        # receivers in chunks keep the [chunk, N, cells] displacement tensor bounded
        chunk = max(1, int(2e7 // max(1, pos.shape[0] * shifts.shape[0])))
        for i0 in range(0, pos.shape[0], chunk):
            p = pos[i0:i0 + chunk]
            disp = p[:, None, None, :] - (pos[None, :, None, :] + shifts[None, None, :, :])
            d2 = (disp ** 2).sum(-1)
            mask = (d2 <= cutoff * cutoff) & (d2 > 1e-8)
            i, j, c = torch.where(mask)
            ei_parts.append(torch.stack([j, i + i0], 0))
            sh_parts.append(shifts[c])
        ei = torch.cat(ei_parts, 1)
        shift = torch.cat(sh_parts, 0)
    if max_neighbors is not None and ei.shape[1]:
        keep = _cap(pos, ei, shift, int(max_neighbors))
        ei, shift = ei[:, keep], shift[keep]
    return ei, shift


def _image_shifts(pos, cutoff, cell, pbc):
    """Cartesian image shifts of the periodic branch (reference geometry.py:70-77)."""
    cell = torch.as_tensor(cell, dtype=pos.dtype).reshape(3, 3)
    pbc = torch.as_tensor(pbc, dtype=torch.bool).reshape(-1).expand(3)
    recip = torch.linalg.inv(cell).transpose(0, 1)
    reps = [int(math.ceil(float(cutoff * torch.linalg.norm(recip[k])))) if bool(pbc[k]) else 0
            for k in range(3)]
    cells = torch.cartesian_prod(*[torch.arange(-r, r + 1, dtype=pos.dtype) for r in reps])
    return cells.reshape(-1, 3) @ cell


# Systems of at least this many atoms take the cell list when the method is "auto"; below it the
# row scan (every row reads all N candidates; fewer launches and no binning) is as fast or faster
# on MI355X.  Measured whole calls at a 6 A cutoff: an aperiodic 2k-atom cluster 0.18 ms (rows)
# against 0.30 ms (cells), 8k atoms 0.46 against 0.37 ms; a 2k-atom periodic crystal 0.65 against
# 0.45 ms (the row scan visits every image of every atom).
CELL_LIST_MIN_ATOMS_APERIODIC = 4096
CELL_LIST_MIN_ATOMS_PERIODIC = 2048


def use_cell_list(n_atoms, periodic):
    """Does method "auto" take the cell list for one system of ``n_atoms``?"""
    return n_atoms >= (CELL_LIST_MIN_ATOMS_PERIODIC if periodic else CELL_LIST_MIN_ATOMS_APERIODIC)


def cell_grid(pos, cutoff, max_bins=None):
    """Bins of the cell-list neighbour search over the atoms ``pos`` [N, 3]: ``(origin [3] fp32,
    inv_h fp32, dims [3])`` with bin coordinate ``u = fl(fl(x - origin) * inv_h)`` per axis.

    The bin side ``h = 1 / inv_h`` exceeds the cutoff by a margin above every rounding error of
    the fp32 distance test and of u itself (2^-10 of the cutoff plus 2^-12 of the box extent;
    both errors are below 2^-20 relative), so any pair that passes the distance test lies in
    neighbouring bins on every axis.  The origin sits 1.5 bins below the atoms' bounding box and
    ``dims`` spans it plus 2.5 bins above, so every atom's bin and its neighbours are on the
    grid.  At most ``max_bins`` (default max(4096, 2 N)) bins: a sparse system gets wider
    bins."""
    p = np.asarray(pos, np.float32).reshape(-1, 3)
    n = p.shape[0]
    q = np.ascontiguousarray(p.T)                  # per-axis rows: fast reductions
    mn = np.fmin.reduce(q, axis=1).astype(np.float64) if n else np.zeros(3)
    mx = np.fmax.reduce(q, axis=1).astype(np.float64) if n else np.zeros(3)
    if not (np.isfinite(mn).all() and np.isfinite(mx).all()):
        # infinite or all-NaN coordinates: the box of the finite atoms (the others have no edge)
        fin = p[np.isfinite(p).all(1)].astype(np.float64)
        mn = fin.min(0) if fin.shape[0] else np.zeros(3)
        mx = fin.max(0) if fin.shape[0] else np.zeros(3)
    ext = mx - mn
    cap = int(max_bins) if max_bins is not None else max(4096, 2 * n)
    h = float(cutoff) * (1.0 + 2.0 ** -10) + float(ext.max()) * 2.0 ** -12
    while True:
        dims = np.floor(ext / h).astype(np.int64) + 4
        if int(np.prod(dims)) <= cap:
            break
        h *= 1.25
    inv_h = np.float32(1.0 / (h * (1.0 + 2.0 ** -20)))     # fp32 rounding keeps 1 / inv_h >= h
    origin = (mn - 1.5 * h).astype(np.float32)
    return tuple(float(v) for v in origin), float(inv_h), tuple(int(v) for v in dims)


def radius_graph_device(pos, cutoff, cell=None, pbc=None, max_neighbors=None, *,
                        node_ranges=None, device=None, method="auto"):
    """``radius_graph`` computed on the GPU: the same edges in the same order with the same
    ``cell_shift`` values (device tensors).  ``node_ranges`` ([N] lo, [N] hi) restricts every
    node's candidates to its own system in a batch of disjoint aperiodic systems (the
    concatenation of the per-system graphs, node indices global).  ``method``: "rows" scans
    every candidate of a row (O(N^2)), "cells" bins the atoms (and periodic images) and scans the
    27 bins around each one (O(N), one system: no ``node_ranges``), "auto" takes the cell list
    for one system as large as ``use_cell_list`` asks.  Both give the same graph."""
    if method not in ("auto", "rows", "cells"):
        raise ValueError("method must be 'auto', 'rows' or 'cells'")
    if method == "cells" and node_ranges is not None:
        raise ValueError("the cell list builds one system; batches with node_ranges use 'rows'")
    dev = torch.device(device) if device is not None else (
        pos.device if torch.is_tensor(pos) and pos.is_cuda else torch.device("cuda"))
    pos_h = torch.as_tensor(pos, dtype=torch.float32).detach().cpu()
    N = pos_h.shape[0]
    periodic = cell is not None and pbc is not None and bool(torch.as_tensor(pbc).any())
    if periodic and node_ranges is not None:
        raise ValueError("node_ranges applies to aperiodic batches only")
    if node_ranges is not None:
        # the kernels read pos[lo .. hi) of every row unchecked: bound the ranges on the host
        lo_h = torch.as_tensor(node_ranges[0]).detach().cpu().reshape(-1).long()
        hi_h = torch.as_tensor(node_ranges[1]).detach().cpu().reshape(-1).long()
        if lo_h.numel() != N or hi_h.numel() != N:
            raise ValueError(f"node_ranges need {N} lo and {N} hi entries, got "
                             f"{lo_h.numel()} and {hi_h.numel()}")
        if N and not bool(((lo_h >= 0) & (lo_h <= hi_h) & (hi_h <= N)).all()):
            raise ValueError("node_ranges must satisfy 0 <= lo <= hi <= N for every node")
    mid2, cut2, min2 = 0.0, 0.0, 0.0
    if periodic:
        shifts = _image_shifts(pos_h, cutoff, cell, pbc)
        cut2 = float(np.float32(cutoff * cutoff))      # the fp32 of the host's d2 <= cutoff^2
        min2 = float(np.float32(1e-8))
    else:
        shifts = pos_h.new_zeros(1, 3)
        # d < fp32(cutoff) with d = fp32 sqrt(s)  <=>  s < m^2, m the midpoint below fp32(cutoff)
        c32 = np.float32(cutoff)
        m = (float(np.nextafter(c32, np.float32(-np.inf))) + float(c32)) / 2.0
        mid2 = m * m
    lo = hi = None
    if node_ranges is not None:
        lo = torch.as_tensor(node_ranges[0]).to(dev, torch.int32).contiguous()
        hi = torch.as_tensor(node_ranges[1]).to(dev, torch.int32).contiguous()
    from . import _native as nat
    k = int(max_neighbors) if max_neighbors is not None else 0
    sh_d = shifts.to(dev).contiguous()
    cells = method == "cells" or (method == "auto" and node_ranges is None
                                  and use_cell_list(N, periodic)
                                  and (not periodic or N * shifts.shape[0] < (1 << 30)))
    if cells:
        src, tgt, c = nat.radius_graph_cells(pos_h.to(dev).contiguous(), sh_d, periodic,
                                             cell_grid(pos_h.numpy(), cutoff), mid2, cut2, min2,
                                             k)
    else:
        src, tgt, c = nat.radius_graph_passes(pos_h.to(dev).contiguous(), lo, hi, sh_d,
                                              periodic, mid2, cut2, min2, k)
    ei = torch.stack([src, tgt], 0)
    shift = sh_d[c.long()] if periodic else torch.zeros(src.shape[0], 3, device=dev)
    return ei, shift


def _periodic_batch_device(items, cutoff, max_neighbors):
    """One batched device pass for periodic systems [(pos, cell, pbc)]: node ranges keep every
    receiver's candidates in its system and per-row ranges into the concatenated image-shift
    tables give it its own system's images, so each system's edges, order, cells and cap are those
    of ``radius_graph_device`` on it alone.  Returns [(edge_index, cell_shift)] on the host, each
    in its system's own node numbering."""
    from . import _native as nat
    pos_l, sh_l = [], []
    for pos, cell, pbc in items:
        p = torch.as_tensor(pos, dtype=torch.float32).detach().cpu()
        pos_l.append(p)
        sh_l.append(_image_shifts(p, cutoff, cell, pbc))
    sizes = np.asarray([p.shape[0] for p in pos_l], np.int64)
    nsh = np.asarray([s.shape[0] for s in sh_l], np.int64)
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    cst = np.concatenate([[0], np.cumsum(nsh)[:-1]]).astype(np.int64)
    lo, hi = np.repeat(starts, sizes), np.repeat(starts + sizes, sizes)
    clo, chi = np.repeat(cst, sizes), np.repeat(cst + nsh, sizes)
    N, n_cells = int(sizes.sum()), int(nsh.sum())
    # the kernels index pos[lo..hi) and shifts[clo..chi) unchecked: bound them here
    if N == 0 or not (lo.min() >= 0 and hi.max() <= N and clo.min() >= 0 and chi.max() <= n_cells
                      and n_cells < (1 << 20)):
        raise ValueError("periodic batch: empty or out-of-range node / image ranges")
    dev = torch.device("cuda")
    i32 = lambda a: torch.from_numpy(a.astype(np.int32)).to(dev)
    shifts = torch.cat(sh_l).to(torch.float32)
    sh_d = shifts.to(dev).contiguous()
    k = int(max_neighbors) if max_neighbors is not None else 0
    src, tgt, c = nat.radius_graph_passes(
        torch.cat(pos_l).to(dev).contiguous(), i32(lo), i32(hi), sh_d, True, 0.0,
        float(np.float32(cutoff * cutoff)), float(np.float32(1e-8)), k, i32(clo), i32(chi))
    src, tgt, c = src.cpu(), tgt.cpu(), c.cpu().long()
    # periodic rows are receivers: edges come grouped by system in order
    bounds = np.searchsorted(tgt.numpy(), np.concatenate([starts, [N]]))
    out = []
    for q in range(len(items)):
        a, b = int(bounds[q]), int(bounds[q + 1])
        ei = torch.stack([src[a:b], tgt[a:b]], 0) - int(starts[q])
        out.append((ei, shifts[c[a:b]]))
    return out


def system_graphs(systems, cutoff, max_neighbors=None, neighbor_list="host"):
    """Per-system neighbour lists of a disjoint batch: ``systems`` = [(pos [n,3], cell or None,
    pbc or None)], result [(edge_index [2,E_k] int64, cell_shift [E_k,3])] on the host, each in
    its system's own node numbering.  ``neighbor_list="device"`` builds all aperiodic systems in
    one batched GPU pass and all periodic ones in another; the graphs are identical to the
    host's."""
    if neighbor_list not in ("host", "device"):
        raise ValueError("neighbor_list must be 'host' or 'device'")
    out = [None] * len(systems)
    periodic = [c is not None and p is not None and bool(np.asarray(p).any())
                for (_, c, p) in systems]
    if neighbor_list == "device":
        # large systems one at a time through the cell list, the rest in batched row scans
        for k, (pos, cell, pbc) in enumerate(systems):
            if use_cell_list(int(np.asarray(pos).reshape(-1, 3).shape[0]), periodic[k]):
                ei, sh = radius_graph_device(torch.as_tensor(np.asarray(pos), dtype=torch.float32),
                                             cutoff, cell if periodic[k] else None,
                                             pbc if periodic[k] else None, max_neighbors,
                                             method="cells")
                out[k] = (ei.cpu(), sh.cpu())
        ap = [k for k in range(len(systems)) if not periodic[k] and out[k] is None]
        if ap:
            sizes = [int(systems[k][0].shape[0]) for k in ap]
            starts = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
            lo = np.repeat(starts, sizes)
            hi = np.repeat(starts + np.asarray(sizes, np.int64), sizes)
            ei, _ = radius_graph_device(
                torch.cat([torch.as_tensor(systems[k][0], dtype=torch.float32) for k in ap]),
                cutoff, max_neighbors=max_neighbors,
                node_ranges=(torch.from_numpy(lo), torch.from_numpy(hi)))
            ei = ei.cpu()
            bounds = np.searchsorted(ei[0].numpy(), np.concatenate([starts, [lo.size]]))
            for q, k in enumerate(ap):
                part = ei[:, bounds[q]:bounds[q + 1]] - int(starts[q])
                out[k] = (part, torch.zeros(part.shape[1], 3))
        per = [k for k in range(len(systems)) if periodic[k] and out[k] is None]
        if per:
            for k, g in zip(per, _periodic_batch_device([systems[k] for k in per], cutoff,
                                                        max_neighbors)):
                out[k] = g
    for k, (pos, cell, pbc) in enumerate(systems):
        if out[k] is None:
            out[k] = radius_graph(pos, cutoff, cell, pbc if periodic[k] else None, max_neighbors)
    return out


def _cap(pos, ei, shift, k):
    src, tgt = ei[0], ei[1]
    ev = pos[src] - pos[tgt] + shift
    d2 = (ev[:, 0] * ev[:, 0] + ev[:, 1] * ev[:, 1]) + ev[:, 2] * ev[:, 2]
    E = ei.shape[1]
    by_tgt = torch.argsort(tgt, stable=True)
    o2 = torch.argsort(d2[by_tgt], stable=True)
    o3 = torch.argsort(tgt[by_tgt][o2], stable=True)
    ranked = by_tgt[o2[o3]]
    counts = torch.bincount(tgt[ranked], minlength=int(pos.shape[0]))
    starts = torch.cumsum(counts, 0) - counts
    rank = torch.arange(E) - starts[tgt[ranked]]
    keep = torch.zeros(E, dtype=torch.bool)
    keep[ranked[rank < k]] = True
    return keep


class HostGeometry:
    """Geometric constants of the step (reference geometry.py:174-207 constructor)."""

    def __init__(self, weights, cfg, to_m, gauss_offset, gauss_coeff, *, gamma=0.0,
                 coefficient_index=None, device="cuda"):
        self.lmax = cfg["lmax"]
        self.mmax = cfg.get("mmax", self.lmax)
        if self.lmax != 2 or self.mmax != 2 or coefficient_index is not None:
            raise RuntimeError(_UNSUPPORTED.format(what=f"lmax={self.lmax}, mmax={self.mmax}"))
        tm = torch.as_tensor(to_m).float()
        perm = tuple(int(v) for v in tm.abs().argmax(dim=1).tolist())
        is_perm = bool(((tm == 0) | (tm == 1)).all()) and bool(((tm != 0).sum(1) == 1).all())
        if not is_perm or perm != TO_M_PERM:
            raise RuntimeError(_UNSUPPORTED.format(what=f"to_m permutation {perm}"))
        self.C = cfg["sphere_channels"]
        self.cutoff = float(cfg["cutoff"])
        self.gamma = float(gamma)
        dev = torch.device(device)
        jd = torch.cat([weights[f"Jd_{l}"].reshape(-1).float() for l in range(3)])
        if jd.numel() != 35:
            raise RuntimeError("Jd blocks must be 1x1, 3x3, 5x5")
        self.jd = jd.to(dev).contiguous()
        self.offset = torch.as_tensor(gauss_offset).float().reshape(-1).to(dev).contiguous()
        self.coeff = float(torch.as_tensor(gauss_coeff).reshape(-1)[0])
        self.n_gauss = self.offset.numel()
        self.rescale = float(cfg.get("edge_degree_rescale", 5.0))
