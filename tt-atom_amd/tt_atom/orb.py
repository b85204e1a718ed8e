"""Orb-v3 (MoleculeGNS, conservative) energy + forces on one MI355X.

Host side of the Orb edge-MLP + scatter path: weight bundle, disjoint-union graph assembly,
device weights, and an engine that runs one position -> (energy, forces[, virial]) step as a
fixed sequence of HIP kernels from ``libttatom_hip.so``:

* edge descriptor: Bessel(8) x real SH(l<=3) x polynomial cutoff, and its closed-form VJP, on the
  device (reference: host torch, orb_geometry.py:65-139);
* encoder / interaction-layer / node MLPs: MFMA GEMMs with fused bias + SiLU epilogues;
  RMSNorm + residual + next-layer attention gates in one row kernel;
* the first edge-MLP layer on ``[e | n[send] | n[recv]]`` is evaluated as
  ``e @ W_e + (n @ W_s)[send] + (n @ W_r)[recv]`` -- the node products are node-level GEMMs and the
  gathers are an epilogue term, which removes two thirds of that edge-level GEMM and the
  ``[E, 3C]`` concat; its adjoint segment-sums ``g_a0`` to the nodes before the weight product;
* sender / receiver segment sums over sender-sorted edges (deterministic, no atomics).

Reference counterparts: orb_model.py (Encoder, AttentionInteractionLayer, EnergyHead.batch,
OrbGraphContext), orb_forces.py (mlpnorm_bw, attn_layer_bw, backbone_bw(_batch),
energy_and_forces(_batch)), disjoint.py:162-218 (assemble_orb), orb_weights.py (bundle).
"""
from __future__ import annotations

import json
import math
import pathlib

import numpy as np
import torch

from . import _native as nat
from .engine_cache import cached_engine
from .graphs import StepGraphs
from .geometry import system_graphs
from .model import PRECISIONS, _gw
from .orb_weights import OrbWeights  # noqa: F401  (re-exported: orb.OrbWeights)

HIDDEN_DIM = 1024  # the reference's fixed MLP width (orb_calculator.py:57)


# ----------------------------------------------------------------------------- weights
def save_orb_bundle(path, cfg, weights):
    out = {"config": np.frombuffer(json.dumps(cfg).encode(), dtype=np.uint8)}
    for k, v in weights.items():
        out[f"w@{k}"] = torch.as_tensor(v).detach().float().cpu().numpy()
    np.savez(pathlib.Path(path), **out)


# ----------------------------------------------------------------------------- graph
class OrbBatchedGraph:
    """Disjoint union of systems under Orb's edge convention (disjoint.py:162-218)."""

    def __init__(self, pos, Z, senders, receivers, cell_shift, batch, natoms, charges=None,
                 spins=None):
        self.pos, self.Z = pos, Z
        self.senders, self.receivers, self.cell_shift = senders, receivers, cell_shift
        self.batch, self.natoms = batch, list(natoms)
        self.charges = charges or [0.0] * len(natoms)
        self.spins = spins or [0.0] * len(natoms)

    @property
    def K(self):
        return len(self.natoms)

    def segment_matrices(self):
        """(seg, seg_mean) [K, Ntot] indicator / row-normalised (disjoint.py:109-120)."""
        K, N = self.K, self.pos.shape[0]
        seg = torch.zeros(K, N)
        seg[self.batch, torch.arange(N)] = 1.0
        return seg, seg / torch.tensor(self.natoms, dtype=seg.dtype)[:, None]


def _fields(system):
    if isinstance(system, dict):
        return (system["positions"], system["numbers"], system.get("cell"), system.get("pbc"),
                system.get("charge", 0.0), system.get("spin", 0.0))
    if hasattr(system, "get_positions"):
        info = getattr(system, "info", {}) or {}
        cell = system.get_cell() if any(system.get_pbc()) else None
        return (system.get_positions(), system.get_atomic_numbers(), cell, system.get_pbc(),
                info.get("charge", 0.0), info.get("spin", 0.0))
    pos, Z = system[0], system[1]
    cell = system[2] if len(system) > 2 else None
    pbc = system[3] if len(system) > 3 else None
    return pos, Z, cell, pbc, 0.0, 0.0


def assemble_orb(systems, r_max, max_num_neighbors, neighbor_list="host", truncate=False):
    """Block-diagonal graph of ``systems`` (ASE Atoms, dicts or (pos, Z[, cell, pbc]) tuples):
    per-system neighbour list, senders = tgt and receivers = src (Orb's convention), node
    offsets (disjoint.py:162-218).  As the reference does, a system with an atom whose sender or
    receiver degree exceeds ``max_num_neighbors`` is refused with a ValueError
    (disjoint.py:188-197).  ``truncate=True`` instead keeps, per sender, its
    ``max_num_neighbors`` nearest neighbours (ordered by (d^2, neighbour, image)), the cap rule
    of the eSCN-MD path: an explicit opt-in whose graph is not pinned against orb-models' own
    truncation (parity unpinned for capped graphs).
    ``neighbor_list="device"`` builds the same graph on the GPU (all aperiodic systems in one
    batched pass, all periodic ones in another); the result is identical edge for edge."""
    if len(systems) == 0:
        raise ValueError("empty batch")
    fields = []
    for system in systems:
        pos, Z, cell, pbc, charge, spin = _fields(system)
        fields.append((torch.as_tensor(np.asarray(pos), dtype=torch.float32),
                       torch.as_tensor(np.asarray(Z), dtype=torch.int64), cell, pbc, charge, spin))
    graphs = system_graphs([(f[0], f[2], f[3]) for f in fields], r_max,
                           max_num_neighbors if truncate else None, neighbor_list)
    if not truncate:
        for k, (ei, _) in enumerate(graphs):
            n = int(fields[k][1].shape[0])
            if ei.shape[1] == 0:
                continue
            max_deg = max(int(torch.bincount(ei[1], minlength=n).max()),
                          int(torch.bincount(ei[0], minlength=n).max()))
            if max_deg > max_num_neighbors:
                raise ValueError(
                    f"system {k} has an atom with {max_deg} neighbours within the {r_max} A "
                    f"cutoff, exceeding max_num_neighbors={max_num_neighbors}; pass "
                    "truncate=True to keep each atom's nearest max_num_neighbors instead (a "
                    "graph not pinned against orb-models' own truncation)")
    pos_all, Z_all, s_all, r_all, sh_all, b_all, natoms, q_all, s_spin = ([] for _ in range(9))
    off = 0
    for k, (pos, Z, cell, pbc, charge, spin) in enumerate(fields):
        ei, shift = graphs[k]
        if ei.shape[1] == 0:
            raise ValueError(f"system {k} has no edges within cutoff -- too sparse for this model")
        n = Z.shape[0]
        pos_all.append(pos)
        Z_all.append(Z)
        s_all.append(ei[1] + off)
        r_all.append(ei[0] + off)
        sh_all.append(shift)
        b_all.append(torch.full((n,), k, dtype=torch.long))
        natoms.append(n)
        q_all.append(float(charge))
        s_spin.append(float(spin))
        off += n
    return OrbBatchedGraph(torch.cat(pos_all), torch.cat(Z_all), torch.cat(s_all),
                           torch.cat(r_all), torch.cat(sh_all), torch.cat(b_all), natoms, q_all,
                           s_spin)


class OrbGraph:
    """Device topology of one (batched) graph (orb_model.py:269-304).  The reference edge order
    is kept at the API; internally edges are stably sorted by sender, so sender segments are
    contiguous and the receiver segments go through a permutation."""

    def __init__(self, device, *, senders, receivers, num_nodes, atomic_numbers,
                 cell_shift=None, natoms=None):
        # Sorted on the device the engine runs on (see GraphContext); one host synchronisation
        # for the checks.
        dev = torch.device(device)
        s = torch.as_tensor(senders).to(dev, torch.int64).reshape(-1)
        r = torch.as_tensor(receivers).to(dev, torch.int64).reshape(-1)
        N, E = int(num_nodes), int(s.shape[0])
        if r.shape[0] != E:
            raise ValueError("senders / receivers length mismatch")
        if N >= 2 ** 31 or E >= 2 ** 31:
            raise ValueError("graph too large for int32 indices")
        natoms = [N] if natoms is None else [int(n) for n in natoms]
        if sum(natoms) != N:
            raise ValueError("natoms do not add up to the node count")
        self.N, self.E, self.K = N, E, len(natoms)
        if E and (N == 0 or not bool(((s >= 0) & (s < N) & (r >= 0) & (r < N)).all())):
            raise ValueError("edge index out of range")
        order = torch.argsort(s, stable=True)
        self.order = order
        s_s, r_s = s[order], r[order]
        send_ptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        send_ptr[1:] = torch.cumsum(torch.bincount(s_s, minlength=N), 0)
        recv_perm = torch.argsort(r_s, stable=True)
        recv_ptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        recv_ptr[1:] = torch.cumsum(torch.bincount(r_s, minlength=N), 0)
        seg_ptr = np.zeros(self.K + 1, np.int64)
        seg_ptr[1:] = np.cumsum(natoms)
        nat_t = torch.tensor(natoms, dtype=torch.int64, device=dev)
        batch = torch.repeat_interleave(torch.arange(self.K, device=dev), nat_t, output_size=N)
        if E and bool((batch[s_s] != batch[r_s]).any()):
            raise ValueError("an edge joins two systems of the batch")
        i32 = lambda a: a.to(torch.int32).contiguous()
        self.send, self.recv = i32(s_s), i32(r_s)
        self.send_ptr, self.recv_ptr, self.recv_perm = i32(send_ptr), i32(recv_ptr), i32(recv_perm)
        self.seg_ptr = torch.from_numpy(seg_ptr.astype(np.int32)).to(dev)
        self.batch = i32(batch)
        self.natoms = natoms
        self.Z = torch.as_tensor(atomic_numbers).to(dev, torch.int64)
        self.shift = None
        if cell_shift is not None:
            sh = torch.as_tensor(cell_shift, dtype=torch.float32).to(dev)[order]
            self.shift = sh.contiguous()


# ----------------------------------------------------------------------------- device weights
def _dev(t, device):
    out = torch.empty(tuple(t.shape), dtype=torch.float32, device=device)
    out.copy_(torch.as_tensor(t, dtype=torch.float32))
    return out


class _MLPNorm:
    """One MLPNorm (orb_model.py:127-173): forward w_t [in, out] / bias, backward w [out, in],
    RMSNorm weight."""

    def __init__(self, w, prefix, device, mode=None):
        self.w_t, self.b, self.w = [], [], []
        for i in range(3):
            W = w[f"{prefix}.mlp.NN-{i}.weight"]
            self.w_t.append(_gw(W.T.contiguous(), device, mode))
            self.w.append(_gw(W, device, mode))
            self.b.append(_dev(w[f"{prefix}.mlp.NN-{i}.bias"], device))
        self.norm = _dev(w[f"{prefix}.layer_norm.weight"], device)
        self.hidden = int(self.w_t[0].shape[1])
        self.out_dim = int(self.w_t[2].shape[1])


class _Layer:
    """AttentionInteractionLayer weights (orb_model.py:203-223) with the first edge-MLP weight
    split by input block: W0 = [W_e | W_s | W_r] over [e | n[send] | n[recv]]."""

    def __init__(self, w, prefix, device, C, mode=None):
        self.edge = _MLPNorm(w, f"{prefix}._edge_mlp", device, mode)
        self.node = _MLPNorm(w, f"{prefix}._node_mlp", device, mode)
        W0 = w[f"{prefix}._edge_mlp.mlp.NN-0.weight"]            # [H, 3C]
        if W0.shape[1] != 3 * C:
            raise ValueError(f"{prefix}: edge MLP input is {W0.shape[1]}, expected {3 * C}")
        We, Ws, Wr = W0[:, :C], W0[:, C:2 * C], W0[:, 2 * C:]
        self.we_t = _gw(We.T.contiguous(), device, mode)                    # [C, H]
        self.wsr_t = _gw(torch.cat([Ws.T, Wr.T], 1).contiguous(), device, mode)  # [C, 2H]
        self.we = _gw(We.contiguous(), device, mode)                        # [H, C]
        self.wsr = _gw(torch.cat([Ws, Wr], 0).contiguous(), device, mode)     # [2H, C]
        self.attn_w = _dev(torch.cat([w[f"{prefix}._receive_attn.weight"].reshape(-1),
                                      w[f"{prefix}._send_attn.weight"].reshape(-1)]), device)
        self.attn_b = _dev(torch.cat([w[f"{prefix}._receive_attn.bias"].reshape(-1),
                                      w[f"{prefix}._send_attn.bias"].reshape(-1)]), device)
        self.cond_w_t = self.cond_b = None
        if f"{prefix}._cond_node_proj.weight" in w:
            self.cond_w_t = _dev(w[f"{prefix}._cond_node_proj.weight"].T.contiguous(), device)
            self.cond_b = _dev(w[f"{prefix}._cond_node_proj.bias"], device)


class _Head:
    """Linear-SiLU-Linear readout weights of an energy / force / stress head
    (orb_model.py:307-435): forward w_t [in, out], backward w [out, in], biases."""

    def __init__(self, w, prefix, device, n_out):
        self.w_t = [_dev(w[f"{prefix}.mlp.NN-{i}.weight"].T.contiguous(), device) for i in (0, 1)]
        self.w = [_dev(w[f"{prefix}.mlp.NN-{i}.weight"], device) for i in (0, 1)]
        self.b = [_dev(w[f"{prefix}.mlp.NN-{i}.bias"], device) for i in (0, 1)]
        if self.w_t[1].shape[1] != n_out:
            raise RuntimeError(f"{prefix} must have {n_out} outputs")
        self.hidden = int(self.w_t[0].shape[1])


class OrbModel:
    """Device-resident Orb-v3 weights, built once per checkpoint (orb_calculator.py:54-73)."""

    def __init__(self, weights, cfg, device="cuda", precision="f32"):
        nat.load()
        if precision not in PRECISIONS:
            raise RuntimeError(f"precision must be one of {sorted(PRECISIONS)}")
        self.precision = precision
        mode = PRECISIONS[precision]
        w = {k: torch.as_tensor(v, dtype=torch.float32) for k, v in weights.items()}
        self.cfg = dict(cfg)
        self.device = torch.device(device)
        self.C = int(cfg["latent_dim"])
        self.nb = int(cfg["num_bases"])
        self.r_max = float(cfg["cutoff"])
        if int(cfg.get("lmax", 3)) != 3 or int(cfg["edge_embed_size"]) != 16 * self.nb:
            raise RuntimeError("Orb path supports lmax=3 spherical harmonics with "
                               "edge_embed_size = 16 * num_bases")
        if self.C % 4 or self.C > 1024:
            raise RuntimeError("latent_dim must be a multiple of 4 and at most 1024")
        dev = self.device
        self.node_emb = w["atom_emb.embeddings.weight"]          # host table, gathered per graph
        enc = (_MLPNorm(w, "_encoder._node_fn", dev, mode),
               _MLPNorm(w, "_encoder._edge_fn", dev, mode))
        layers = [_Layer(w, f"gnn_stacks.{i}", dev, self.C, mode)
                  for i in range(int(cfg["num_message_passing_steps"]))]
        # direct checkpoints carry a force head (and usually a stress head) and are evaluated by
        # the forward alone (orb_calculator.py:66-72, 141-185)
        heads = [_Head(w, "energy_head", dev, 1)]
        heads.append(_Head(w, "forces_head", dev, 3) if "forces_head.mlp.NN-0.weight" in w
                     else None)
        heads.append(_Head(w, "stress_head", dev, 6) if "stress_head.mlp.NN-0.weight" in w
                     else None)
        host_w = {k: v for k, v in w.items() if k.startswith(("energy_head.normalizer",
                                                              "energy_head.reference",
                                                              "forces_head.normalizer",
                                                              "stress_head.diag_normalizer",
                                                              "stress_head.offdiag_normalizer",
                                                              "conditioner."))}
        self._finish(enc, layers, heads, host_w)

    def _finish(self, enc, layers, heads, host_w):
        self.enc_node, self.enc_edge = enc
        self.layers = list(layers)
        self.H = self.layers[0].edge.hidden if self.layers else self.enc_edge.hidden
        for L in self.layers:
            if L.edge.hidden != self.H or L.node.hidden != self.H:
                raise RuntimeError("all edge / node MLPs must share one hidden width")
        eh, fh, sh = heads
        self.eh_w_t, self.eh_w, self.eh_b = eh.w_t, eh.w, eh.b
        self.is_direct = fh is not None
        self.has_stress_head = sh is not None
        self.fh_w_t = self.fh_b = self.sh_w_t = self.sh_b = None
        if fh is not None:
            self.fh_w_t, self.fh_b = fh.w_t, fh.b
        if sh is not None:
            self.sh_w_t, self.sh_b = sh.w_t, sh.b
        self.host_w = dict(host_w)
        self.has_cond = "conditioner.charge_embedding.W" in self.host_w

    @classmethod
    def from_parts(cls, enc, layers, heads, *, cfg, device, precision, host_w=None,
                   node_emb=None):
        """A model over already-built device weights (the module objects of tt_atom.orb_model):
        ``enc`` = (node MLPNorm, edge MLPNorm), ``layers`` = interaction-layer weights,
        ``heads`` = (energy head, force head or None, stress head or None)."""
        self = cls.__new__(cls)
        self.precision = precision
        self.cfg = dict(cfg)
        self.device = torch.device(device)
        self.C = int(cfg["latent_dim"])
        self.nb = int(cfg["num_bases"])
        self.r_max = float(cfg["cutoff"])
        if self.nb < 1 or self.nb > 64 or self.nb & (self.nb - 1):
            raise RuntimeError("num_bases must be a power of two <= 64")
        self.node_emb = node_emb
        self._finish(enc, layers, heads, host_w or {})
        return self

    def charge_spin_embedding_batch(self, charges, spins, natoms):
        """charge_spin_embedding of K systems at once, one row per node [sum natoms, C]."""
        return charge_spin_embedding_batch(self.host_w, self.C, charges, spins, natoms)

    def charge_spin_embedding(self, charge, spin, n):
        """sin/cos charge/spin conditioning broadcast to n nodes (orb_model.py:32-56)."""
        def emb(value, W, is_spin):
            proj = float(value) * W * (2.0 * math.pi)
            e = torch.cat([torch.sin(proj), torch.cos(proj)])
            return torch.zeros_like(e) if (is_spin and value == 0) else e
        c = torch.cat([emb(charge, self.host_w["conditioner.charge_embedding.W"], False),
                       emb(spin, self.host_w["conditioner.spin_embedding.W"], True)])
        if c.shape[0] != self.C:
            raise RuntimeError("conditioning width does not match latent_dim")
        return c[None].expand(n, -1)


def charge_spin_embedding_batch(w, C, charges, spins, natoms):
    """sin/cos charge / spin conditioning (orb_model.py:32-56) of K systems at once: the same
    fp32 operations as the one-system form on [K, C/4] blocks, repeated over each system's
    nodes -> [sum natoms, C]; a zero spin gives a zero spin block."""
    Wc = torch.as_tensor(w["conditioner.charge_embedding.W"], dtype=torch.float32)
    Ws = torch.as_tensor(w["conditioner.spin_embedding.W"], dtype=torch.float32)
    q = torch.as_tensor(charges, dtype=torch.float32).reshape(-1, 1)
    sp = torch.as_tensor(spins, dtype=torch.float32).reshape(-1, 1)
    pc = q * Wc[None] * (2.0 * math.pi)
    ps = sp * Ws[None] * (2.0 * math.pi)
    es = torch.cat([torch.sin(ps), torch.cos(ps)], 1) * (sp != 0).to(torch.float32)
    c = torch.cat([torch.sin(pc), torch.cos(pc), es], 1)
    if c.shape[1] != C:
        raise RuntimeError("conditioning width does not match latent_dim")
    return c.repeat_interleave(torch.as_tensor(natoms, dtype=torch.long), dim=0)


# ----------------------------------------------------------------------------- engine
class OrbEngine:
    """One fixed-topology energy + forces step: buffers are allocated once per graph and every
    call is the same kernel sequence, captured as a HIP graph on the second call of each variant
    (with / without stress) and replayed afterwards unless ``use_graph`` is False.  For a direct
    checkpoint the step is the forward and the force / stress heads; otherwise the forward and
    the analytic backward."""

    def __init__(self, model, graph, cond_nodes=None, use_graph=True, node_feat=None):
        self.m, self.g = model, graph
        dev = model.device
        N, E, K, C, H = graph.N, graph.E, graph.K, model.C, model.H
        nb16 = 16 * model.nb
        f = lambda *s: torch.empty(*s, device=dev, dtype=torch.float32)
        self.use_graph = use_graph
        self._graphs = StepGraphs(self._step)
        self.pos = f(N, 3)
        if node_feat is None:
            if model.node_emb is None:
                raise ValueError("node_feat is required for a model built without the atom "
                                 "embedding table")
            node_feat = model.node_emb[graph.Z.cpu()]
        if tuple(node_feat.shape) != (N, model.enc_node.w_t[0].shape[0]):
            raise ValueError(f"node_feat must be [{N}, {model.enc_node.w_t[0].shape[0]}], got "
                             f"{tuple(node_feat.shape)}")
        self.x_node = _dev(node_feat, dev)
        self.cond = None if cond_nodes is None else _dev(cond_nodes, dev)
        He = model.eh_w_t[0].shape[1]
        L = len(model.layers)
        # geometry
        self.vec, self.feat, self.cut = f(E, 3), f(E, nb16), f(E)
        # transient activations
        self.h0, self.h1 = f(E, H), f(E, H)
        self.P = f(N, 2 * H)
        self.edges = [f(E, C), f(E, C)]
        self.nodes = [f(N, C) for _ in range(L + 1)]
        self.node_in = f(N, 3 * C)
        self.hn0, self.hn1, self.hn_out = f(N, H), f(N, H), f(N, C)
        self.enc_h0, self.enc_h1 = f(N, model.enc_node.hidden), f(N, model.enc_node.hidden)
        # saved for the backward
        self.ea0, self.ea1, self.eh2, self.einv = f(E, H), f(E, H), f(E, C), f(E)
        self.a0 = [f(E, H) for _ in range(L)]
        self.a1 = [f(E, H) for _ in range(L)]
        self.h2 = [f(E, C) for _ in range(L)]
        self.ue = [f(E, C) for _ in range(L)]
        self.inv = [f(E) for _ in range(L)]
        self.sig = [f(E, 2) for _ in range(L)]
        self.an0 = [f(N, H) for _ in range(L)]
        self.an1 = [f(N, H) for _ in range(L)]
        self.hn2 = [f(N, C) for _ in range(L)]
        self.ninv = [f(N) for _ in range(L)]
        self.mean, self.ha, self.hh, self.raw = f(K, C), f(K, He), f(K, He), f(K, 1)
        # backward
        self.ones = torch.ones(K, 1, device=dev, dtype=torch.float32)
        self.g_ha, self.g_mean = f(K, He), f(K, C)
        self.g_n, self.g_e, self.g_cut = f(N, C), f(E, C), f(E)
        self.g_hn2, self.g_an1, self.g_an0, self.g_node_in = f(N, C), f(N, H), f(N, H), f(N, 3 * C)
        self.g_h2, self.G = f(E, C), f(N, 2 * H)
        self.g_feat, self.g_vec = f(E, nb16), f(E, 3)
        self.forces, self.virial_buf, self.work = f(N, 3), f(9), f(256 * 9)
        # direct heads
        if model.is_direct:
            self.fa, self.fpred = f(N, model.fh_w_t[0].shape[1]), f(N, 3)
        if model.has_stress_head:
            self.sa, self.raw_s = f(K, model.sh_w_t[0].shape[1]), f(K, 6)

    # -- forward --------------------------------------------------------------------------
    def _mlp3(self, mlp, x, a0, h0, a1, h1, h2):
        nat.linear(x, mlp.w_t[0], mlp.b[0], out=a0, epilogue=nat.EPI_PRE_SILU, out2=h0)
        nat.linear(h0, mlp.w_t[1], mlp.b[1], out=a1, epilogue=nat.EPI_PRE_SILU, out2=h1)
        nat.linear(h1, mlp.w_t[2], mlp.b[2], out=h2)

    def _forward(self, pos):
        m, g = self.m, self.g
        nat.orb_edge_features(pos, g.send, g.recv, g.shift, m.r_max, m.nb, self.vec, self.feat,
                              self.cut)
        # encoder: node path (position independent, not differentiated) and edge path; the two
        # MLPs are independent, so each of their layers is one grouped launch
        en, ee = m.enc_node, m.enc_edge
        nat.linear_group([(self.x_node, en.w_t[0], en.b[0], self.enc_h0, nat.EPI_SILU),
                          (self.feat, ee.w_t[0], ee.b[0], self.ea0, nat.EPI_PRE_SILU, self.h0)])
        nat.linear_group([(self.enc_h0, en.w_t[1], en.b[1], self.enc_h1, nat.EPI_SILU),
                          (self.h0, ee.w_t[1], ee.b[1], self.ea1, nat.EPI_PRE_SILU, self.h1)])
        nat.linear_group([(self.enc_h1, en.w_t[2], en.b[2], self.hn_out),
                          (self.h1, ee.w_t[2], ee.b[2], self.eh2)])
        nat.rms_residual(self.hn_out, en.norm, None, None, self.nodes[0], None)
        L0 = m.layers[0] if m.layers else None
        nat.rms_residual(self.eh2, ee.norm, None, None, self.edges[0], self.einv,
                         None if L0 is None else L0.attn_w, None if L0 is None else L0.attn_b,
                         None if L0 is None else self.sig[0])
        H = m.H
        for l, lay in enumerate(m.layers):
            n_l, e_l, e_next = self.nodes[l], self.edges[l % 2], self.edges[(l + 1) % 2]
            if lay.cond_w_t is not None and self.cond is not None:
                nat.linear(self.cond, lay.cond_w_t, lay.cond_b, out=n_l, epilogue=nat.EPI_ACCUM)
            nat.linear(n_l, lay.wsr_t, out=self.P)
            nat.linear_gather(e_l, lay.we_t, lay.edge.b[0], self.a0[l], self.P, g.send, g.recv, H,
                              epilogue=nat.EPI_PRE_SILU, out2=self.h0)
            nat.linear(self.h0, lay.edge.w_t[1], lay.edge.b[1], out=self.a1[l],
                       epilogue=nat.EPI_PRE_SILU, out2=self.h1)
            nat.linear(self.h1, lay.edge.w_t[2], lay.edge.b[2], out=self.h2[l])
            nxt = m.layers[l + 1] if l + 1 < len(m.layers) else None
            nat.rms_residual(self.h2[l], lay.edge.norm, e_l, self.ue[l], e_next, self.inv[l],
                             None if nxt is None else nxt.attn_w,
                             None if nxt is None else nxt.attn_b,
                             None if nxt is None else self.sig[l + 1])
            nat.orb_segsum(self.ue[l], self.sig[l], self.cut, g.send_ptr, g.recv_ptr, g.recv_perm,
                           n_l, self.node_in)
            self._mlp3(lay.node, self.node_in, self.an0[l], self.hn0, self.an1[l], self.hn1,
                       self.hn2[l])
            nat.rms_residual(self.hn2[l], lay.node.norm, n_l, None, self.nodes[l + 1],
                             self.ninv[l])
        nat.segment_mean(self.nodes[len(m.layers)], g.seg_ptr, self.mean)
        nat.linear(self.mean, m.eh_w_t[0], m.eh_b[0], out=self.ha, epilogue=nat.EPI_PRE_SILU,
                   out2=self.hh)
        nat.linear(self.hh, m.eh_w_t[1], m.eh_b[1], out=self.raw)

    # -- backward -------------------------------------------------------------------------
    def _backward(self, compute_stress):
        m, g = self.m, self.g
        nat.linear(self.ones, m.eh_w[1], out=self.g_ha, epilogue=nat.EPI_SILU_GRAD, aux=self.ha)
        nat.linear(self.g_ha, m.eh_w[0], out=self.g_mean)
        nat.segment_mean_bwd(self.g_mean, g.batch, g.seg_ptr, self.g_n)
        nat.fill(self.g_e, 0.0)
        nat.fill(self.g_cut, 0.0)
        C = m.C
        for l in reversed(range(len(m.layers))):
            lay = m.layers[l]
            nat.rms_bwd(self.g_n, self.hn2[l], lay.node.norm, self.ninv[l], self.g_hn2)
            nat.linear(self.g_hn2, lay.node.w[2], out=self.g_an1, epilogue=nat.EPI_SILU_GRAD,
                       aux=self.an1[l])
            nat.linear(self.g_an1, lay.node.w[1], out=self.g_an0, epilogue=nat.EPI_SILU_GRAD,
                       aux=self.an0[l])
            nat.linear(self.g_an0, lay.node.w[0], out=self.g_node_in)
            nat.orb_edge_bwd(self.g_e, self.g_node_in, self.ue[l], self.sig[l], self.cut,
                             self.h2[l], self.inv[l], lay.edge.norm, lay.attn_w, g.send, g.recv,
                             self.g_h2, self.g_cut)
            nat.linear(self.g_h2, lay.edge.w[2], out=self.h1, epilogue=nat.EPI_SILU_GRAD,
                       aux=self.a1[l])
            nat.linear(self.h1, lay.edge.w[1], out=self.h0, epilogue=nat.EPI_SILU_GRAD,
                       aux=self.a0[l])
            nat.orb_node_segsum2(self.h0, g.send_ptr, g.recv_ptr, g.recv_perm, self.G)
            nat.add_rows(self.g_node_in[:, :C], self.g_n)
            # the edge input adjoint and the node adjoint through [W_s | W_r]: one launch
            nat.linear_group([(self.h0, lay.we, None, self.g_e, nat.EPI_ACCUM),
                              (self.G, lay.wsr, None, self.g_n, nat.EPI_ACCUM)])
        ee = m.enc_edge
        nat.rms_bwd(self.g_e, self.eh2, ee.norm, self.einv, self.g_h2)
        nat.linear(self.g_h2, ee.w[2], out=self.h1, epilogue=nat.EPI_SILU_GRAD, aux=self.ea1)
        nat.linear(self.h1, ee.w[1], out=self.h0, epilogue=nat.EPI_SILU_GRAD, aux=self.ea0)
        nat.linear(self.h0, ee.w[0], out=self.g_feat)
        nat.orb_edge_features_bwd(self.vec, self.g_feat, self.g_cut, m.r_max, m.nb, self.g_vec)
        # vec = pos[recv] - pos[send]: F[n] = sum_{send=n} g_vec - sum_{recv=n} g_vec
        nat.node_forces(self.g_vec, g.recv_ptr, g.recv_perm, g.send_ptr, self.forces)
        if compute_stress:
            nat.virial(self.vec, self.g_vec, self.work, self.virial_buf)

    # -- direct heads (orb_model.py:381-435) ------------------------------------------------
    def _direct_heads(self, compute_stress):
        m, g = self.m, self.g
        nodes = self.nodes[len(m.layers)]
        nat.linear(nodes, m.fh_w_t[0], m.fh_b[0], out=self.fa, epilogue=nat.EPI_SILU)
        nat.linear(self.fa, m.fh_w_t[1], m.fh_b[1], out=self.fpred)
        nat.segment_center(self.fpred, g.seg_ptr, self.forces)     # per-system net force removal
        if compute_stress:                                          # on the energy head's mean
            nat.linear(self.mean, m.sh_w_t[0], m.sh_b[0], out=self.sa, epilogue=nat.EPI_SILU)
            nat.linear(self.sa, m.sh_w_t[1], m.sh_b[1], out=self.raw_s)

    def _step(self, compute_stress):
        self._forward(self.pos)
        if self.m.is_direct:
            self._direct_heads(compute_stress)
        else:
            self._backward(compute_stress)

    def step(self, pos, compute_stress=False, eager=False):
        """Enqueue one step on the current stream; results stay in the device buffers (raw,
        forces, virial_buf).  Without ``eager`` (and with ``use_graph``) it replays a HIP graph
        captured on the second call of each variant (the first runs eagerly)."""
        if compute_stress and self.m.is_direct and not self.m.has_stress_head:
            raise ValueError("stress requested but this direct checkpoint carries no "
                             "stress_head weights")
        self.pos.copy_(torch.as_tensor(pos, dtype=torch.float32).reshape(-1, 3),
                       non_blocking=True)
        if self.use_graph and not eager:
            self._graphs.run(bool(compute_stress))
        else:
            self._step(compute_stress)

    def run(self, pos, compute_stress=False, eager=False):
        """pos [N, 3] fp32 (node order of the graph) -> (raw energies [K] fp64 host, raw forces
        [N, 3] device view, stress term or None); raw = normalised space, as
        orb_forces.energy_and_forces returns.  The stress term is the raw virial dE/dstrain
        [3, 3] (device view) for a conservative checkpoint and the StressHead's raw Voigt
        vectors [K, 6] for a direct one."""
        self.step(pos, compute_stress, eager)
        raw = self.raw.view(-1).double().cpu()
        if not compute_stress:
            return raw, self.forces, None
        return raw, self.forces, (self.raw_s if self.m.is_direct else self.virial_buf.view(3, 3))


# ----------------------------------------------------------------------------- functional API
def _prepare(model, pos, senders, receivers, atomic_numbers, cell_shift, natoms, cond_nodes,
             slot):
    """The step engine of this topology: the one kept on ``model`` from the last call with the
    same senders, receivers, species, cell shifts, system sizes and conditioning
    (``engine_cache``, so a fixed-topology loop replays the captured step), else a new one."""
    dev = model.device
    N = int(torch.as_tensor(atomic_numbers).shape[0])

    def build():
        graph = OrbGraph(dev, senders=senders, receivers=receivers, num_nodes=N,
                         atomic_numbers=atomic_numbers, cell_shift=cell_shift, natoms=natoms)
        return OrbEngine(model, graph, cond_nodes)

    key = (senders, receivers, atomic_numbers, cell_shift,
           None if natoms is None else tuple(int(n) for n in natoms), cond_nodes)
    eng = cached_engine(model, slot, key, build)
    p = torch.as_tensor(pos, dtype=torch.float32).to(dev).contiguous()
    return eng, p


def energy_and_forces(model, *, pos, senders, receivers, atomic_numbers, cell_shift=None,
                      compute_stress=False, cond_nodes=None):
    """Single system (orb_forces.py:307-378): raw energy (float), raw forces [N, 3] (host fp32)
    and, with ``compute_stress``, the raw virial dE/dstrain [3, 3]."""
    eng, p = _prepare(model, pos, senders, receivers, atomic_numbers, cell_shift, None, cond_nodes,
                      "energy_and_forces")
    raw, F, vir = eng.run(p, compute_stress)
    out = (float(raw[0]), F.detach().cpu().clone())
    return out if not compute_stress else out + (vir.detach().cpu().clone(),)


def energy_and_forces_batch(model, *, pos, senders, receivers, atomic_numbers, natoms,
                            cell_shift=None, cond_nodes=None):
    """Disjoint-union batch (orb_forces.py:257-304): raw energies [K] (fp64) and raw forces."""
    eng, p = _prepare(model, pos, senders, receivers, atomic_numbers, cell_shift, natoms,
                      cond_nodes, "energy_and_forces_batch")
    raw, F, _ = eng.run(p, False)
    return raw, F.detach().cpu().clone()


def denormalize_energy(raw, Z, n, w):
    """(raw sigma + mu) n + sum ref[Z] (orb_model.py:588-600)."""
    sigma = w["energy_head.normalizer.bn.running_var"].double().sqrt()
    mu = w["energy_head.normalizer.bn.running_mean"].double()
    ref = w["energy_head.reference.linear.weight"].double().reshape(-1)
    return (torch.as_tensor(raw).double() * sigma + mu) * n + ref[torch.as_tensor(Z).long()].sum()


def denormalize_energy_batch(raw, Z, batch, natoms, w):
    """denormalize_energy of K systems at once: raw [K] -> [K] (fp64)."""
    sigma = w["energy_head.normalizer.bn.running_var"].double().sqrt()
    mu = w["energy_head.normalizer.bn.running_mean"].double()
    ref = w["energy_head.reference.linear.weight"].double().reshape(-1)
    refs = torch.zeros(len(natoms), dtype=torch.float64).index_add_(
        0, torch.as_tensor(batch).long(), ref[torch.as_tensor(Z).long()])
    return (torch.as_tensor(raw).double() * sigma + mu) * torch.as_tensor(
        natoms, dtype=torch.float64) + refs


def denormalize_forces(raw_f, n, w):
    """raw forces * sigma * n (orb_model.py:459-469)."""
    return raw_f.double() * w["energy_head.normalizer.bn.running_var"].double().sqrt() * n


def denormalize_stress(virial, n, cell, w):
    """virial * sigma * n / volume -> Voigt [xx, yy, zz, yz, xz, xy] (orb_model.py:472-488)."""
    sigma = w["energy_head.normalizer.bn.running_var"].double().sqrt()
    s = virial.double() * sigma * n / torch.linalg.det(torch.as_tensor(cell).double()).abs()
    return torch.stack([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]),
                        0.5 * (s[0, 2] + s[2, 0]), 0.5 * (s[0, 1] + s[1, 0])])


def denormalize_direct_forces(raw_f, w):
    """Direct ForceHead output raw sigma + mu (orb_model.py:438-442)."""
    sigma = w["forces_head.normalizer.bn.running_var"].double().sqrt()
    return raw_f.double() * sigma + w["forces_head.normalizer.bn.running_mean"].double()


def denormalize_direct_stress(raw_s, w):
    """Direct StressHead Voigt vector: components 0..2 through the diagonal normaliser, 3..5
    through the off-diagonal one, no volume division (orb_model.py:445-457)."""
    raw = raw_s.double().reshape(-1, 6)
    p = "stress_head.diag_normalizer.bn."
    q = "stress_head.offdiag_normalizer.bn."
    diag = raw[:, :3] * w[p + "running_var"].double().sqrt() + w[p + "running_mean"].double()
    off = raw[:, 3:] * w[q + "running_var"].double().sqrt() + w[q + "running_mean"].double()
    return torch.cat([diag, off], dim=1).reshape(raw_s.shape)
