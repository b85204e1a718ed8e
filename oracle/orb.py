"""CPU oracle for the Orb-v3 edge-MLP + scatter path (TEST INFRASTRUCTURE ONLY).

Plain PyTorch restatement of the reference's Orb forward (orb_geometry.py, orb_model.py) with
``torch.autograd`` standing in for the analytic VJP of orb_forces.py.  Used only by ``tests/``
and by ``bench.py``'s ``cpu_baseline`` leg, as the checker.

Pins (tests/test_oracle_orb.py):
  * Bessel basis: orthonormality on [0, r_max] with weight r^2, closed values;
  * real spherical harmonics: sum_m Y_lm^2 = 2l+1, Monte-Carlo orthonormality, harmonicity of
    r^l Y_lm, and the component order/signs against ``tests/golden/orb_geometry_small.npz``
    (vectors written by the reference's own functions, see tests/golden/gen_orb_geometry.py);
  * cutoff envelope: value 1 / slope 0 at r=0, value, slope and curvature 0 at r_max;
  * edge geometry and its force VJP against that fixture (fp64);
  * backbone: fp64 finite differences of energy and stress, translation invariance, atom
    permutation invariance, disjoint-union batching == per-system evaluation, segment sums vs
    dense one-hot products.
  * direct heads: per-system net force exactly zero, atom-permutation equivariance of the forces
    and invariance of the stress head, batch == per-system, the normaliser split of the six
    stress components on known values;
  * known answers (tests/test_oracle_orb.py, "known answers" section): selection-matrix weights
    reduce MLPNorm, the attention layer (for every choice of the concatenation block each MLP
    reads, with and without conditioning), the energy / force / stress heads and a two-layer
    encoder + layers + head composition to closed forms evaluated by explicit loops over the
    edge list; planted wiring mistakes (swapped sender / receiver sums, concatenation orders,
    gate channels, a misplaced RMSNorm weight, batch-wide head means) fail them;
  * denormalisers and the charge / spin conditioning against hand-evaluated values.
No Orb golden vector of the reference is committed (they are gated), so the composition is pinned
by the reference's statement of each layer through those known answers and by the invariants.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .geometry import neighbor_list

N_SH = 16


# ----------------------------------------------------------------------------- geometry
def bessel(r, r_max=6.0, nb=8):
    """sqrt(2/r_max) sin(n pi r / r_max) / r, n = 1..nb (orb_geometry.py:29-34)."""
    n = torch.arange(1, nb + 1, dtype=r.dtype)
    return math.sqrt(2.0 / r_max) * torch.sin(r[:, None] * (n * (math.pi / r_max))) / r[:, None]


def sph_l3(u):
    """Real spherical harmonics l = 0..3 of unit vectors, component normalisation (each l block
    scaled by sqrt(2l+1)); component order as orb_geometry.py:37-62."""
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    s3 = math.sqrt(3.0)
    xx, yy, zz = x * x, y * y, z * z
    p = xx + zz
    c20, c21, c22, c23, c24 = s3 * x * z, s3 * x * y, yy - 0.5 * p, s3 * y * z, 0.5 * s3 * (zz - xx)
    cols = [torch.ones_like(x), x, y, z, c20, c21, c22, c23, c24,
            math.sqrt(5.0 / 6.0) * (c20 * z + c24 * x),
            math.sqrt(5.0) * c20 * y,
            math.sqrt(3.0 / 8.0) * (4.0 * yy - p) * x,
            0.5 * y * (2.0 * yy - 3.0 * p),
            math.sqrt(3.0 / 8.0) * (4.0 * yy - p) * z,
            math.sqrt(5.0) * c24 * y,
            math.sqrt(5.0 / 6.0) * (c24 * z - c20 * x)]
    scale = torch.tensor([math.sqrt(2 * l + 1) for l in range(4) for _ in range(2 * l + 1)],
                         dtype=u.dtype)
    return torch.stack(cols, dim=1) * scale


def envelope(r, r_max=6.0):
    """Polynomial cutoff p=4 (orb_model.py:69-82): 1 - 15 q^4 + 24 q^5 - 10 q^6, 0 at r >= r_max."""
    q = r / r_max
    q4 = q ** 4
    val = 1.0 - 15.0 * q4 + 24.0 * q4 * q - 10.0 * q4 * q * q
    return val * (r < r_max).to(r.dtype)


def edge_features(pos, senders, receivers, shift=None, r_max=6.0, nb=8, strain=None):
    """pos -> (edge_feat [E, nb*16], cutoff [E, 1], vectors [E, 3]); orb_geometry.py:65-97.

    vectors = pos[receivers] - pos[senders] + shift; edge_feat[e, n*16 + m] =
    cutoff[e] * rbf_n(r_e) * Y_m(v_e / r_e)."""
    v = pos[receivers] - pos[senders]
    if shift is not None:
        v = v + shift
    if strain is not None:
        v = v + v @ (0.5 * (strain + strain.transpose(0, 1)))
    r = torch.linalg.norm(v, dim=1)
    u = F.normalize(v, dim=1)
    cut = envelope(r, r_max)[:, None]
    feat = (bessel(r, r_max, nb)[:, :, None] * sph_l3(u)[:, None, :]).reshape(v.shape[0], -1)
    return cut * feat, cut, v


# ----------------------------------------------------------------------------- network
def rmsnorm(x, w, eps=1e-6):
    """torch.nn.RMSNorm over the last dim (orb_model.py:92-112)."""
    return x * torch.rsqrt((x * x).mean(dim=-1, keepdim=True) + eps) * w


def _lin(x, w, name):
    return F.linear(x, w[f"{name}.weight"], w[f"{name}.bias"])


def mlp_norm(x, w, prefix):
    """Linear-SiLU-Linear-SiLU-Linear then RMSNorm (orb_model.py:127-173)."""
    h = F.silu(_lin(x, w, f"{prefix}.mlp.NN-0"))
    h = F.silu(_lin(h, w, f"{prefix}.mlp.NN-1"))
    h = _lin(h, w, f"{prefix}.mlp.NN-2")
    return rmsnorm(h, w[f"{prefix}.layer_norm.weight"])


def attention_layer(nodes, edges, senders, receivers, cut, w, prefix, cond_nodes=None):
    """One AttentionInteractionLayer (orb_model.py:225-266): sigmoid attention gates scaled by
    the cutoff, edge MLP on [e | n[send] | n[recv]], sender / receiver segment sums, node MLP on
    [n | recv_agg | sent_agg], residual on both."""
    N = nodes.shape[0]
    if cond_nodes is not None and f"{prefix}._cond_node_proj.weight" in w:
        nodes = nodes + _lin(cond_nodes, w, f"{prefix}._cond_node_proj")
    ra = torch.sigmoid(_lin(edges, w, f"{prefix}._receive_attn")) * cut
    sa = torch.sigmoid(_lin(edges, w, f"{prefix}._send_attn")) * cut
    ue = mlp_norm(torch.cat([edges, nodes[senders], nodes[receivers]], dim=1), w,
                  f"{prefix}._edge_mlp")
    C = ue.shape[1]
    sent = torch.zeros(N, C, dtype=ue.dtype).index_add_(0, senders, ue * sa)
    recv = torch.zeros(N, C, dtype=ue.dtype).index_add_(0, receivers, ue * ra)
    un = mlp_norm(torch.cat([nodes, recv, sent], dim=1), w, f"{prefix}._node_mlp")
    return nodes + un, edges + ue


def energy_head(nodes, batch, natoms, w):
    """Per-system mean of node features, then Linear-SiLU-Linear -> raw [K]
    (orb_model.py:329-355)."""
    K = len(natoms)
    mean = torch.zeros(K, nodes.shape[1], dtype=nodes.dtype).index_add_(0, batch, nodes)
    mean = mean / torch.as_tensor(natoms, dtype=nodes.dtype)[:, None]
    h = F.silu(_lin(mean, w, "energy_head.mlp.NN-0"))
    return _lin(h, w, "energy_head.mlp.NN-1")[:, 0]


def node_features(w, Z):
    """Atomic-number embedding lookup (orb_model.py:59-66)."""
    return w["atom_emb.embeddings.weight"][Z]


def force_head(nodes, batch, natoms, w):
    """Direct ForceHead (orb_model.py:381-404): per-node Linear-SiLU-Linear -> [N, 3], then each
    system's mean predicted force is subtracted (net-force removal per system, as the batched
    form does; one system = the single-system form)."""
    h = F.silu(_lin(nodes, w, "forces_head.mlp.NN-0"))
    pred = _lin(h, w, "forces_head.mlp.NN-1")
    K = len(natoms)
    mean = torch.zeros(K, pred.shape[1], dtype=pred.dtype).index_add_(0, batch, pred)
    mean = mean / torch.as_tensor(natoms, dtype=pred.dtype)[:, None]
    return pred - mean[batch]


def stress_head(nodes, batch, natoms, w):
    """Direct StressHead (orb_model.py:429-435): per-system mean of node features, then
    Linear-SiLU-Linear -> raw Voigt [K, 6] ([xx, yy, zz, yz, xz, xy])."""
    K = len(natoms)
    mean = torch.zeros(K, nodes.shape[1], dtype=nodes.dtype).index_add_(0, batch, nodes)
    mean = mean / torch.as_tensor(natoms, dtype=nodes.dtype)[:, None]
    h = F.silu(_lin(mean, w, "stress_head.mlp.NN-0"))
    return _lin(h, w, "stress_head.mlp.NN-1")


def node_embedding(w, cfg, Z, edge_feat, cut, senders, receivers, cond_nodes=None):
    """Encoder and the message-passing layers -> final node features [N, latent]."""
    nodes = mlp_norm(node_features(w, Z), w, "_encoder._node_fn")
    edges = mlp_norm(edge_feat, w, "_encoder._edge_fn")
    for i in range(cfg["num_message_passing_steps"]):
        nodes, edges = attention_layer(nodes, edges, senders, receivers, cut, w,
                                       f"gnn_stacks.{i}", cond_nodes)
    return nodes


def backbone(w, cfg, Z, edge_feat, cut, senders, receivers, batch, natoms, cond_nodes=None):
    nodes = node_embedding(w, cfg, Z, edge_feat, cut, senders, receivers, cond_nodes)
    return energy_head(nodes, batch, natoms, w)


def direct_forward(w, cfg, pos, Z, senders, receivers, shift, batch, natoms, *,
                   compute_stress=False, cond_nodes=None):
    """Direct checkpoint, forward only (orb_calculator.py:141-185, 266-277): raw energies [K],
    raw forces from the ForceHead [N, 3] and, with ``compute_stress``, the raw StressHead Voigt
    vectors [K, 6]."""
    dt = pos.dtype
    w = {k: v.to(dt) for k, v in w.items()}
    feat, cut, _ = edge_features(pos, senders, receivers, shift, cfg["cutoff"], cfg["num_bases"])
    nodes = node_embedding(w, cfg, Z, feat, cut, senders, receivers,
                           None if cond_nodes is None else cond_nodes.to(dt))
    raw_e = energy_head(nodes, batch, natoms, w)
    raw_f = force_head(nodes, batch, natoms, w)
    raw_s = stress_head(nodes, batch, natoms, w) if compute_stress else None
    return raw_e, raw_f, raw_s


def energy_and_forces(w, cfg, pos, Z, senders, receivers, shift, batch, natoms, *,
                      compute_stress=False, cond_nodes=None):
    """Raw (normalised-space) per-system energies [K], raw forces -d(sum_k E_k)/dpos [N, 3] and
    optionally the raw virial dE/dstrain [3, 3] (orb_forces.py:257-378)."""
    dt = pos.dtype
    w = {k: v.to(dt) for k, v in w.items()}
    pos = pos.detach().clone().requires_grad_(True)
    strain = torch.zeros(3, 3, dtype=dt, requires_grad=True) if compute_stress else None
    feat, cut, _ = edge_features(pos, senders, receivers, shift, cfg["cutoff"], cfg["num_bases"],
                                 strain)
    raw = backbone(w, cfg, Z, feat, cut, senders, receivers, batch, natoms,
                   None if cond_nodes is None else cond_nodes.to(dt))
    ins = [pos] if strain is None else [pos, strain]
    grads = torch.autograd.grad(raw.sum(), ins)
    if strain is None:
        return raw.detach(), -grads[0]
    return raw.detach(), -grads[0], grads[1]


# ----------------------------------------------------------------------------- host pieces
def charge_spin_embedding(w, charge, spin, n):
    """sin/cos conditioning embedding broadcast to n nodes (orb_model.py:32-56)."""
    def emb(value, W, is_spin):
        proj = float(value) * W * (2.0 * math.pi)
        e = torch.cat([torch.sin(proj), torch.cos(proj)])
        return torch.zeros_like(e) if (is_spin and value == 0) else e
    c = torch.cat([emb(charge, w["conditioner.charge_embedding.W"], False),
                   emb(spin, w["conditioner.spin_embedding.W"], True)])
    return c[None].expand(n, -1).contiguous()


def assemble(systems, r_max, max_neighbors):
    """Disjoint union under Orb's convention (disjoint.py:162-218): per-system neighbour list,
    senders = tgt, receivers = src, node offsets.  Departure (builder decision): instead of
    refusing a system whose degree exceeds the cap, the cap rule of ``neighbor_list`` (nearest
    ``max_neighbors`` per sender) is applied.  ``systems``: list of (pos, Z[, cell, pbc])."""
    pos_all, Z_all, s_all, r_all, sh_all, b_all, natoms = [], [], [], [], [], [], []
    off = 0
    for k, sysk in enumerate(systems):
        pos, Z = sysk[0], sysk[1]
        cell = sysk[2] if len(sysk) > 2 else None
        pbc = sysk[3] if len(sysk) > 3 else None
        ei, shift = neighbor_list(pos, r_max, cell, pbc, max_neighbors)
        if ei.shape[1] == 0:
            raise ValueError(f"system {k} has no edges within cutoff")
        n = Z.shape[0]
        pos_all.append(pos)
        Z_all.append(Z)
        s_all.append(ei[1] + off)
        r_all.append(ei[0] + off)
        sh_all.append(shift)
        b_all.append(torch.full((n,), k, dtype=torch.long))
        natoms.append(n)
        off += n
    return dict(pos=torch.cat(pos_all), Z=torch.cat(Z_all), senders=torch.cat(s_all),
                receivers=torch.cat(r_all), shift=torch.cat(sh_all), batch=torch.cat(b_all),
                natoms=natoms)


def denormalize_energy(raw, Z, n, running_mean, running_var, ref_weight):
    """(raw sigma + mu) n + sum ref[Z] (orb_model.py:588-600)."""
    return ((raw.double() * running_var.double().sqrt() + running_mean.double()) * n
            + ref_weight.double().reshape(-1)[Z].sum())


def denormalize_forces(raw_f, n, running_var):
    """raw forces * sigma * n (orb_model.py:459-469)."""
    return raw_f.double() * running_var.double().sqrt() * n


def denormalize_direct_forces(raw_f, running_mean, running_var):
    """ForceHead's scalar normaliser inverse raw sigma + mu (orb_model.py:438-442)."""
    return raw_f.double() * running_var.double().sqrt() + running_mean.double()


def denormalize_direct_stress(raw_s, diag_mean, diag_var, offdiag_mean, offdiag_var):
    """StressHead's two normalisers: components 0..2 and 3..5 each raw sigma + mu, no volume
    division (orb_model.py:445-457)."""
    raw = raw_s.double().reshape(-1, 6)
    diag = raw[:, :3] * diag_var.double().sqrt() + diag_mean.double()
    off = raw[:, 3:] * offdiag_var.double().sqrt() + offdiag_mean.double()
    return torch.cat([diag, off], dim=1).reshape(raw_s.shape)
