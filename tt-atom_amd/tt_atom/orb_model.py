"""Orb-v3 modules under the reference's names and constructors (orb_model.py:32-600).

The reference builds one device module per block -- ``Encoder``, ``AttentionInteractionLayer``
per message-passing step, ``EnergyHead`` (and a direct checkpoint's ``ForceHead`` /
``StressHead``) -- plus an ``OrbGraphContext`` per topology, and hands them to
``orb_forces.energy_and_forces(encoder, layers, ehead, device, ...)``.  The classes below take
the same constructor arguments and hold the weights in the layout of this build's kernels
(fp32 ``[in, out]`` / ``[out, in]`` operands, packed planes for the split MFMA GEMM, the first
edge-MLP weight split by input block); ``tt_atom.orb_forces`` assembles them into one
``OrbEngine`` step, where the whole forward and backward run as a fixed sequence of HIP kernels
fused across module boundaries (RMSNorm + residual + the next layer's attention gates in one
kernel).  The modules can also be called one by one on fp32 device tensors, as the reference's
ttnn ``__call__`` (orb_model.py:107-266, 329-355), with the reverse pass in
``orb_forces.rmsnorm_bw / mlpnorm_bw / attn_layer_bw / energy_bw(_batch)`` over the activations a
call keeps: the same kernels, launched per module (edges in the graph's edge order at the
interface).

``fast=True`` (the reference's bfloat8 weights) selects bf16 GEMM operands here;
``precision=`` picks any of ``tt_atom.model.PRECISIONS`` explicitly.

The ``host_*`` functions are the reference's fixed host terms (conditioning embedding, atom
embedding lookup, normalisers, ZBL pair repulsion), computed on the host in fp64 / fp32 as there.
"""
from __future__ import annotations

import torch

from . import _native as nat
from . import orb as _orb
from .model import PRECISIONS

__all__ = ["RMSNorm", "MLPNorm", "Encoder", "AttentionInteractionLayer", "OrbGraphContext",
           "EnergyHead", "ForceHead", "StressHead", "host_charge_spin_embedding",
           "host_node_features", "host_energy_denormalize", "host_force_denormalize",
           "host_stress_denormalize", "host_conservative_force_denormalize",
           "host_conservative_stress", "host_zbl_energy", "host_zbl_forces", "host_zbl_stress"]


def _precision(fast, precision):
    p = precision if precision is not None else ("bf16" if fast else "f32")
    if p not in PRECISIONS:
        raise ValueError(f"precision must be one of {sorted(PRECISIONS)}")
    return p


def _w32(weights):
    """State dict view with fp32 tensors (what the weight builders index)."""
    class _View(dict):
        def __missing__(self, key):
            v = torch.as_tensor(weights[key], dtype=torch.float32)
            self[key] = v
            return v

        def __contains__(self, key):
            return key in weights
    return _View()


def _device(device):
    return torch.device("cuda") if device is None else torch.device(device)


def _f32(t, device):
    """An fp32 contiguous tensor on ``device`` (module calls take device tensors)."""
    return torch.as_tensor(t).to(device=device, dtype=torch.float32).contiguous()


# ----------------------------------------------------------------------------- modules
class RMSNorm:
    """``torch.nn.RMSNorm`` weight over the last dim (orb_model.py:92-112); the normalisation
    runs fused with the residual add in the step's row kernel."""

    def __init__(self, weights, prefix, device, dim, eps=1e-6):
        w = torch.as_tensor(weights[f"{prefix}.weight"], dtype=torch.float32).reshape(-1)
        if w.numel() != dim:
            raise ValueError(f"{prefix}.weight has {w.numel()} entries, expected {dim}")
        if eps != 1e-6:
            raise ValueError("the Orb RMSNorm kernels use eps = 1e-6")
        self.dim, self.eps = int(dim), float(eps)
        self.w = _orb._dev(w, _device(device))

    def __call__(self, x):
        """x [R, dim] -> x rsqrt(mean(x^2) + eps) w (orb_model.py:107-112); keeps x and the
        per-row inverse RMS for ``orb_forces.rmsnorm_bw``."""
        x = _f32(x, self.w.device)
        y = torch.empty_like(x)
        inv = torch.empty(x.shape[0], device=x.device, dtype=torch.float32)
        nat.rms_residual(x, self.w, None, None, y, inv, eps=self.eps)
        self._cache_x, self._cache_inv = x, inv
        return y


class MLPNorm:
    """Linear-SiLU-Linear-SiLU-Linear + RMSNorm (orb_model.py:127-173); keys
    ``{prefix}.mlp.NN-{0,1,2}.{weight,bias}`` and ``{prefix}.layer_norm.weight``."""

    def __init__(self, weights, prefix, device, in_dim, hidden_dim, out_dim, *, fast=False,
                 minimal_matmul=False, precision=None):
        self.precision = _precision(fast, precision)
        self._p = _orb._MLPNorm(_w32(weights), prefix, _device(device),
                                PRECISIONS[self.precision])
        got = (int(self._p.w_t[0].shape[0]), self._p.hidden, self._p.out_dim)
        if got != (int(in_dim), int(hidden_dim), int(out_dim)):
            raise ValueError(f"{prefix}: weights are {got}, expected "
                             f"{(in_dim, hidden_dim, out_dim)}")
        self.norm = RMSNorm(weights, f"{prefix}.layer_norm", device, out_dim)

    def __call__(self, x):
        """x [R, in] -> RMSNorm(L2(silu(L1(silu(L0 x))))) (orb_model.py:155-173); keeps the
        pre-SiLU activations for ``orb_forces.mlpnorm_bw``."""
        p = self._p
        x = _f32(x, p.b[0].device)
        R = x.shape[0]
        f = lambda n: torch.empty(R, n, device=x.device, dtype=torch.float32)
        a0, h0, a1, h1, h2 = f(p.hidden), f(p.hidden), f(p.hidden), f(p.hidden), f(p.out_dim)
        nat.linear(x, p.w_t[0], p.b[0], out=a0, epilogue=nat.EPI_PRE_SILU, out2=h0)
        nat.linear(h0, p.w_t[1], p.b[1], out=a1, epilogue=nat.EPI_PRE_SILU, out2=h1)
        nat.linear(h1, p.w_t[2], p.b[2], out=h2)
        self._cache_a0, self._cache_a1 = a0, a1
        return self.norm(h2)


class Encoder:
    """``gns.Encoder``: node and edge MLPNorm blocks (orb_model.py:176-186)."""

    def __init__(self, weights, device, *, node_in, edge_in, latent_dim, hidden_dim, fast=False,
                 precision=None):
        self.node_fn = MLPNorm(weights, "_encoder._node_fn", device, node_in, hidden_dim,
                               latent_dim, fast=fast, precision=precision)
        self.edge_fn = MLPNorm(weights, "_encoder._edge_fn", device, edge_in, hidden_dim,
                               latent_dim, fast=fast, precision=precision)
        self.node_in, self.edge_in = int(node_in), int(edge_in)
        self.latent_dim, self.hidden_dim = int(latent_dim), int(hidden_dim)
        self.precision = self.node_fn.precision

    def __call__(self, node_features, edge_features):
        return self.node_fn(node_features), self.edge_fn(edge_features)


class AttentionInteractionLayer:
    """``gns.AttentionInteractionNetwork`` step (orb_model.py:189-266): edge and node MLPNorms,
    sigmoid attention gates times the cutoff, sender / receiver segment sums and the optional
    charge / spin conditioning projection."""

    def __init__(self, weights, prefix, device, *, latent_dim, hidden_dim, fast=False,
                 precision=None):
        self.precision = _precision(fast, precision)
        self.C = int(latent_dim)
        self._p = _orb._Layer(_w32(weights), prefix, _device(device), self.C,
                              PRECISIONS[self.precision])
        if self._p.edge.hidden != hidden_dim or self._p.node.hidden != hidden_dim:
            raise ValueError(f"{prefix}: MLP hidden width is {self._p.edge.hidden}, expected "
                             f"{hidden_dim}")
        self.has_cond = self._p.cond_w_t is not None
        # the two attention linears as one [C, 2] product (receive, send)
        self._attn_w_t = self._p.attn_w.view(2, self.C).t().contiguous()

    def __call__(self, nodes, edges, graph):
        """(nodes [N, C], edges [E, C]) -> (nodes + node update, edges + edge update), one
        message-passing step (orb_model.py:225-266): the conditioning projection (when the layer
        and ``graph.cond_nodes`` have one), sigmoid attention gates times ``graph.cutoff``, the
        edge MLPNorm on [e | n[send] | n[recv]] (its first layer as node products [W_s | W_r]
        gathered per edge), the sender / receiver sums of the gated messages, the node MLPNorm on
        [n | recv | sent].  Keeps what ``orb_forces.attn_layer_bw`` needs."""
        p, C = self._p, self.C
        t = graph._module_topology()
        dev, order = t.send.device, t.order
        N, E, H = graph.N, graph.E, p.edge.hidden
        f = lambda *sh: torch.empty(*sh, device=dev, dtype=torch.float32)
        n_l = _f32(nodes, dev).clone()
        if self.has_cond and graph.cond_nodes is not None:
            nat.linear(_f32(graph.cond_nodes, dev), p.cond_w_t, p.cond_b, out=n_l,
                       epilogue=nat.EPI_ACCUM)
        e_s = _f32(edges, dev)[order].contiguous()            # sender order inside
        sig = f(E, 2)
        nat.linear(e_s, self._attn_w_t, p.attn_b, out=sig, epilogue=nat.EPI_SIGMOID)
        P = f(N, 2 * H)
        nat.linear(n_l, p.wsr_t, out=P)
        a0, h0, a1, h1, h2 = f(E, H), f(E, H), f(E, H), f(E, H), f(E, C)
        nat.linear_gather(e_s, p.we_t, p.edge.b[0], a0, P, t.send, t.recv, H,
                          epilogue=nat.EPI_PRE_SILU, out2=h0)
        nat.linear(h0, p.edge.w_t[1], p.edge.b[1], out=a1, epilogue=nat.EPI_PRE_SILU, out2=h1)
        nat.linear(h1, p.edge.w_t[2], p.edge.b[2], out=h2)
        ue, e_new, inv = f(E, C), f(E, C), f(E)
        nat.rms_residual(h2, p.edge.norm, e_s, ue, e_new, inv)
        node_in = f(N, 3 * C)
        nat.orb_segsum(ue, sig, t.cut, t.send_ptr, t.recv_ptr, t.recv_perm, n_l, node_in)
        Hn = p.node.hidden
        an0, hn0, an1, hn1, hn2 = f(N, Hn), f(N, Hn), f(N, Hn), f(N, Hn), f(N, C)
        nat.linear(node_in, p.node.w_t[0], p.node.b[0], out=an0, epilogue=nat.EPI_PRE_SILU,
                   out2=hn0)
        nat.linear(hn0, p.node.w_t[1], p.node.b[1], out=an1, epilogue=nat.EPI_PRE_SILU, out2=hn1)
        nat.linear(hn1, p.node.w_t[2], p.node.b[2], out=hn2)
        n_new, ninv = f(N, C), f(N)
        nat.rms_residual(hn2, p.node.norm, n_l, None, n_new, ninv)
        self._cache = dict(sig=sig, a0=a0, a1=a1, h2=h2, ue=ue, inv=inv, an0=an0, an1=an1,
                           hn2=hn2, ninv=ninv, graph=graph)
        e_out = torch.empty_like(e_new)
        e_out[order] = e_new
        return n_new, e_out


class _HeadModule:
    prefix, n_out = "", 0

    def __init__(self, weights, device, *, latent_dim, hidden_dim, fast=False, precision=None):
        # hidden_dim is taken from the weights (the reference passes the MLP width here while
        # the heads carry their own, narrower one; it does not read the argument either)
        self._p = _orb._Head(_w32(weights), self.prefix, _device(device), self.n_out)
        if int(self._p.w_t[0].shape[0]) != latent_dim:
            raise ValueError(f"{self.prefix}: input width is {int(self._p.w_t[0].shape[0])}, "
                             f"expected latent_dim = {latent_dim}")
        self.precision = _precision(fast, precision)


class EnergyHead(_HeadModule):
    """``forcefield_heads.EnergyHead`` (orb_model.py:307-355): per-system mean of the node
    features, Linear-SiLU-Linear to one raw energy per system."""
    prefix, n_out = "energy_head", 1

    def _mlp(self, mean):
        p = self._p
        K = mean.shape[0]
        a0 = torch.empty(K, p.hidden, device=mean.device, dtype=torch.float32)
        h = torch.empty_like(a0)
        raw = torch.empty(K, 1, device=mean.device, dtype=torch.float32)
        nat.linear(mean, p.w_t[0], p.b[0], out=a0, epilogue=nat.EPI_PRE_SILU, out2=h)
        nat.linear(h, p.w_t[1], p.b[1], out=raw)
        self._cache_a0 = a0
        return raw

    def __call__(self, node_features):
        """node_features [N, C] of one system -> the raw energy [1, 1] (orb_model.py:329-338)."""
        x = _f32(node_features, self._p.b[0].device)
        N = x.shape[0]
        ptr = torch.tensor([0, N], dtype=torch.int32, device=x.device)
        mean = torch.empty(1, x.shape[1], device=x.device, dtype=torch.float32)
        nat.segment_mean(x, ptr, mean)
        self._cache_N = N
        return self._mlp(mean)

    def batch(self, node_features, seg_mean):
        """node_features [N, C] of K systems, ``seg_mean`` [K, N] the row-normalised segment
        matrix -> raw energies [K, 1] (orb_model.py:340-355)."""
        x = _f32(node_features, self._p.b[0].device)
        sm = _f32(seg_mean, x.device)
        mean = nat.linear(sm, x)
        return self._mlp(mean)


class ForceHead(_HeadModule):
    """Direct ``ForceHead`` (orb_model.py:358-404): per-node Linear-SiLU-Linear to [N, 3], each
    system's mean prediction removed."""
    prefix, n_out = "forces_head", 3


class StressHead(_HeadModule):
    """Direct ``StressHead`` (orb_model.py:407-435): per-system mean, Linear-SiLU-Linear to the
    raw Voigt-6 stress."""
    prefix, n_out = "stress_head", 6


class OrbGraphContext:
    """One fixed topology (orb_model.py:269-304): the edge lists in the reference's order,
    sorted by sender on the device for the segment kernels, and the optional conditioning rows.
    ``cutoff`` is accepted for signature compatibility and checked for shape only -- the step
    recomputes the envelope from the positions on the device.  Bucketing's padded graphs
    (``gather_edge_count`` below the edge count) do not exist here: the kernels take any shape."""

    def __init__(self, device, *, senders, receivers, cutoff, num_nodes, cond_nodes=None,
                 gather_edge_count=None, gather_width=0, natoms=None):
        E = int(torch.as_tensor(senders).numel())
        if gather_edge_count is not None and int(gather_edge_count) != E:
            raise ValueError("padded (bucketed) graphs are not used by this build: pass the true "
                             "edges only")
        if cutoff is not None and int(torch.as_tensor(cutoff).numel()) != E:
            raise ValueError("cutoff must hold one value per edge")
        self.device = _device(device)
        self.E, self.N = E, int(num_nodes)
        self.senders = torch.as_tensor(senders)
        self.receivers = torch.as_tensor(receivers)
        self.cutoff = cutoff
        self.cond_nodes = cond_nodes
        self.natoms = natoms
        self._topo = None

    def _module_topology(self):
        """The sender-sorted device topology and the cutoff in that order, for module calls
        (built on first use)."""
        if self._topo is None:
            if self.cutoff is None:
                raise ValueError("module calls need the graph's cutoff envelope")
            t = _orb.OrbGraph(self.device, senders=self.senders, receivers=self.receivers,
                              num_nodes=self.N,
                              atomic_numbers=torch.zeros(self.N, dtype=torch.int64))
            t.cut = _f32(self.cutoff, self.device).reshape(-1)[t.order].contiguous()
            t.inv_order = torch.empty_like(t.order)
            t.inv_order[t.order] = torch.arange(self.E, device=t.order.device)
            self._topo = t
        return self._topo

    def topology(self, atomic_numbers, cell_shift=None, natoms=None):
        return _orb.OrbGraph(self.device, senders=self.senders, receivers=self.receivers,
                             num_nodes=self.N, atomic_numbers=atomic_numbers,
                             cell_shift=cell_shift, natoms=natoms or self.natoms)


# ----------------------------------------------------------------------------- host terms
def host_charge_spin_embedding(weights, charge, spin, n_node, latent_dim):
    """sin/cos charge / spin conditioning of one system broadcast to its nodes
    (orb_model.py:32-56) -> [n_node, latent_dim]."""
    return _orb.charge_spin_embedding_batch(weights, int(latent_dim), [float(charge)],
                                            [float(spin)], [int(n_node)])


def host_node_features(weights, atomic_numbers):
    """Encoder node input: the atom-embedding row of each atomic number (orb_model.py:59-66)."""
    return torch.as_tensor(weights["atom_emb.embeddings.weight"])[
        torch.as_tensor(atomic_numbers).long()]


def host_energy_denormalize(raw_pred, atomic_numbers, n_node, *, running_mean, running_var,
                            ref_weight):
    """(raw sigma + mu) n + sum ref[Z] (orb_model.py:588-600), fp64."""
    w = {"energy_head.normalizer.bn.running_mean": torch.as_tensor(running_mean),
         "energy_head.normalizer.bn.running_var": torch.as_tensor(running_var),
         "energy_head.reference.linear.weight": torch.as_tensor(ref_weight)}
    return _orb.denormalize_energy(raw_pred, atomic_numbers, n_node, w)


def host_force_denormalize(raw_pred, *, running_mean, running_var):
    """ForceHead normaliser inverse raw sigma + mu (orb_model.py:438-442), fp64."""
    return _orb.denormalize_direct_forces(
        torch.as_tensor(raw_pred), {"forces_head.normalizer.bn.running_mean":
                                        torch.as_tensor(running_mean),
                                    "forces_head.normalizer.bn.running_var":
                                        torch.as_tensor(running_var)})


def host_stress_denormalize(raw_pred, *, diag_mean, diag_var, offdiag_mean, offdiag_var):
    """StressHead normalisers: components 0..2 and 3..5 each raw sigma + mu
    (orb_model.py:445-457), fp64."""
    p, q = "stress_head.diag_normalizer.bn.", "stress_head.offdiag_normalizer.bn."
    t = torch.as_tensor
    return _orb.denormalize_direct_stress(
        t(raw_pred), {p + "running_mean": t(diag_mean), p + "running_var": t(diag_var),
                      q + "running_mean": t(offdiag_mean), q + "running_var": t(offdiag_var)})


def host_conservative_force_denormalize(raw_forces, n_node, *, running_var):
    """raw forces sigma n (orb_model.py:459-469), fp64."""
    return _orb.denormalize_forces(
        torch.as_tensor(raw_forces), n_node,
        {"energy_head.normalizer.bn.running_var": torch.as_tensor(running_var)})


def host_conservative_stress(virial, n_node, cell, *, running_var):
    """virial sigma n / |det cell| -> Voigt [xx, yy, zz, yz, xz, xy] (orb_model.py:472-488)."""
    return _orb.denormalize_stress(
        torch.as_tensor(virial), n_node, cell,
        {"energy_head.normalizer.bn.running_var": torch.as_tensor(running_var)})


def _radii(covalent_radii):
    from .orb_calculator import _default_radii
    return _default_radii() if covalent_radii is None else covalent_radii


def host_zbl_energy(atomic_numbers, senders, receivers, vectors, *, p=6, node_aggregation="mean",
                    covalent_radii=None):
    """ZBL pair-repulsion energy of one system (orb_model.py:491-538), fp64; the covalent
    radii default to ASE's table, as in the reference."""
    from .orb_calculator import zbl_energy
    return zbl_energy(torch.as_tensor(atomic_numbers).long(), torch.as_tensor(senders).long(),
                      torch.as_tensor(receivers).long(), torch.as_tensor(vectors),
                      _radii(covalent_radii), p=p, aggregation=node_aggregation)


def host_zbl_forces(atomic_numbers, senders, receivers, pos, cell_shift=None, *,
                    node_aggregation="mean", covalent_radii=None):
    """-dV_ZBL/dpos [N, 3] (orb_model.py:541-562), fp64."""
    from .orb_calculator import zbl_energy_forces_stress
    _, F, _ = zbl_energy_forces_stress(
        torch.as_tensor(atomic_numbers).long(), torch.as_tensor(senders).long(),
        torch.as_tensor(receivers).long(), pos, cell_shift, _radii(covalent_radii),
        aggregation=node_aggregation)
    return torch.from_numpy(F)


def host_zbl_stress(atomic_numbers, senders, receivers, vectors, cell, *,
                    node_aggregation="mean", covalent_radii=None):
    """ZBL virial stress in Voigt-6 order [xx, yy, zz, yz, xz, xy] (orb_model.py:565-585):
    the strain derivative of the pair energy over |det cell|, fp64."""
    strain = torch.zeros(3, 3, dtype=torch.float64, requires_grad=True)
    sym = 0.5 * (strain + strain.T)
    v = torch.as_tensor(vectors).double().detach() @ (torch.eye(3, dtype=torch.float64) + sym)
    e = host_zbl_energy(atomic_numbers, senders, receivers, v,
                        node_aggregation=node_aggregation, covalent_radii=covalent_radii)
    (vir,) = torch.autograd.grad(e, strain)
    s = vir / torch.linalg.det(torch.as_tensor(cell).double()).abs()
    return torch.stack([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]),
                        0.5 * (s[0, 2] + s[2, 0]), 0.5 * (s[0, 1] + s[1, 0])])
