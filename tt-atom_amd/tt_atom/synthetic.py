"""Seeded synthetic systems and random-init weight bundles for the benchmark configurations.

Configurations (BASELINE.json ``configs``; seeds and unstated dimensions are builder decisions):

* C1 -- tiny eSCN-MD, 24-atom molecule in a 6 A cube (0.9 A rejection), lmax=mmax=2, 2 layers,
  C=H=edge_channels=16, 8 gaussians, cutoff 5 A, cap 20, grid FF, pos_emb charge/spin.
* C2 -- isolated edgewise kernel: N=8192 nodes, in-degree 25 (dst-sorted), C=128.
* C3 -- uma-s-1 architecture: 4 layers, C=H=edge_channels=128, 512 gaussians (the "512-wide
  edge/radial MLP"), cutoff 6 A, cap 30, spectral FF, rand_emb charge/spin, task omol; 2048
  atoms uniform in a 17 A ball (1.0 A rejection), charge 0, spin 1.
* C4 -- C3 weights (task omat) on FCC Cu 8x8x8 (a = 3.61 A) with N(0, 0.05 A) noise, PBC.

Every generator uses ``numpy.random.Generator(PCG64(seed))``; the weight seed is the config
seed + 100.  Element probabilities {H:.5, C:.3, N:.1, O:.1}.
"""
from __future__ import annotations

import math

import numpy as np
import torch

ELEMENTS = np.array([1, 6, 7, 8])
ELEMENT_P = np.array([0.5, 0.3, 0.1, 0.1])

SEEDS = {"C1": 1, "C2": 2, "C3": 3, "C4": 4, "C5": 5}
WEIGHT_SEED_OFFSET = 100

CFG_C1 = dict(sphere_channels=16, lmax=2, mmax=2, num_layers=2, hidden_channels=16,
              edge_channels=16, num_distance_basis=8, cutoff=5.0, max_neighbors=20,
              ff_type="grid", norm_type="rms_norm_sh", act_type="gate",
              chg_spin_emb_type="pos_emb", task="omat")
CFG_UMA_S = dict(sphere_channels=128, lmax=2, mmax=2, num_layers=4, hidden_channels=128,
                 edge_channels=128, num_distance_basis=512, cutoff=6.0, max_neighbors=30,
                 ff_type="spectral", norm_type="rms_norm_sh", act_type="gate",
                 chg_spin_emb_type="rand_emb", task="omol")


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


# ------------------------------------------------------------------------------ systems
def _rejection_fill(rng, n, sample, dmin, cell_size):
    """Sequential rejection sampling with a cell list (accept if >= dmin from every atom)."""
    pts = np.empty((n, 3))
    grid = {}
    k = 0
    inv = 1.0 / cell_size
    tries = 0
    while k < n:
        tries += 1
        if tries > 200 * n + 10000:
            raise RuntimeError("rejection sampling did not converge")
        p = sample()
        key = tuple(np.floor(p * inv).astype(int))
        ok = True
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    for j in grid.get((key[0] + dx, key[1] + dy, key[2] + dz), ()):
                        if np.sum((pts[j] - p) ** 2) < dmin * dmin:
                            ok = False
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if not ok:
                break
        if ok:
            pts[k] = p
            grid.setdefault(key, []).append(k)
            k += 1
    return pts


def molecule_in_cube(n, side, dmin, seed):
    rng = _rng(seed)
    Z = rng.choice(ELEMENTS, size=n, p=ELEMENT_P)
    pos = _rejection_fill(rng, n, lambda: rng.uniform(0.0, side, size=3), dmin, max(dmin, 1e-3))
    return pos.astype(np.float32), Z.astype(np.int64)


def c1_system(seed=SEEDS["C1"]):
    """24-atom non-periodic molecule in a 6 A cube, 0.9 A minimum distance."""
    return molecule_in_cube(24, 6.0, 0.9, seed)


def c3_system(seed=SEEDS["C3"], n=2048, radius=17.0, dmin=1.0):
    """2048 atoms uniform in a ball of radius 17 A with 1.0 A rejection."""
    rng = _rng(seed)
    Z = rng.choice(ELEMENTS, size=n, p=ELEMENT_P)

    def sample():
        while True:
            p = rng.uniform(-radius, radius, size=3)
            if p @ p <= radius * radius:
                return p

    pos = _rejection_fill(rng, n, sample, dmin, dmin)
    return pos.astype(np.float32), Z.astype(np.int64)


def c4_system(seed=SEEDS["C4"], reps=8, a=3.61, noise=0.05, Z=29):
    """FCC supercell reps^3 conventional cells (4 atoms each), N(0, noise) displacements."""
    rng = _rng(seed)
    basis = np.array([[0, 0, 0], [0, 0.5, 0.5], [0.5, 0, 0.5], [0.5, 0.5, 0]])
    g = np.stack(np.meshgrid(np.arange(reps), np.arange(reps), np.arange(reps), indexing="ij"), -1)
    frac = (g.reshape(-1, 1, 3) + basis[None]).reshape(-1, 3)
    pos = frac * a + rng.normal(0.0, noise, size=frac.shape)
    cell = np.eye(3) * a * reps
    return pos.astype(np.float32), np.full(len(pos), Z, np.int64), cell.astype(np.float32)


def lattice_cluster(n, spacing=2.2, seed=0):
    """About ``n`` atoms on a jittered cubic lattice (spacing 2.2 A, N(0, 0.55 A) jitter) inside a
    ball, in random index order: a large aperiodic neighbour-list workload (about 75 neighbours
    within 6 A) whose index order carries no spatial locality."""
    rng = np.random.default_rng(seed)
    r = (3.0 * n / (4.0 * np.pi)) ** (1.0 / 3.0) * spacing
    m = int(np.ceil(r / spacing))
    g = np.stack(np.meshgrid(*[np.arange(-m, m + 1)] * 3, indexing="ij"), -1).reshape(-1, 3)
    p = g * spacing + rng.normal(0.0, 0.25 * spacing, g.shape)
    p = p[(p * p).sum(1) <= r * r]
    return p[rng.permutation(p.shape[0])].astype(np.float32)


def shuffled_fcc(reps, seed=0):
    """The C4 FCC supercell (reps^3 conventional cells) with its atoms in random index order:
    (pos, cell)."""
    pos, Z, cell = c4_system(reps=reps)
    perm = np.random.default_rng(seed).permutation(pos.shape[0])
    return pos[perm], cell


def c2_graph(seed=SEEDS["C2"], N=8192, deg=25):
    """Isolated edgewise workload: dst-sorted edges (in-degree ``deg``), uniform random src != dst,
    unit directions with lengths uniform in [0.8, 6] A."""
    rng = _rng(seed)
    tgt = np.repeat(np.arange(N), deg)
    src = rng.integers(0, N - 1, size=N * deg)
    src = src + (src >= tgt)                      # uniform over [0, N) \ {dst}
    d = rng.normal(size=(N * deg, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    vec = d * rng.uniform(0.8, 6.0, size=(N * deg, 1))
    return (np.stack([src, tgt]).astype(np.int64), vec.astype(np.float32))


# ------------------------------------------------------------------------------ weights
def jd_matrices():
    """The fixed Wigner ``J_l`` blocks (l = 0, 1, 2) of the e3nn convention.

    J_1 is the axis-exchange matrix in the (x, y, z) basis of the l = 1 real harmonics; J_2 is
    the same rotation represented on the l = 2 real harmonics
    [sqrt3 xz, sqrt3 xy, y^2 - (x^2+z^2)/2, sqrt3 yz, sqrt3/2 (z^2 - x^2)], obtained by solving
    Y2(J_1 v) = J_2 Y2(v) exactly over a fixed set of directions."""
    J1 = np.array([[0.0, -1.0, 0.0], [-1.0, 0.0, 0.0], [0.0, 0.0, 1.0]])
    s3 = math.sqrt(3.0)

    def y2(v):
        x, y, z = v
        return np.array([s3 * x * z, s3 * x * y, y * y - 0.5 * (x * x + z * z), s3 * y * z,
                         s3 / 2 * (z * z - x * x)])

    V = np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 0], [1, 0, 1], [0, 1, 1], [1, 2, 3],
                  [3, -1, 2], [-2, 1, 1]], dtype=np.float64).T
    S = np.stack([y2(V[:, k]) for k in range(V.shape[1])], 1)
    SR = np.stack([y2(J1 @ V[:, k]) for k in range(V.shape[1])], 1)
    J2 = SR @ np.linalg.pinv(S)
    J2[np.abs(J2) < 1e-12] = 0.0
    return [torch.ones(1, 1), torch.from_numpy(J1).float(), torch.from_numpy(J2).float()]


def to_m_matrix():
    perm = [0, 2, 6, 3, 7, 1, 5, 8, 4]
    m = torch.zeros(9, 9)
    m[torch.arange(9), torch.tensor(perm)] = 1.0
    return m


def gaussian_buffers(nb, cutoff):
    """GaussianSmearing(0, cutoff, nb) with width 2 x spacing: offsets and coefficient."""
    off = torch.linspace(0.0, cutoff, nb)
    coeff = -0.5 / float(2.0 * (off[1] - off[0])) ** 2
    return off, torch.tensor([coeff], dtype=torch.float32)


def random_uma_weights(cfg, seed):
    """Random-init weights of the eSCN-MD architecture in the reference key layout."""
    gen = torch.Generator().manual_seed(int(seed))
    C, H, L = cfg["sphere_channels"], cfg["hidden_channels"], cfg["lmax"]
    ec, nb = cfg["edge_channels"], cfg["num_distance_basis"]
    w = {}

    def lin(name, n_in, n_out, bias=True):
        b = 1.0 / math.sqrt(n_in)
        w[f"{name}.weight"] = (torch.rand(n_out, n_in, generator=gen) * 2 - 1) * b
        if bias:
            w[f"{name}.bias"] = (torch.rand(n_out, generator=gen) * 2 - 1) * b

    def ln(name, n):
        w[f"{name}.weight"] = 1.0 + 0.1 * torch.randn(n, generator=gen)
        w[f"{name}.bias"] = 0.1 * torch.randn(n, generator=gen)

    def radial(p, n_in, n_out):
        lin(f"{p}.net.0", n_in, ec)
        ln(f"{p}.net.1", ec)
        lin(f"{p}.net.3", ec, ec)
        ln(f"{p}.net.4", ec)
        lin(f"{p}.net.6", ec, n_out)

    def norm(p):
        w[f"{p}.affine_weight"] = 1.0 + 0.1 * torch.randn(L + 1, C, generator=gen)
        w[f"{p}.affine_bias"] = 0.1 * torch.randn(C, generator=gen)

    w["sphere_embedding.weight"] = torch.randn(100, C, generator=gen)
    w["source_embedding.weight"] = torch.randn(100, ec, generator=gen)
    w["target_embedding.weight"] = torch.randn(100, ec, generator=gen)
    if cfg.get("chg_spin_emb_type", "pos_emb") == "rand_emb":
        w["charge_embedding.rand_emb.weight"] = torch.randn(201, C, generator=gen)
        w["spin_embedding.rand_emb.weight"] = torch.randn(101, C, generator=gen)
    else:
        w["charge_embedding.W"] = torch.randn(C // 2, generator=gen)
        w["spin_embedding.W"] = torch.randn(C // 2, generator=gen)
    w[f"dataset_embedding.dataset_emb_dict.{cfg.get('task', 'omat')}.weight"] = \
        torch.randn(1, C, generator=gen)
    lin("mix_csd", 3 * C, C)
    for l, J in enumerate(jd_matrices()):
        w[f"Jd_{l}"] = J
    k_in = nb + 2 * ec
    radial("edge_degree_embedding.rad_func", k_in, (L + 1) * C)
    for i in range(cfg["num_layers"]):
        p = f"blocks.{i}"
        norm(f"{p}.norm_1")
        norm(f"{p}.norm_2")
        for c, (cin, hout, extra) in ((1, (2 * C, H, L * H)), (2, (H, C, 0))):
            q = f"{p}.edge_wise.so2_conv_{c}"
            lin(f"{q}.fc_m0", 3 * cin, extra + 3 * hout)
            lin(f"{q}.so2_m_conv.0.fc", 2 * cin, 2 * 2 * hout, bias=False)
            lin(f"{q}.so2_m_conv.1.fc", 1 * cin, 2 * 1 * hout, bias=False)
        radial(f"{p}.edge_wise.so2_conv_1.rad_func", k_in, 6 * 2 * C)
        if cfg.get("ff_type", "grid") == "spectral":
            lin(f"{p}.atom_wise.scalar_mlp.0", C, L * H)
            for n, (ci, co) in (("so3_linear_1", (C, H)), ("so3_linear_2", (H, C))):
                b = 1.0 / math.sqrt(ci)
                w[f"{p}.atom_wise.{n}.weight"] = (torch.rand(L + 1, co, ci, generator=gen) * 2 - 1) * b
                w[f"{p}.atom_wise.{n}.bias"] = (torch.rand(co, generator=gen) * 2 - 1) * b
        else:
            for gi in (0, 2, 4):
                lin(f"{p}.atom_wise.grid_mlp.{gi}", C, C, bias=False)
    norm("norm")
    lin("energy_block.0", C, H)
    lin("energy_block.2", H, H)
    lin("energy_block.4", H, 1)
    return w


def random_uma_bundle(cfg, seed, grid_mats=None):
    """(weights, host buffers) of a random-init bundle.  The grid feed-forward needs the fixed
    S2-grid projection matrices (``grid_mats = (to_grid, from_grid)``)."""
    w = random_uma_weights(cfg, seed)
    off, coeff = gaussian_buffers(cfg["num_distance_basis"], cfg["cutoff"])
    host = dict(to_m=to_m_matrix(), gauss_offset=off, gauss_coeff=coeff)
    if cfg.get("ff_type", "grid") != "spectral":
        if grid_mats is None:
            raise ValueError("the grid feed-forward needs to_grid/from_grid matrices")
        host["to_grid_mat"], host["from_grid_mat"] = grid_mats
    return w, host


def system_embedding_inputs(cfg, charge=0, spin=1):
    return torch.tensor([float(charge)]), torch.tensor([float(spin)])


# ------------------------------------------------------------------------------ Orb-v3
# Orb-v3-conservative architecture (orb_calculator.py:56-65; tools/export_orb_weights.py:49-62):
# 5 attention message-passing layers, latent 256, MLP hidden 1024, 8 Bessel bases x 16 real SH
# (lmax 3) = edge_embed_size 128, cutoff 6 A, cap 20.  ``mlp_hidden_dim`` and
# ``head_hidden_dim`` are parameters here (the reference hard-codes 1024 and the checkpoint's 256)
# so that the CPU parity configuration stays small.
CFG_ORB_C5 = dict(latent_dim=256, num_message_passing_steps=5, edge_embed_size=128,
                  node_embed_size=256, lmax=3, num_bases=8, outer_product_with_cutoff=True,
                  checkpoint="random-init", task="omat", has_charge_spin_cond=False, cutoff=6.0,
                  max_num_neighbors=20, mlp_hidden_dim=1024, head_hidden_dim=256)
CFG_ORB_TINY = dict(CFG_ORB_C5, latent_dim=32, num_message_passing_steps=2, node_embed_size=24,
                    mlp_hidden_dim=48, head_hidden_dim=16)


def c5_systems(seed=SEEDS["C5"], K=256, n_min=20, n_max=60, side=7.0, dmin=0.9):
    """K molecules, sizes uniform in {n_min..n_max}, H/C/N/O, uniform in a ``side`` A cube with
    ``dmin`` rejection; one generator stream for sizes, elements and positions."""
    rng = _rng(seed)
    out = []
    for _ in range(K):
        n = int(rng.integers(n_min, n_max + 1))
        Z = rng.choice(ELEMENTS, size=n, p=ELEMENT_P)
        pos = _rejection_fill(rng, n, lambda: rng.uniform(0.0, side, size=3), dmin, dmin)
        out.append((pos.astype(np.float32), Z.astype(np.int64)))
    return out


def random_orb_weights(cfg, seed, direct=False):
    """Random-init MoleculeGNS weights in the orb-models state-dict key layout
    (tools/export_orb_weights.py:64-80): nn.Linear-style U(-1/sqrt(fan_in), 1/sqrt(fan_in))
    linears, RMSNorm weights 1 + 0.1 N(0,1), N(0,1) atom embeddings, energy-head normaliser and a
    per-element reference energy.  ``direct`` adds the direct checkpoint's force head (3 outputs)
    and stress head (6 outputs) with their normalisers (orb_model.py:358-457), drawn after every
    conservative weight so the shared weights are the same either way."""
    gen = torch.Generator().manual_seed(int(seed))
    C, Hd, He = cfg["latent_dim"], cfg.get("mlp_hidden_dim", 1024), cfg.get("head_hidden_dim", 256)
    w = {}

    def lin(name, n_in, n_out):
        b = 1.0 / math.sqrt(n_in)
        w[f"{name}.weight"] = (torch.rand(n_out, n_in, generator=gen) * 2 - 1) * b
        w[f"{name}.bias"] = (torch.rand(n_out, generator=gen) * 2 - 1) * b

    def mlp_norm(p, n_in):
        lin(f"{p}.mlp.NN-0", n_in, Hd)
        lin(f"{p}.mlp.NN-1", Hd, Hd)
        lin(f"{p}.mlp.NN-2", Hd, C)
        w[f"{p}.layer_norm.weight"] = 1.0 + 0.1 * torch.randn(C, generator=gen)

    w["atom_emb.embeddings.weight"] = torch.randn(119, cfg["node_embed_size"], generator=gen)
    mlp_norm("_encoder._node_fn", cfg["node_embed_size"])
    mlp_norm("_encoder._edge_fn", cfg["edge_embed_size"])
    for i in range(cfg["num_message_passing_steps"]):
        p = f"gnn_stacks.{i}"
        mlp_norm(f"{p}._edge_mlp", 3 * C)
        mlp_norm(f"{p}._node_mlp", 3 * C)
        lin(f"{p}._receive_attn", C, 1)
        lin(f"{p}._send_attn", C, 1)
        if cfg.get("has_charge_spin_cond", False):
            lin(f"{p}._cond_node_proj", C, C)
    if cfg.get("has_charge_spin_cond", False):
        w["conditioner.charge_embedding.W"] = torch.randn(C // 4, generator=gen)
        w["conditioner.spin_embedding.W"] = torch.randn(C // 4, generator=gen)
    lin("energy_head.mlp.NN-0", C, He)
    lin("energy_head.mlp.NN-1", He, 1)
    w["energy_head.normalizer.bn.running_mean"] = torch.tensor(-1.5)
    w["energy_head.normalizer.bn.running_var"] = torch.tensor(2.25)
    w["energy_head.reference.linear.weight"] = -torch.rand(1, 119, generator=gen) * 10.0
    if direct:
        lin("forces_head.mlp.NN-0", C, He)
        lin("forces_head.mlp.NN-1", He, 3)
        w["forces_head.normalizer.bn.running_mean"] = torch.tensor(0.02)
        w["forces_head.normalizer.bn.running_var"] = torch.tensor(0.64)
        lin("stress_head.mlp.NN-0", C, He)
        lin("stress_head.mlp.NN-1", He, 6)
        w["stress_head.diag_normalizer.bn.running_mean"] = torch.tensor(-0.003)
        w["stress_head.diag_normalizer.bn.running_var"] = torch.tensor(4e-4)
        w["stress_head.offdiag_normalizer.bn.running_mean"] = torch.tensor(0.001)
        w["stress_head.offdiag_normalizer.bn.running_var"] = torch.tensor(1e-4)
    return w


# ------------------------------------------------------------------------------ small batches
# The reference's small-system throughput legs (scripts/release_gate.py:536-555,
# docs/perf_baselines.json) time evaluate_batch on K rattled copies of CH3CH2OH (G2 geometry) or
# of diamond Si 2x1x1; these are the same inputs built without ASE (rattle = N(0, stdev) per
# coordinate from RandomState(seed), as ase.Atoms.rattle draws it).
ETHANOL_Z = np.array([6, 6, 8, 1, 1, 1, 1, 1, 1], dtype=np.int64)
ETHANOL_POS = np.array([[1.168181, -0.400382, 0.0], [0.0, 0.559462, 0.0],
                        [-1.190083, -0.227669, 0.0], [-1.946623, 0.381525, 0.0],
                        [0.042557, 1.207508, 0.886933], [0.042557, 1.207508, -0.886933],
                        [2.115891, 0.1448, 0.0], [1.128599, -1.037234, 0.885881],
                        [1.128599, -1.037234, -0.885881]])


def _rattled(pos, stdev, seed):
    return (pos + np.random.RandomState(seed).normal(scale=stdev, size=pos.shape)).astype(
        np.float32)


def ethanol_batch(k, stdev=0.08, seed0=10):
    """K rattled ethanol molecules (charge 0, spin 1) as evaluate_batch system dicts."""
    return [dict(positions=_rattled(ETHANOL_POS, stdev, seed0 + i), numbers=ETHANOL_Z.copy(),
                 charge=0.0, spin=1.0) for i in range(k)]


def si_batch(k, a=5.43, stdev=0.08, seed0=10):
    """K rattled diamond-Si 2x1x1 cells (4 atoms, periodic) as evaluate_batch system dicts."""
    h = a / 2.0
    prim = np.array([[0.0, h, h], [h, 0.0, h], [h, h, 0.0]])
    base = np.array([[0.0, 0.0, 0.0], [a / 4, a / 4, a / 4]])
    pos = np.concatenate([base, base + prim[0]])
    cell = np.stack([2 * prim[0], prim[1], prim[2]])
    return [dict(positions=_rattled(pos, stdev, seed0 + i), numbers=np.full(4, 14, np.int64),
                 cell=cell.astype(np.float32), pbc=[True] * 3) for i in range(k)]


# ------------------------------------------------------------------------------ C2
def c2_weights(seed=SEEDS["C2"] + WEIGHT_SEED_OFFSET, C=128, prefix="c2"):
    """SO(2) convolution weights of the isolated edgewise workload, N(0, 1/sqrt(fan_in)), m = 0
    bias 0, in the reference key layout: fc_m0 [3C, 3C], so2_m_conv.0.fc [4C, 2C],
    so2_m_conv.1.fc [2C, C] (torch [out, in])."""
    gen = torch.Generator().manual_seed(int(seed))
    w = {}
    for name, (n_out, n_in) in (("fc_m0", (3 * C, 3 * C)), ("so2_m_conv.0.fc", (4 * C, 2 * C)),
                                ("so2_m_conv.1.fc", (2 * C, C))):
        w[f"{prefix}.{name}.weight"] = torch.randn(n_out, n_in, generator=gen) / math.sqrt(n_in)
    w[f"{prefix}.fc_m0.bias"] = torch.zeros(3 * C)
    return w


def c2_tensors(seed=SEEDS["C2"], N=8192, deg=25, C=128):
    """(edge_index [2, E], edge vectors [E, 3], node features [N, 9, C] ~ N(0,1), upstream adjoint
    of the scattered output [N, 9, C] ~ N(0,1)); the graph from ``c2_graph(seed)``, the features
    from the generator seeded ``seed + 1``."""
    ei, vec = c2_graph(seed, N, deg)
    rng = _rng(seed + 1)
    x = rng.standard_normal((N, 9, C)).astype(np.float32)
    g = rng.standard_normal((N, 9, C)).astype(np.float32)
    return ei, vec, x, g
