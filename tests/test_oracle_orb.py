"""Pins of the Orb-v3 CPU oracle (oracle/orb.py): reference-written geometry vectors, closed
forms of the Bessel / spherical-harmonic / cutoff functions, and invariants of the backbone."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import orb as O
from tt_atom import synthetic as S

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def geo():
    return {k: torch.from_numpy(v) for k, v in
            np.load(os.path.join(HERE, "golden", "orb_geometry_small.npz")).items()}


def test_sh_bessel_envelope_match_reference_vectors(geo):
    torch.testing.assert_close(O.sph_l3(geo["units"]), geo["sh"], rtol=0, atol=1e-13)
    torch.testing.assert_close(O.bessel(geo["r"]), geo["bessel"], rtol=0, atol=1e-13)
    torch.testing.assert_close(O.envelope(geo["r"])[:, None], geo["envelope"], rtol=0, atol=1e-13)


def test_edge_features_and_force_vjp_match_reference_vectors(geo):
    pos = geo["pos"].clone().requires_grad_(True)
    feat, cut, vec = O.edge_features(pos, geo["senders"], geo["receivers"], geo["shift"])
    torch.testing.assert_close(feat, geo["edge_feat"], rtol=0, atol=1e-12)
    torch.testing.assert_close(cut, geo["cutoff"], rtol=0, atol=1e-13)
    torch.testing.assert_close(vec, geo["vectors"], rtol=0, atol=1e-13)
    # the reference's closed-form VJP (orb_geometry.py:100-139) == autograd of the oracle
    g = torch.autograd.grad([feat, cut], pos, grad_outputs=[geo["g_edge"], geo["g_cutoff"]])[0]
    torch.testing.assert_close(-g, geo["forces"], rtol=2e-12, atol=2e-12)


def _sphere_quadrature(n=8):
    """Gauss-Legendre in cos(theta) x uniform phi: exact for polynomials of degree < 2n."""
    ct, wt = np.polynomial.legendre.leggauss(n)
    phi = np.arange(2 * n) * (2 * math.pi / (2 * n))
    st = np.sqrt(1 - ct ** 2)
    u = np.stack([np.outer(st, np.cos(phi)), np.outer(st, np.sin(phi)),
                  np.outer(ct, np.ones_like(phi))], -1).reshape(-1, 3)
    w = np.outer(wt, np.full(2 * n, 1.0 / (2 * n))).reshape(-1) / 2.0   # mean over the sphere
    return torch.from_numpy(u), torch.from_numpy(w)


def test_sh_closed_forms():
    u, w = _sphere_quadrature()
    Y = O.sph_l3(u)
    # component normalisation: mean over the sphere of Y_a Y_b = delta_ab
    gram = (Y * w[:, None]).T @ Y
    torch.testing.assert_close(gram, torch.eye(16, dtype=torch.float64), rtol=0, atol=1e-12)
    # sum_m Y_lm(u)^2 = 2l + 1 at every point
    for l, (a, b) in enumerate(((0, 1), (1, 4), (4, 9), (9, 16))):
        s = (Y[:, a:b] ** 2).sum(1)
        torch.testing.assert_close(s, torch.full_like(s, 2 * l + 1.0), rtol=0, atol=1e-12)
    # r^l Y_lm(x / r) is a harmonic polynomial: zero Laplacian (central differences, fp64)
    x0 = torch.tensor([[0.3, -0.7, 0.5], [1.1, 0.2, -0.4]], dtype=torch.float64)
    ls = torch.tensor([0] + [1] * 3 + [2] * 5 + [3] * 7, dtype=torch.float64)

    def P(x):
        r = torch.linalg.norm(x, dim=1, keepdim=True)
        return O.sph_l3(x / r) * r ** ls

    h = 1e-3
    lap = -6.0 * P(x0)
    for k in range(3):
        d = torch.zeros(3, dtype=torch.float64)
        d[k] = h
        lap = lap + P(x0 + d) + P(x0 - d)
    assert (lap / h ** 2).abs().max() < 1e-6


def test_bessel_and_envelope_closed_forms():
    r_max = 6.0
    x, wq = np.polynomial.legendre.leggauss(200)
    r = torch.from_numpy((x + 1) * r_max / 2)
    wr = torch.from_numpy(wq * r_max / 2)
    B = O.bessel(r, r_max, 8)
    gram = (B * (wr * r * r)[:, None]).T @ B          # int_0^rmax b_n b_m r^2 dr = delta
    torch.testing.assert_close(gram, torch.eye(8, dtype=torch.float64), rtol=0, atol=1e-10)
    rr = torch.tensor([1e-9, r_max * (1 - 1e-12)], dtype=torch.float64, requires_grad=True)
    env = O.envelope(rr, r_max)
    d1 = torch.autograd.grad(env.sum(), rr, create_graph=True)[0]
    d2 = torch.autograd.grad(d1.sum(), rr)[0]
    assert abs(env[0].item() - 1) < 1e-12 and abs(env[1].item()) < 1e-10
    assert abs(d1[0].item()) < 1e-12 and abs(d1[1].item()) < 1e-9 and abs(d2[1].item()) < 1e-8
    assert O.envelope(torch.tensor([r_max, 7.0], dtype=torch.float64)).abs().max() == 0


def _tiny(K=3, seed=11, cond=False):
    cfg = dict(S.CFG_ORB_TINY, has_charge_spin_cond=cond)
    w = S.random_orb_weights(cfg, seed + S.WEIGHT_SEED_OFFSET)
    systems = [(torch.from_numpy(p).double(), torch.from_numpy(z))
               for p, z in S.c5_systems(seed, K=K, n_min=6, n_max=12, side=5.0)]
    bg = O.assemble(systems, cfg["cutoff"], cfg["max_num_neighbors"])
    return cfg, w, systems, bg


def _eval(cfg, w, bg, pos=None, **kw):
    return O.energy_and_forces(w, cfg, bg["pos"] if pos is None else pos, bg["Z"], bg["senders"],
                               bg["receivers"], bg["shift"], bg["batch"], bg["natoms"], **kw)


def test_backbone_forces_match_finite_differences():
    cfg, w, _, bg = _tiny(K=2)
    raw, F = _eval(cfg, w, bg)
    pos = bg["pos"]
    h = 1e-5
    for (a, k) in ((0, 0), (3, 1), (pos.shape[0] - 1, 2)):
        p1, p2 = pos.clone(), pos.clone()
        p1[a, k] += h
        p2[a, k] -= h
        e1 = _eval(cfg, w, bg, p1)[0].sum()
        e2 = _eval(cfg, w, bg, p2)[0].sum()
        assert abs(-(e1 - e2) / (2 * h) - F[a, k]) < 1e-7 * max(1.0, abs(F[a, k].item()))


def test_backbone_stress_matches_finite_differences():
    cfg, w, _, bg = _tiny(K=1)
    raw, F, vir = _eval(cfg, w, bg, compute_stress=True)
    torch.testing.assert_close(vir, vir.T, rtol=0, atol=1e-12)
    h = 1e-6
    for (i, j) in ((0, 0), (1, 2)):
        eps = torch.zeros(3, 3, dtype=torch.float64)
        eps[i, j] = eps[j, i] = h
        e1 = _eval(cfg, w, bg, bg["pos"] @ (torch.eye(3, dtype=torch.float64) + eps))[0].sum()
        e2 = _eval(cfg, w, bg, bg["pos"] @ (torch.eye(3, dtype=torch.float64) - eps))[0].sum()
        fd = (e1 - e2) / (2 * h) / (1 if i == j else 2)
        assert abs(fd - vir[i, j]) < 1e-6 * max(1.0, abs(vir[i, j].item()))


def test_backbone_invariances_and_batching():
    cfg, w, systems, bg = _tiny(K=3, cond=True)
    cond = torch.cat([O.charge_spin_embedding(w, q, s, n) for q, s, n in
                      ((0, 1, bg["natoms"][0]), (1, 2, bg["natoms"][1]), (-1, 0, bg["natoms"][2]))])
    raw, F = _eval(cfg, w, bg, cond_nodes=cond)
    # translation invariance; forces sum to zero per system
    raw2, F2 = _eval(cfg, w, bg, bg["pos"] + torch.tensor([0.7, -1.3, 2.1], dtype=torch.float64),
                     cond_nodes=cond)
    torch.testing.assert_close(raw2, raw, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(F2, F, rtol=1e-10, atol=1e-10)
    for k in range(3):
        assert F[bg["batch"] == k].sum(0).abs().max() < 1e-10
    # the disjoint union gives each system its own energy and forces
    off = 0
    for k, (p, z) in enumerate(systems):
        one = O.assemble([(p, z)], cfg["cutoff"], cfg["max_num_neighbors"])
        n = z.shape[0]
        rk, Fk = _eval(cfg, w, one, cond_nodes=cond[off:off + n])
        torch.testing.assert_close(rk[0], raw[k], rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(Fk, F[off:off + n], rtol=1e-10, atol=1e-10)
        off += n
    # relabelling atoms (and hence edges) leaves energies unchanged
    perm = torch.randperm(bg["pos"].shape[0], generator=torch.Generator().manual_seed(0))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    raw3, F3 = O.energy_and_forces(w, cfg, bg["pos"][perm], bg["Z"][perm], inv[bg["senders"]],
                                   inv[bg["receivers"]], bg["shift"], bg["batch"][perm],
                                   bg["natoms"], cond_nodes=cond[perm])
    torch.testing.assert_close(raw3, raw, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(F3, F[perm], rtol=1e-10, atol=1e-10)


def test_segment_sums_match_dense_products():
    cfg, w, _, bg = _tiny(K=2)
    N, E = bg["pos"].shape[0], bg["senders"].numel()
    x = torch.randn(E, 5, dtype=torch.float64)
    S_send = torch.zeros(N, E, dtype=torch.float64)
    S_send[bg["senders"], torch.arange(E)] = 1
    ref = torch.zeros(N, 5, dtype=torch.float64).index_add_(0, bg["senders"], x)
    torch.testing.assert_close(S_send @ x, ref, rtol=0, atol=1e-13)


def test_assemble_cap_and_convention():
    cfg, w, systems, bg = _tiny(K=2)
    # senders are the neighbour list's receivers (tgt): each sender keeps <= cap neighbours
    assert torch.bincount(bg["senders"]).max() <= cfg["max_num_neighbors"]
    assert int(bg["batch"][bg["senders"]].ne(bg["batch"][bg["receivers"]]).sum()) == 0
    v = bg["pos"][bg["receivers"]] - bg["pos"][bg["senders"]]
    assert (torch.linalg.norm(v, dim=1) < cfg["cutoff"]).all()


def test_direct_heads_invariants_and_batching():
    """Direct checkpoint (ForceHead / StressHead): per-system net force zero, the shared weights
    and energy equal to the conservative draw, batch == per-system (which a whole-batch mean
    removal would break: the systems' mean predictions differ), atom relabelling permutes forces
    and leaves energies and stress unchanged."""
    seed = 11
    cfg = dict(S.CFG_ORB_TINY)
    w = S.random_orb_weights(cfg, seed + S.WEIGHT_SEED_OFFSET, direct=True)
    wc = S.random_orb_weights(cfg, seed + S.WEIGHT_SEED_OFFSET)
    assert all(torch.equal(wc[k], w[k]) for k in wc)
    systems = [(torch.from_numpy(p).double(), torch.from_numpy(z))
               for p, z in S.c5_systems(seed, K=3, n_min=6, n_max=12, side=5.0)]
    bg = O.assemble(systems, cfg["cutoff"], cfg["max_num_neighbors"])
    args = (bg["pos"], bg["Z"], bg["senders"], bg["receivers"], bg["shift"], bg["batch"],
            bg["natoms"])
    e, f, s = O.direct_forward(w, cfg, *args, compute_stress=True)
    assert f.shape == (bg["pos"].shape[0], 3) and s.shape == (3, 6)
    torch.testing.assert_close(e, _eval(cfg, wc, bg)[0], rtol=1e-12, atol=1e-12)
    for k in range(3):
        assert f[bg["batch"] == k].sum(0).abs().max() < 1e-12
    assert f.abs().max() > 1e-3 and s.abs().max() > 1e-3
    # the systems' mean raw predictions differ, so a whole-batch mean would change the forces
    wd = {k: v.double() for k, v in w.items()}
    feat, cut, _ = O.edge_features(bg["pos"], bg["senders"], bg["receivers"], bg["shift"],
                                   cfg["cutoff"], cfg["num_bases"])
    nodes = O.node_embedding(wd, cfg, bg["Z"], feat, cut, bg["senders"], bg["receivers"])
    pred = O._lin(torch.nn.functional.silu(O._lin(nodes, wd, "forces_head.mlp.NN-0")), wd,
                  "forces_head.mlp.NN-1")
    means = torch.stack([pred[bg["batch"] == k].mean(0) for k in range(3)])
    assert (means[0] - means[1]).abs().max() > 1e-4 and (means[1] - means[2]).abs().max() > 1e-4
    # batch == per system
    off = 0
    for k, (p, z) in enumerate(systems):
        one = O.assemble([(p, z)], cfg["cutoff"], cfg["max_num_neighbors"])
        ek, fk, sk = O.direct_forward(w, cfg, one["pos"], one["Z"], one["senders"],
                                      one["receivers"], one["shift"], one["batch"], one["natoms"],
                                      compute_stress=True)
        n = z.shape[0]
        torch.testing.assert_close(ek[0], e[k], rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(fk, f[off:off + n], rtol=1e-10, atol=1e-12)
        torch.testing.assert_close(sk[0], s[k], rtol=1e-10, atol=1e-12)
        off += n
    # relabelling atoms
    perm = torch.randperm(bg["pos"].shape[0], generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    e3, f3, s3 = O.direct_forward(w, cfg, bg["pos"][perm], bg["Z"][perm], inv[bg["senders"]],
                                  inv[bg["receivers"]], bg["shift"], bg["batch"][perm],
                                  bg["natoms"], compute_stress=True)
    torch.testing.assert_close(e3, e, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(f3, f[perm], rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(s3, s, rtol=1e-10, atol=1e-12)


def test_direct_denormalisers_known_values():
    """x sigma + mu with sigma = sqrt(var); the stress's first three components take the diagonal
    normaliser and the last three the off-diagonal one (distinct values catch a swap)."""
    f = O.denormalize_direct_forces(torch.tensor([[1.0, -2.0, 0.0]]), torch.tensor(0.5),
                                    torch.tensor(0.25))
    torch.testing.assert_close(f, torch.tensor([[1.0, -0.5, 0.5]], dtype=torch.float64))
    s = O.denormalize_direct_stress(torch.tensor([1.0, 2.0, 3.0, 1.0, 2.0, 3.0]),
                                    torch.tensor(0.1), torch.tensor(4.0),
                                    torch.tensor(-1.0), torch.tensor(9.0))
    torch.testing.assert_close(s, torch.tensor([2.1, 4.1, 6.1, 2.0, 5.0, 8.0],
                                               dtype=torch.float64))
