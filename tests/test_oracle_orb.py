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


# ----------------------------------------------------------------------------- known answers
# Weights that reduce each module to a closed form, with the expected values computed by explicit
# loops over the edge list from the reference's statement of the layer (orb_model.py:225-266,
# 127-173, 92-112, 329-355, 381-435).  Every Linear is a scaled permutation-selection matrix in
# torch [out, in] layout (F.linear(x, W)[i] = sum_j W[i, j] x[j] = scale[i] * x[off + perm[i]]),
# non-symmetric so a transposed weight changes the answer; RMSNorm weights are non-uniform so a
# weight applied before the normalisation changes it.
_SILU = lambda v: v / (1.0 + math.exp(-v))
_SIG = lambda v: 1.0 / (1.0 + math.exp(-v))


def _sel(n_out, n_in, off, perm, scale):
    W = torch.zeros(n_out, n_in, dtype=torch.float64)
    for i in range(n_out):
        W[i, off + perm[i]] = scale[i]
    return W


_P0, _P1, _P2 = [1, 2, 3, 0], [3, 0, 1, 2], [2, 3, 0, 1]
_S0, _S1, _S2 = [1.0, -0.5, 2.0, 0.7], [1.3, 2.0, 0.5, -1.0], [0.8, -1.2, 1.5, 0.4]
_B0, _B1, _B2 = [0.1, -0.2, 0.3, 0.0], [0.05, 0.0, -0.15, 0.2], [0.3, -0.1, 0.0, 0.25]
_LN = [1.0, 2.0, 0.5, 3.0]


def _mlpnorm_weights(w, prefix, n_in, off, ln):
    w[f"{prefix}.mlp.NN-0.weight"] = _sel(4, n_in, off, _P0, _S0)
    w[f"{prefix}.mlp.NN-0.bias"] = torch.tensor(_B0, dtype=torch.float64)
    w[f"{prefix}.mlp.NN-1.weight"] = _sel(4, 4, 0, _P1, _S1)
    w[f"{prefix}.mlp.NN-1.bias"] = torch.tensor(_B1, dtype=torch.float64)
    w[f"{prefix}.mlp.NN-2.weight"] = _sel(4, 4, 0, _P2, _S2)
    w[f"{prefix}.mlp.NN-2.bias"] = torch.tensor(_B2, dtype=torch.float64)
    w[f"{prefix}.layer_norm.weight"] = torch.tensor(ln, dtype=torch.float64)


def _mlpnorm_expected(v, ln):
    """Linear-SiLU-Linear-SiLU-Linear then x * rsqrt(mean(x^2) + 1e-6) * w, for the selection
    weights of _mlpnorm_weights, on one input block v (4 values)."""
    h0 = [_SILU(_S0[i] * v[_P0[i]] + _B0[i]) for i in range(4)]
    h1 = [_SILU(_S1[i] * h0[_P1[i]] + _B1[i]) for i in range(4)]
    h2 = [_S2[i] * h1[_P2[i]] + _B2[i] for i in range(4)]
    inv = 1.0 / math.sqrt(sum(t * t for t in h2) / 4 + 1e-6)
    return [h2[i] * inv * ln[i] for i in range(4)]


_SEND, _RECV = [0, 0, 0, 1, 2], [1, 2, 3, 3, 3]       # sender degrees 3,1,1,0; receiver 0,1,1,3
_CUT = [1.0, 0.5, 0.25, 0.8, 0.6]
_GR, _BR, _GS, _BS = 0.9, 0.3, -1.4, -1.1              # attention weight on channel 0 / 1, bias
_LN_NODE = [0.5, 1.5, 2.5, -1.0]


def _layer_case(edge_block, node_block, cond):
    """One attention layer (C = hidden = 4) whose edge MLP reads only input block `edge_block`
    of [e | n[send] | n[recv]] and whose node MLP reads only block `node_block` of
    [n | recv_agg | sent_agg]; returns (oracle (nodes, edges), expected (nodes, edges))."""
    N, E, C = 4, 5, 4
    nodes = torch.tensor([[0.3 * i - 0.2 * j + 0.05 * i * j for j in range(C)] for i in range(N)],
                         dtype=torch.float64)
    edges = torch.tensor([[0.1 * (e + 1) * (-1) ** j + 0.07 * j for j in range(C)]
                          for e in range(E)], dtype=torch.float64)
    p = "gnn_stacks.0"
    w = {}
    _mlpnorm_weights(w, f"{p}._edge_mlp", 3 * C, edge_block * C, _LN)
    _mlpnorm_weights(w, f"{p}._node_mlp", 3 * C, node_block * C, _LN_NODE)
    w[f"{p}._receive_attn.weight"] = torch.tensor([[_GR, 0.0, 0.0, 0.0]], dtype=torch.float64)
    w[f"{p}._receive_attn.bias"] = torch.tensor([_BR], dtype=torch.float64)
    w[f"{p}._send_attn.weight"] = torch.tensor([[0.0, _GS, 0.0, 0.0]], dtype=torch.float64)
    w[f"{p}._send_attn.bias"] = torch.tensor([_BS], dtype=torch.float64)
    cond_nodes = None
    n_eff = [list(map(float, r)) for r in nodes]
    if cond:
        cond_nodes = torch.tensor([[0.2 * i + 0.1 * j for j in range(6)] for i in range(N)],
                                  dtype=torch.float64)
        w[f"{p}._cond_node_proj.weight"] = _sel(C, 6, 2, [3, 0, 2, 1], [1.0, -2.0, 0.5, 1.5])
        w[f"{p}._cond_node_proj.bias"] = torch.tensor([0.01, 0.02, -0.03, 0.04],
                                                      dtype=torch.float64)
        cp = [3, 0, 2, 1]
        cs = [1.0, -2.0, 0.5, 1.5]
        cb = [0.01, 0.02, -0.03, 0.04]
        n_eff = [[n_eff[i][j] + cs[j] * float(cond_nodes[i, 2 + cp[j]]) + cb[j] for j in range(C)]
                 for i in range(N)]
    got = O.attention_layer(nodes, edges, torch.tensor(_SEND), torch.tensor(_RECV),
                            torch.tensor(_CUT, dtype=torch.float64)[:, None], w, p, cond_nodes)
    # expected, edge by edge
    ue = []
    for e in range(E):
        block = [list(map(float, edges[e])), n_eff[_SEND[e]], n_eff[_RECV[e]]][edge_block]
        ue.append(_mlpnorm_expected(block, _LN))
    sent = [[0.0] * C for _ in range(N)]
    recv = [[0.0] * C for _ in range(N)]
    for e in range(E):
        sa = _SIG(_GS * float(edges[e, 1]) + _BS) * _CUT[e]
        ra = _SIG(_GR * float(edges[e, 0]) + _BR) * _CUT[e]
        for j in range(C):
            sent[_SEND[e]][j] += ue[e][j] * sa
            recv[_RECV[e]][j] += ue[e][j] * ra
    new_nodes = []
    for i in range(N):
        block = [n_eff[i], recv[i], sent[i]][node_block]
        un = _mlpnorm_expected(block, _LN_NODE)
        new_nodes.append([n_eff[i][j] + un[j] for j in range(C)])
    new_edges = [[float(edges[e, j]) + ue[e][j] for j in range(C)] for e in range(E)]
    return got, (torch.tensor(new_nodes, dtype=torch.float64),
                 torch.tensor(new_edges, dtype=torch.float64))


@pytest.mark.parametrize("cond", [False, True])
@pytest.mark.parametrize("edge_block,node_block", [(j, k) for j in range(3) for k in range(3)])
def test_attention_layer_known_answers(edge_block, node_block, cond):
    """Edge MLP input [e | n[send] | n[recv]], attention gates sigmoid(e W + b) * cutoff from the
    pre-update edges, sent_agg summed over each node's outgoing (sender) edges and recv_agg over
    its incoming (receiver) edges, node MLP input [n | recv_agg | sent_agg], the conditioning
    projection added to the nodes before everything else, residuals on both: against the closed
    form for every choice of the block each MLP reads.  A swap of the two sums, of the blocks of
    either concatenation, of the gate channels or a misplaced RMSNorm weight fails here (the
    sender and receiver degrees of the graph all differ)."""
    (nodes, edges), (ref_nodes, ref_edges) = _layer_case(edge_block, node_block, cond)
    torch.testing.assert_close(edges, ref_edges, rtol=0, atol=1e-12)
    torch.testing.assert_close(nodes, ref_nodes, rtol=0, atol=1e-12)


def test_mlpnorm_rmsnorm_known_answer():
    """MLPNorm on one row against hand-evaluated numbers (not only the closed-form helper): the
    RMSNorm eps is 1e-6 inside the square root and the weight multiplies after normalising."""
    w = {}
    _mlpnorm_weights(w, "m", 4, 0, _LN)
    x = torch.tensor([[0.4, -0.3, 1.2, 0.05]], dtype=torch.float64)
    got = O.mlp_norm(x, w, "m")[0]
    h0 = [_SILU(1.0 * -0.3 + 0.1), _SILU(-0.5 * 1.2 - 0.2), _SILU(2.0 * 0.05 + 0.3),
          _SILU(0.7 * 0.4 + 0.0)]
    h1 = [_SILU(1.3 * h0[3] + 0.05), _SILU(2.0 * h0[0]), _SILU(0.5 * h0[1] - 0.15),
          _SILU(-1.0 * h0[2] + 0.2)]
    h2 = [0.8 * h1[2] + 0.3, -1.2 * h1[3] - 0.1, 1.5 * h1[0], 0.4 * h1[1] + 0.25]
    rms = math.sqrt((h2[0] ** 2 + h2[1] ** 2 + h2[2] ** 2 + h2[3] ** 2) / 4 + 1e-6)
    ref = torch.tensor([h2[0] / rms * 1.0, h2[1] / rms * 2.0, h2[2] / rms * 0.5,
                        h2[3] / rms * 3.0], dtype=torch.float64)
    torch.testing.assert_close(got, ref, rtol=0, atol=1e-14)


def _head_weights(name, n_out, scale_out, bias_out):
    w = {f"{name}.mlp.NN-0.weight": _sel(3, 4, 0, [2, 0, 3], [1.5, -0.8, 0.6]),
         f"{name}.mlp.NN-0.bias": torch.tensor([0.1, -0.2, 0.05], dtype=torch.float64),
         f"{name}.mlp.NN-1.weight": torch.tensor(scale_out, dtype=torch.float64).reshape(n_out, 3),
         f"{name}.mlp.NN-1.bias": torch.tensor(bias_out, dtype=torch.float64)}
    return w


_HEAD_NODES = torch.tensor([[0.5, -1.0, 0.25, 2.0], [1.5, 0.0, -0.75, 1.0],
                            [-0.2, 0.4, 1.1, -0.6], [0.9, 0.3, -1.3, 0.2],
                            [0.0, 1.2, 0.8, -0.4]], dtype=torch.float64)
_HEAD_BATCH, _HEAD_NATOMS = torch.tensor([0, 0, 1, 1, 1]), [2, 3]


def _head_hidden(row):
    return [_SILU(1.5 * row[2] + 0.1), _SILU(-0.8 * row[0] - 0.2), _SILU(0.6 * row[3] + 0.05)]


def _sys_means():
    out = []
    off = 0
    for n in _HEAD_NATOMS:
        out.append([sum(float(_HEAD_NODES[off + a, j]) for a in range(n)) / n for j in range(4)])
        off += n
    return out


def test_energy_head_known_answer_per_system():
    """EnergyHead(.batch): mean of each system's own node features, then Linear-SiLU-Linear
    (orb_model.py:329-355); a batch-wide mean would give both systems one value."""
    wo = [0.7, -1.3, 0.4]
    w = _head_weights("energy_head", 1, wo, [0.2])
    got = O.energy_head(_HEAD_NODES, _HEAD_BATCH, _HEAD_NATOMS, w)
    ref = [sum(wo[i] * h for i, h in enumerate(_head_hidden(m))) + 0.2 for m in _sys_means()]
    torch.testing.assert_close(got, torch.tensor(ref, dtype=torch.float64), rtol=0, atol=1e-14)
    assert abs(ref[0] - ref[1]) > 0.1


def test_force_and_stress_heads_known_answers_per_system():
    """ForceHead.batch: per-node Linear-SiLU-Linear, minus the mean prediction of the node's own
    system (orb_model.py:381-404); StressHead: per-system node mean, then Linear-SiLU-Linear to
    six Voigt components (orb_model.py:429-435)."""
    wf = [1.0, 0.5, -0.3, -0.7, 0.2, 1.1, 0.4, -1.5, 0.9]
    w = _head_weights("forces_head", 3, wf, [0.3, -0.1, 0.2])
    got = O.force_head(_HEAD_NODES, _HEAD_BATCH, _HEAD_NATOMS, w)
    pred = []
    for a in range(5):
        h = _head_hidden([float(v) for v in _HEAD_NODES[a]])
        pred.append([sum(wf[3 * c + i] * h[i] for i in range(3)) + [0.3, -0.1, 0.2][c]
                     for c in range(3)])
    ref, off = [], 0
    for n in _HEAD_NATOMS:
        mean = [sum(pred[off + a][c] for a in range(n)) / n for c in range(3)]
        ref += [[pred[off + a][c] - mean[c] for c in range(3)] for a in range(n)]
        off += n
    torch.testing.assert_close(got, torch.tensor(ref, dtype=torch.float64), rtol=0, atol=1e-14)
    ws = [0.1 * (k + 1) * (-1) ** k for k in range(18)]
    bs = [0.01 * k for k in range(6)]
    w = _head_weights("stress_head", 6, ws, bs)
    got = O.stress_head(_HEAD_NODES, _HEAD_BATCH, _HEAD_NATOMS, w)
    ref = []
    for m in _sys_means():
        h = _head_hidden(m)
        ref.append([sum(ws[3 * c + i] * h[i] for i in range(3)) + bs[c] for c in range(6)])
    torch.testing.assert_close(got, torch.tensor(ref, dtype=torch.float64), rtol=0, atol=1e-14)


def test_backbone_composition_known_answer():
    """Encoder then layers then the energy head (orb_model.py:176-186, gns stacks in order): a
    two-layer stack whose first layer's MLPs read blocks (n[send], recv_agg) and second (e,
    sent_agg), composed by hand from the layer closed form, with the encoder MLPs on the atom
    embedding and the edge features."""
    C = 4
    Z = torch.tensor([1, 6, 8, 6])
    emb = torch.tensor([[0.1 * z - 0.05 * j for j in range(C)] for z in range(10)],
                       dtype=torch.float64)
    feat = torch.tensor([[0.2 * e - 0.1 * j + 0.03 * e * j for j in range(C)] for e in range(5)],
                        dtype=torch.float64)
    w = {"atom_emb.embeddings.weight": emb}
    _mlpnorm_weights(w, "_encoder._node_fn", C, 0, [1.0, 0.5, 2.0, 1.5])
    _mlpnorm_weights(w, "_encoder._edge_fn", C, 0, [0.7, 1.0, 1.3, 0.9])
    for li, (eb, nb) in enumerate(((1, 1), (0, 2))):
        p = f"gnn_stacks.{li}"
        _mlpnorm_weights(w, f"{p}._edge_mlp", 3 * C, eb * C, _LN)
        _mlpnorm_weights(w, f"{p}._node_mlp", 3 * C, nb * C, _LN_NODE)
        w[f"{p}._receive_attn.weight"] = torch.tensor([[_GR, 0, 0, 0]], dtype=torch.float64)
        w[f"{p}._receive_attn.bias"] = torch.tensor([_BR], dtype=torch.float64)
        w[f"{p}._send_attn.weight"] = torch.tensor([[0, _GS, 0, 0]], dtype=torch.float64)
        w[f"{p}._send_attn.bias"] = torch.tensor([_BS], dtype=torch.float64)
    w.update(_head_weights("energy_head", 1, [0.7, -1.3, 0.4], [0.2]))
    cfg = {"num_message_passing_steps": 2}
    cut = torch.tensor(_CUT, dtype=torch.float64)[:, None]
    s, r = torch.tensor(_SEND), torch.tensor(_RECV)
    got = O.backbone(w, cfg, Z, feat, cut, s, r, torch.zeros(4, dtype=torch.long), [4])
    # by hand: encoder rows, then the two layers through the layer closed form of the test above
    nodes = [_mlpnorm_expected([float(v) for v in emb[z]], [1.0, 0.5, 2.0, 1.5]) for z in Z]
    edges = [_mlpnorm_expected([float(v) for v in feat[e]], [0.7, 1.0, 1.3, 0.9])
             for e in range(5)]
    for eb, nb in ((1, 1), (0, 2)):
        ue = [_mlpnorm_expected([edges[e], nodes[_SEND[e]], nodes[_RECV[e]]][eb], _LN)
              for e in range(5)]
        sent = [[0.0] * C for _ in range(4)]
        recv = [[0.0] * C for _ in range(4)]
        for e in range(5):
            sa = _SIG(_GS * edges[e][1] + _BS) * _CUT[e]
            ra = _SIG(_GR * edges[e][0] + _BR) * _CUT[e]
            for j in range(C):
                sent[_SEND[e]][j] += ue[e][j] * sa
                recv[_RECV[e]][j] += ue[e][j] * ra
        un = [_mlpnorm_expected([nodes[i], recv[i], sent[i]][nb], _LN_NODE) for i in range(4)]
        nodes = [[nodes[i][j] + un[i][j] for j in range(C)] for i in range(4)]
        edges = [[edges[e][j] + ue[e][j] for j in range(C)] for e in range(5)]
    mean = [sum(nodes[i][j] for i in range(4)) / 4 for j in range(C)]
    ref = sum(c * h for c, h in zip([0.7, -1.3, 0.4], _head_hidden(mean))) + 0.2
    assert abs(float(got[0]) - ref) < 1e-12, (float(got[0]), ref)


def test_known_answer_tests_catch_planted_wiring_mistakes(monkeypatch):
    """The layer closed form above is sensitive to each plausible wiring mistake: planted into a
    copy of the oracle's layer, each one fails the known-answer comparison."""
    import torch.nn.functional as F

    def layer(mistake):
        def f(nodes, edges, senders, receivers, cut, w, prefix, cond_nodes=None):
            N = nodes.shape[0]
            if cond_nodes is not None and f"{prefix}._cond_node_proj.weight" in w:
                nodes = nodes + O._lin(cond_nodes, w, f"{prefix}._cond_node_proj")
            ra = torch.sigmoid(O._lin(edges, w, f"{prefix}._receive_attn")) * cut
            sa = torch.sigmoid(O._lin(edges, w, f"{prefix}._send_attn")) * cut
            if mistake == "gates":
                ra, sa = sa, ra
            cat = [edges, nodes[senders], nodes[receivers]]
            if mistake == "edge_order":
                cat = [edges, nodes[receivers], nodes[senders]]
            ue = O.mlp_norm(torch.cat(cat, dim=1), w, f"{prefix}._edge_mlp")
            if mistake == "norm_weight":
                h = torch.cat(cat, dim=1)
                for i in range(2):
                    h = F.silu(O._lin(h, w, f"{prefix}._edge_mlp.mlp.NN-{i}"))
                h = O._lin(h, w, f"{prefix}._edge_mlp.mlp.NN-2")
                ue = O.rmsnorm(h * w[f"{prefix}._edge_mlp.layer_norm.weight"],
                               torch.ones_like(w[f"{prefix}._edge_mlp.layer_norm.weight"]))
            C = ue.shape[1]
            si, ri = (receivers, senders) if mistake == "sums" else (senders, receivers)
            sent = torch.zeros(N, C, dtype=ue.dtype).index_add_(0, si, ue * sa)
            recv = torch.zeros(N, C, dtype=ue.dtype).index_add_(0, ri, ue * ra)
            node_cat = [nodes, sent, recv] if mistake == "node_order" else [nodes, recv, sent]
            un = O.mlp_norm(torch.cat(node_cat, dim=1), w, f"{prefix}._node_mlp")
            return nodes + un, edges + ue
        return f

    for mistake in ("gates", "edge_order", "norm_weight", "sums", "node_order"):
        monkeypatch.setattr(O, "attention_layer", layer(mistake))
        caught = False
        for j in range(3):
            for k in range(3):
                (nodes, edges), (rn, re_) = _layer_case(j, k, False)
                if not (torch.allclose(nodes, rn, rtol=0, atol=1e-12)
                        and torch.allclose(edges, re_, rtol=0, atol=1e-12)):
                    caught = True
        assert caught, mistake


def test_conservative_denormalisers_and_conditioning_known_values():
    """EnergyHead.denormalize: (raw sigma + mu) n + sum ref[Z] (orb_model.py:588-600); the
    conservative force and stress scales sigma n (and / |det cell|) with the Voigt order
    [xx, yy, zz, yz, xz, xy] (orb_model.py:459-488); the sin/cos charge / spin conditioning with
    the spin part zeroed at spin 0 (orb_model.py:32-56).  Oracle and package host functions
    against hand-evaluated numbers."""
    from tt_atom import orb as P
    ref_w = torch.zeros(119, dtype=torch.float64)
    ref_w[1], ref_w[6], ref_w[8] = -0.5, -3.0, -4.25
    Z = torch.tensor([6, 1, 1, 8])
    e = O.denormalize_energy(torch.tensor(0.5), Z, 4, torch.tensor(1.0), torch.tensor(4.0), ref_w)
    assert abs(float(e) - ((0.5 * 2 + 1) * 4 - 3.0 - 0.5 - 0.5 - 4.25)) < 1e-12
    w = {"energy_head.normalizer.bn.running_var": torch.tensor(4.0),
         "energy_head.normalizer.bn.running_mean": torch.tensor(1.0),
         "energy_head.reference.linear.weight": ref_w[None]}
    assert abs(float(P.denormalize_energy(0.5, Z, 4, w)) - float(e)) < 1e-12
    eb = P.denormalize_energy_batch(torch.tensor([0.5, -1.0]), torch.tensor([6, 1, 1, 8, 8]),
                                    torch.tensor([0, 0, 0, 0, 1]), [4, 1], w)
    torch.testing.assert_close(eb, torch.tensor([float(e), (-1.0 * 2 + 1) * 1 - 4.25],
                                                dtype=torch.float64), rtol=0, atol=1e-12)
    f = O.denormalize_forces(torch.tensor([[1.0, -2.0, 0.25]]), 4, torch.tensor(4.0))
    torch.testing.assert_close(f, torch.tensor([[8.0, -16.0, 2.0]], dtype=torch.float64))
    torch.testing.assert_close(P.denormalize_forces(torch.tensor([[1.0, -2.0, 0.25]]), 4, w), f)
    vir = torch.tensor([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0], [7.0, 8.0, 9.0]])
    cell = torch.diag(torch.tensor([2.0, 2.0, 4.0]))                  # volume 16
    s = P.denormalize_stress(vir, 4, cell, w)                         # scale sigma n / V = 0.5
    torch.testing.assert_close(s, torch.tensor([0.5, 2.5, 4.5, 3.5, 2.5, 1.5],
                                               dtype=torch.float64))
    wc = {"conditioner.charge_embedding.W": torch.tensor([0.25, -0.1], dtype=torch.float64),
          "conditioner.spin_embedding.W": torch.tensor([0.5, 0.125], dtype=torch.float64)}
    c = O.charge_spin_embedding(wc, 1.0, 0.0, 2)
    tp = 2 * math.pi
    ref = [math.sin(tp * 0.25), math.sin(-tp * 0.1), math.cos(tp * 0.25), math.cos(-tp * 0.1),
           0.0, 0.0, 0.0, 0.0]
    torch.testing.assert_close(c, torch.tensor([ref, ref], dtype=torch.float64), rtol=0,
                               atol=1e-15)
    c = O.charge_spin_embedding(wc, -2.0, 3.0, 1)
    ref = [math.sin(-2 * tp * 0.25), math.sin(2 * tp * 0.1), math.cos(-2 * tp * 0.25),
           math.cos(2 * tp * 0.1), math.sin(3 * tp * 0.5), math.sin(3 * tp * 0.125),
           math.cos(3 * tp * 0.5), math.cos(3 * tp * 0.125)]
    torch.testing.assert_close(c, torch.tensor([ref], dtype=torch.float64), rtol=0, atol=1e-14)
