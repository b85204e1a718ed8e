"""Pins the CPU oracle (UMA path) against the reference's committed fairchem goldens, closed forms,
invariants and finite differences.  CPU only."""
import math

import numpy as np
import pytest
import torch

from conftest import golden_bufs
from oracle import geometry as G
from oracle import uma
from oracle import forces as OF


def _model(g, ref=None):
    return OF.Model(g.w(), dict(g.config), golden_bufs(g, ref))


# ------------------------------------------------------------------ per-module vs fairchem golden
# (reference tests/test_so2.py, test_edgewise.py, test_norm.py, test_grid.py, test_model.py)

def test_so2_conv_vs_golden(golden):
    cfg, w = golden.config, golden.w()
    L, C, H = cfg["lmax"], cfg["sphere_channels"], cfg["hidden_channels"]
    out, extra = uma.so2(golden.act("block0.so2_1.in0"), golden.act("block0.so2_1.in1"), w,
                         "blocks.0.edge_wise.so2_conv_1", L, cfg["mmax"], 2 * C, H, L * H)
    assert (out - golden.act("block0.so2_1.out0")).abs().max() < 1e-5
    assert (extra - golden.act("block0.so2_1.out1")).abs().max() < 1e-5
    out2 = uma.so2(golden.act("block0.so2_2.in0"), None, w, "blocks.0.edge_wise.so2_conv_2", L,
                   cfg["mmax"], H, C, 0)
    assert (out2 - golden.act("block0.so2_2.out0")).abs().max() < 1e-5


def test_gate_vs_golden(golden):
    cfg = golden.config
    L, H = cfg["lmax"], cfg["hidden_channels"]
    y = uma.gate(golden.act("block0.so2_1.out1"), golden.act("block0.so2_1.out0"), L, cfg["mmax"], H)
    assert (y - golden.act("block0.so2_2.in0")).abs().max() < 1e-6


def test_edgewise_vs_golden(golden):
    cfg, w = dict(golden.config), golden.w()
    ei = golden.inp("edge_index").long()
    for b in (0, 1):
        x = golden.act(f"block{b}.edgewise.in0")
        out = uma.edgewise(x, w, f"blocks.{b}.edge_wise", cfg, golden.host("wigner"),
                           golden.host("wigner_inv"), golden.host("x_edge"),
                           golden.host("edge_envelope"), ei, x.shape[0])
        ref = golden.act(f"block{b}.edgewise.out0")
        assert (out - ref).abs().max() < 1e-5 * max(1.0, float(ref.abs().max()))


def test_norm_and_grid_vs_golden(golden):
    cfg, w = golden.config, golden.w()
    L, C = cfg["lmax"], cfg["sphere_channels"]
    for b in (0, 1):
        for n in ("norm_1", "norm_2"):
            y = uma.rms_norm_sh(golden.act(f"block{b}.{n}.in0"), w, f"blocks.{b}.{n}", L, C)
            if n == "norm_1":
                # fairchem adds the system embedding to the norm_1 output in place after its
                # forward hook captured it (the captured array shares that memory)
                y[:, 0, :] += golden.host("sys_node_embedding")
            assert (y - golden.act(f"block{b}.{n}.out0")).abs().max() < 1e-5
        y = uma.grid_atomwise(golden.act(f"block{b}.atomwise.in0"), w, f"blocks.{b}.atom_wise",
                              golden.host("to_grid_mat"), golden.host("from_grid_mat"))
        assert (y - golden.act(f"block{b}.atomwise.out0")).abs().max() < 1e-5
    y = uma.rms_norm_sh(golden.act("final_norm.in0"), w, "norm", L, C)
    assert (y - golden.act("final_norm.out0")).abs().max() < 1e-5


def test_backbone_energy_vs_golden(golden):
    cfg, w = dict(golden.config), golden.w()
    ne = uma.backbone(w, cfg, golden.host("x_message_init"), golden.host("wigner"),
                      golden.host("wigner_inv"), golden.host("x_edge"), golden.host("edge_envelope"),
                      golden.host("sys_node_embedding"), golden.inp("edge_index").long(),
                      golden.host("to_grid_mat"), golden.host("from_grid_mat"))
    assert (ne - golden.out("node_embedding")).abs().max() < 5e-6
    E, Eref = float(uma.energy(ne, w)), float(golden.out("energy")[0])
    assert abs(E - Eref) <= 1e-6 * abs(Eref)


# ------------------------------------------------------------------ host geometry vs golden
# (reference tests/test_end2end.py:22-29; the Wigner itself is gauge-dependent, x_init is not)

def test_geometry_vs_golden(golden):
    m = _model(golden)
    t = m.geo(golden.inp("pos").float(), golden.inp("atomic_numbers").long(),
              golden.inp("edge_index").long(), golden.host("sys_node_embedding"))
    assert (t["edge_distance"] - golden.host("edge_distance")).abs().max() < 1e-6
    assert (t["x_edge"] - golden.host("x_edge")).abs().max() < 1e-6
    assert (t["edge_envelope"] - golden.host("edge_envelope")).abs().max() < 1e-6
    assert (t["x_init"] - golden.host("x_message_init")).abs().max() < 2e-6


def test_energy_forces_from_positions_molecule(golden):
    m = _model(golden)
    E, F = OF.energy_and_forces(m, golden.inp("pos").float(), golden.inp("atomic_numbers").long(),
                                golden.inp("edge_index").long(), golden.host("sys_node_embedding"))
    Eref = float(golden.out("energy")[0])
    assert abs(E - Eref) <= 2e-6 * abs(Eref)
    assert (F - golden.out("forces")).abs().max() < 1e-6


def test_energy_forces_from_positions_bulk(golden_bulk, golden):
    g = golden_bulk
    m = _model(g, golden)
    pos = g.inp("pos").float()
    ei, shift = G.neighbor_list(pos, g.config["cutoff"], g.inp("cell").float().reshape(3, 3),
                                [True, True, True])
    E, F = OF.energy_and_forces(m, pos, g.inp("atomic_numbers").long(), ei,
                                g.host("sys_node_embedding"), shift)
    Eref = float(g.out("energy")[0])
    assert abs(E - Eref) <= 2e-6 * abs(Eref)
    assert (F - g.out("forces")).abs().max() < 1e-6


# ------------------------------------------------------------------ neighbour list
def _brute_aperiodic(pos, cutoff):
    out = []
    N = pos.shape[0]
    for i in range(N):
        for j in range(N):
            d = torch.linalg.norm(pos[i] - pos[j])
            if float(d) < cutoff and float(d) > 0:
                out.append((i, j))
    return out


def _brute_periodic(pos, cutoff, cell, reps):
    out = []
    N = pos.shape[0]
    cells = [(a, b, c) for a in range(-reps[0], reps[0] + 1) for b in range(-reps[1], reps[1] + 1)
             for c in range(-reps[2], reps[2] + 1)]
    for i in range(N):
        for j in range(N):
            for ci, n in enumerate(cells):
                s = torch.tensor(n, dtype=pos.dtype) @ cell
                disp = pos[i] - (pos[j] + s)
                d2 = (disp ** 2).sum()
                if float(d2) <= cutoff * cutoff and float(d2) > 1e-8:
                    out.append((j, i, ci))
    return out


def test_radius_graph_matches_golden_edge_sets(golden, golden_bulk):
    pos = golden.inp("pos").float()
    ei, _ = G.neighbor_list(pos, 5.0)
    assert sorted(map(tuple, ei.T.tolist())) == sorted(map(tuple, golden.inp("edge_index").T.tolist()))
    g = golden_bulk
    pos = g.inp("pos").float()
    ei, sh = G.neighbor_list(pos, 5.0, g.inp("cell").float().reshape(3, 3), [True] * 3)
    ref = g.inp("edge_index")
    # the fixture carries no cell offsets; compare (src, tgt, |r|) multisets
    mine = sorted(zip(ei[0].tolist(), ei[1].tolist(),
                      np.round((pos[ei[0]] - pos[ei[1]] + sh).norm(dim=1).numpy(), 4).tolist()))
    assert sorted(zip(*ref.tolist())) == [(a, b) for a, b, _ in mine]
    d_ref = np.sort(np.round(g.host("edge_distance").numpy(), 4)) if g.has("host@edge_distance") else None
    if d_ref is not None:
        assert np.allclose(np.sort([x[2] for x in mine]), d_ref, atol=1e-4)


def test_radius_graph_brute_force():
    gen = torch.Generator().manual_seed(7)
    pos = torch.rand(11, 3, generator=gen) * 4.0
    ei, _, _ = G.radius_graph(pos, 2.5)
    assert list(map(tuple, ei.T.tolist())) == _brute_aperiodic(pos, 2.5)
    cell = torch.tensor([[3.0, 0.0, 0.0], [0.7, 3.2, 0.0], [0.1, 0.4, 2.9]])
    pos = torch.rand(5, 3, generator=gen) @ cell
    ei, sh, c = G.radius_graph(pos, 3.5, cell, [True, True, True])
    recip = torch.linalg.inv(cell).T
    reps = [int(math.ceil(float(3.5 * torch.linalg.norm(recip[k])))) for k in range(3)]
    brute = _brute_periodic(pos, 3.5, cell, reps)
    # reference order: (tgt, src, cell) ascending
    assert list(zip(ei[0].tolist(), ei[1].tolist(), c.tolist())) == brute


def test_cap_rule_brute_force():
    gen = torch.Generator().manual_seed(3)
    pos = torch.rand(30, 3, generator=gen) * 5.0
    ei, sh, _ = G.radius_graph(pos, 3.0)
    keep = G.cap_neighbors(pos, ei, sh, 4)
    ev = pos[ei[0]] - pos[ei[1]]
    d2 = (ev[:, 0] * ev[:, 0] + ev[:, 1] * ev[:, 1]) + ev[:, 2] * ev[:, 2]
    for n in range(30):
        idx = [e for e in range(ei.shape[1]) if int(ei[1, e]) == n]
        ranked = sorted(idx, key=lambda e: (float(d2[e]), int(ei[0, e]), e))[:4]
        assert sorted(ranked) == [e for e in idx if bool(keep[e])]
    assert int(torch.bincount(ei[1][keep], minlength=30).max()) <= 4


# ------------------------------------------------------------------ Wigner closed forms
def test_wigner_closed_forms(golden):
    m = _model(golden)
    gen = torch.Generator().manual_seed(0)
    ev = torch.randn(64, 3, generator=gen, dtype=torch.float64)
    m64 = m.to(torch.float64)
    wM, wMi = m64.geo.wigner(ev)
    # orthogonality and W_inv == W^T
    eye = torch.eye(9, dtype=torch.float64).expand(64, 9, 9)
    assert (wM @ wM.transpose(1, 2) - eye).abs().max() < 1e-6      # Jd is stored fp32
    assert (wMi - wM.transpose(1, 2)).abs().max() == 0
    # to_m is a permutation; D_0 = 1
    assert sorted(m.geo.perm.tolist()) == list(range(9))
    assert (wM[:, 0, 0] - 1).abs().max() == 0
    # the l=1 block (natural order rows 1..3 of the unpermuted matrix) maps the edge direction
    # (basis x, y, z) onto the +y axis: the edge frame's polar axis
    wig = G.eulers_to_wigner(G.euler_angles(ev), 2, m64.geo.Jd)
    u = ev / ev.norm(dim=1, keepdim=True)
    r = (wig[:, 1:4, 1:4] @ u.unsqueeze(-1)).squeeze(-1)
    assert (r - torch.tensor([0.0, 1.0, 0.0], dtype=torch.float64)).abs().max() < 1e-6
    # gamma=0 leaves 32 structurally nonzero entries out of the 35 block-diagonal slots
    assert int((wM.abs().amax(0) > 1e-6).sum()) == 32


# ------------------------------------------------------------------ forces / stress
def _fd_check(model, pos, Z, ei, se, shift=None, idx=((0, 0), (1, 2), (3, 1)), h=1e-5):
    E, F = OF.energy_and_forces(model, pos, Z, ei, se, shift)
    for (a, k) in idx:
        p1, p2 = pos.clone(), pos.clone()
        p1[a, k] += h
        p2[a, k] -= h
        e1 = float(OF.forward_energy(model, p1, Z, ei, se, shift)[0])
        e2 = float(OF.forward_energy(model, p2, Z, ei, se, shift)[0])
        assert abs(-(e1 - e2) / (2 * h) - float(F[a, k])) < 1e-7 * max(1.0, abs(float(F[a, k])))


def test_forces_finite_difference_fp64(golden):
    m = _model(golden).to(torch.float64)
    _fd_check(m, golden.inp("pos").double(), golden.inp("atomic_numbers").long(),
              golden.inp("edge_index").long(), golden.host("sys_node_embedding").double())


def test_stress_finite_difference_fp64(golden_bulk, golden):
    g = golden_bulk
    m = _model(g, golden).to(torch.float64)
    pos = g.inp("pos").double()
    cell = g.inp("cell").double().reshape(3, 3)
    ei, sh = G.neighbor_list(pos.float(), 5.0, cell.float(), [True] * 3)
    sh = sh.double()
    Z, se = g.inp("atomic_numbers").long(), g.host("sys_node_embedding").double()
    E, F, V = OF.energy_and_forces(m, pos, Z, ei, se, sh, compute_stress=True)
    assert (V - V.T).abs().max() < 1e-12
    h = 1e-6
    for (a, b) in ((0, 0), (0, 1), (2, 2)):
        eps = torch.zeros(3, 3, dtype=torch.float64)
        eps[a, b] += 0.5 * h
        eps[b, a] += 0.5 * h
        e1 = float(OF.forward_energy(m, pos, Z, ei, se, sh, strain=eps)[0])
        e2 = float(OF.forward_energy(m, pos, Z, ei, se, sh, strain=-eps)[0])
        assert abs((e1 - e2) / (2 * h) - float(V[a, b])) < 1e-6 * max(1.0, abs(float(V[a, b])))
    # forces sum to zero (translation invariance)
    assert F.sum(0).abs().max() < 1e-10


def test_rotation_invariance(golden):
    m = _model(golden).to(torch.float64)
    pos = golden.inp("pos").double()
    Z, ei = golden.inp("atomic_numbers").long(), golden.inp("edge_index").long()
    se = golden.host("sys_node_embedding").double()
    E0, F0 = OF.energy_and_forces(m, pos, Z, ei, se)
    q, _ = torch.linalg.qr(torch.randn(3, 3, dtype=torch.float64, generator=torch.Generator().manual_seed(1)))
    if torch.det(q) < 0:
        q[:, 0] = -q[:, 0]
    E1, F1 = OF.energy_and_forces(m, pos @ q.T + 0.37, Z, ei, se)
    # the grid feed-forward's S2 projection matrices (and Jd) are stored fp32, so the model is
    # equivariant only to fp32 resolution even when evaluated in fp64
    assert abs(E1 - E0) < 1e-6 * max(1.0, abs(E0))
    assert (F1 - F0 @ q.T).abs().max() < 1e-5


# ------------------------------------------------------------------ system embedding known answers
# (geometry.py:23-45)
@pytest.mark.parametrize("fixture", ["golden", "golden_bulk"])
def test_csd_embedding_vs_golden(fixture, request):
    """The system embedding of the committed fairchem goldens (pos_emb encoding, charge 0, spin
    0, dataset omat): the oracle and the package's host function both reproduce
    host@sys_node_embedding (one row per node, all equal)."""
    from tt_atom import geometry as TG
    g = request.getfixturevalue(fixture)
    w, ref = g.w(), g.host("sys_node_embedding")
    chg, spin = g.inp("charge").float(), g.inp("spin").float()
    for fn in (G.csd_embedding, lambda *a, **k: TG.csd_embedding(*a, **k)):
        got = fn(w, chg, spin, dataset="omat")
        assert got.shape == (1, ref.shape[1])
        assert (got.expand_as(ref) - ref).abs().max() < 1e-6


def _csd_select_weights(C):
    """mix_csd = a scaled selection [4, 12] (C = 4) reading input columns 1, 6, 11 and 2 of
    [charge | spin | dataset]: the second charge component, the third spin component, the last
    dataset component and the third charge component, scaled by 1 + i/8."""
    assert C == 4
    cols = [1, 6, 11, 2]
    W = torch.zeros(C, 3 * C, dtype=torch.float64)
    for i, c in enumerate(cols):
        W[i, c] = 1.0 + i / 8
    return W, cols


def _silu(v):
    return v / (1.0 + math.exp(-v))


@pytest.mark.parametrize("impl", ["oracle", "package"])
def test_csd_embedding_rand_emb_known_rows(impl):
    """rand_emb (uma-s-1): charge c reads row c + 100 of the charge table and spin s row s of the
    spin table, concatenated with the dataset token before mix_csd and SiLU.  Tables whose rows
    encode their own index make a wrong offset or a swapped table visible."""
    from tt_atom import geometry as TG
    fn = G.csd_embedding if impl == "oracle" else TG.csd_embedding
    C = 4
    rows = (torch.arange(201, dtype=torch.float64)[:, None] * 0.01
            + torch.arange(C, dtype=torch.float64) * 0.001)
    w = {"charge_embedding.rand_emb.weight": rows,
         "spin_embedding.rand_emb.weight": -rows[:101] - 0.5,
         "dataset_embedding.dataset_emb_dict.omol.weight":
             torch.tensor([[0.3, -0.2, 0.1, 0.05]], dtype=torch.float64),
         "mix_csd.bias": torch.tensor([0.01, -0.02, 0.03, 0.0], dtype=torch.float64)}
    w["mix_csd.weight"], cols = _csd_select_weights(C)
    charge, spin = torch.tensor([-2.0, 0.0, 3.0]), torch.tensor([1.0, 0.0, 5.0])
    got = fn(w, charge, spin, dataset="omol")
    for s in range(3):
        inp = ([0.01 * (charge[s].item() + 100) + 0.001 * j for j in range(C)]
               + [-(0.01 * spin[s].item() + 0.001 * j) - 0.5 for j in range(C)]
               + [0.3, -0.2, 0.1, 0.05])
        ref = [_silu((1.0 + i / 8) * inp[cols[i]] + [0.01, -0.02, 0.03, 0.0][i]) for i in range(C)]
        assert max(abs(float(got[s, i]) - ref[i]) for i in range(C)) < 1e-12, (s, got[s], ref)


@pytest.mark.parametrize("impl", ["oracle", "package"])
def test_csd_embedding_pos_emb_known_values(impl):
    """pos_emb: x -> [sin(2 pi x W) | cos(2 pi x W)] per charge and spin, the spin part zeroed
    where spin == 0 (the charge part never), against hand-evaluated sines and cosines."""
    from tt_atom import geometry as TG
    fn = G.csd_embedding if impl == "oracle" else TG.csd_embedding
    C = 4
    Wc, Ws = [0.13, -0.4], [0.7, 0.25]
    w = {"charge_embedding.W": torch.tensor(Wc, dtype=torch.float64),
         "spin_embedding.W": torch.tensor(Ws, dtype=torch.float64),
         "dataset_embedding.dataset_emb_dict.omat.weight":
             torch.tensor([[0.5, 0.25, -0.75, 1.0]], dtype=torch.float64),
         "mix_csd.bias": torch.zeros(C, dtype=torch.float64)}
    w["mix_csd.weight"], cols = _csd_select_weights(C)
    charge, spin = torch.tensor([1.0, 0.0, -1.0]), torch.tensor([0.0, 2.0, 1.0])
    got = fn(w, charge.double(), spin.double(), dataset="omat")
    tp = 2 * math.pi
    for s in range(3):
        q, sp = charge[s].item(), spin[s].item()
        enc_q = [math.sin(tp * q * Wc[0]), math.sin(tp * q * Wc[1]),
                 math.cos(tp * q * Wc[0]), math.cos(tp * q * Wc[1])]
        enc_s = [math.sin(tp * sp * Ws[0]), math.sin(tp * sp * Ws[1]),
                 math.cos(tp * sp * Ws[0]), math.cos(tp * sp * Ws[1])] if sp != 0 else [0.0] * 4
        inp = enc_q + enc_s + [0.5, 0.25, -0.75, 1.0]
        ref = [_silu((1.0 + i / 8) * inp[cols[i]]) for i in range(C)]
        assert max(abs(float(got[s, i]) - ref[i]) for i in range(C)) < 1e-12, (s, got[s], ref)
    # the selection reaches both halves of both encodings and the dataset token
    assert {c // C for c in cols} == {0, 1, 2}


# ------------------------------------------------------------------ spectral FF known answers
# (spectral.py:146-188: gating = SiLU(scalar_mlp(x0)); h = SO3_Linear_1(x) with one [out, in]
# weight per degree and the bias on l = 0; SiLU on h0, sigmoid(gating[(l-1)H:lH]) on degree l;
# SO3_Linear_2)
def _spectral_weights(C, H, lmax, scalar_w, scalar_b):
    p = "ff"
    w = {f"{p}.scalar_mlp.0.weight": scalar_w, f"{p}.scalar_mlp.0.bias": scalar_b}
    # SO3 linears: degree l uses a non-symmetric selection [out, in] scaled by (l + 1)
    for name, (o, i) in (("so3_linear_1", (H, C)), ("so3_linear_2", (C, H))):
        Wt = torch.zeros(lmax + 1, o, i, dtype=torch.float64)
        for l in range(lmax + 1):
            for r in range(o):
                Wt[l, r, (r + l + 1) % i] = (l + 1) * (1.0 if name.endswith("1") else 0.5)
        w[f"{p}.{name}.weight"] = Wt
        w[f"{p}.{name}.bias"] = torch.tensor([0.1 * (r + 1) * (-1) ** r for r in range(o)],
                                             dtype=torch.float64)
    return w


def _spectral_expected(x, w, C, H, lmax):
    """Explicit loops over nodes, coefficients and channels from the reference's statement."""
    p = "ff"
    deg = [l for l in range(lmax + 1) for _ in range(2 * l + 1)]
    Ws, bs = w[f"{p}.scalar_mlp.0.weight"], w[f"{p}.scalar_mlp.0.bias"]
    out = torch.zeros_like(x)
    for n in range(x.shape[0]):
        a = [sum(float(Ws[r, i]) * float(x[n, 0, i]) for i in range(C)) + float(bs[r])
             for r in range(lmax * H)]
        gating = [_silu(v) for v in a]
        for c, l in enumerate(deg):
            W1, b1 = w[f"{p}.so3_linear_1.weight"][l], w[f"{p}.so3_linear_1.bias"]
            h = [sum(float(W1[r, i]) * float(x[n, c, i]) for i in range(C))
                 + (float(b1[r]) if c == 0 else 0.0) for r in range(H)]
            if c == 0:
                g = [_silu(v) for v in h]
            else:
                g = [h[r] / (1.0 + math.exp(-gating[(l - 1) * H + r])) for r in range(H)]
            W2, b2 = w[f"{p}.so3_linear_2.weight"][l], w[f"{p}.so3_linear_2.bias"]
            for r in range(C):
                out[n, c, r] = (sum(float(W2[r, i]) * g[i] for i in range(H))
                                + (float(b2[r]) if c == 0 else 0.0))
    return out


def test_spectral_ff_gate_known_constants():
    """Zero scalar-MLP weight with a known bias makes every gate a constant: degree 1 is scaled
    by sigmoid(SiLU(0)) = 1/2 and degree 2 by sigmoid(SiLU(2)) = 0.85341..., l = 0 goes through
    SiLU; with the identity-like SO3 linears below the output is known in closed form."""
    C = H = 3
    lmax = 2
    w = {"ff.scalar_mlp.0.weight": torch.zeros(lmax * H, C, dtype=torch.float64),
         "ff.scalar_mlp.0.bias": torch.tensor([0.0] * H + [2.0] * H, dtype=torch.float64)}
    for name in ("so3_linear_1", "so3_linear_2"):
        w[f"ff.{name}.weight"] = torch.eye(C, dtype=torch.float64).expand(lmax + 1, C, C).clone()
        w[f"ff.{name}.bias"] = torch.zeros(C, dtype=torch.float64)
    x = torch.linspace(-1.5, 2.0, 2 * 9 * C, dtype=torch.float64).reshape(2, 9, C)
    got = uma.spectral_atomwise(x, w, "ff", lmax, H)
    g2 = 1.0 / (1.0 + math.exp(-_silu(2.0)))
    assert abs(g2 - 0.8534092045709026) < 1e-12
    ref = x.clone()
    ref[:, 0, :] = x[:, 0, :] * torch.sigmoid(x[:, 0, :])
    ref[:, 1:4, :] = 0.5 * x[:, 1:4, :]
    ref[:, 4:9, :] = g2 * x[:, 4:9, :]
    assert (got - ref).abs().max() < 1e-14


def _spectral_case():
    C, H, lmax = 3, 4, 2
    gen = torch.Generator().manual_seed(5)
    Ws = torch.randn(lmax * H, C, generator=gen, dtype=torch.float64)
    bs = torch.randn(lmax * H, generator=gen, dtype=torch.float64)
    w = _spectral_weights(C, H, lmax, Ws, bs)
    x = torch.randn(3, 9, C, generator=gen, dtype=torch.float64)
    return x, w, C, H, lmax


def test_spectral_ff_known_answer_loops():
    """Random scalar MLP, per-degree selection SO3 linears with distinct scales and biases: the
    oracle equals the loop evaluation of the reference's statement."""
    x, w, C, H, lmax = _spectral_case()
    got = uma.spectral_atomwise(x, w, "ff", lmax, H)
    assert (got - _spectral_expected(x, w, C, H, lmax)).abs().max() < 1e-12


def test_spectral_ff_known_answer_catches_planted_mistakes(monkeypatch):
    """Each plausible wiring mistake, planted into a copy of the oracle's spectral FF, fails the
    loop known answer: a missing SiLU on the gating, swapped degree-1 / degree-2 gate rows, the
    bias on every coefficient, transposed per-degree weights, or one shared weight for all
    degrees."""
    import torch.nn.functional as F
    x, w, C, H, lmax = _spectral_case()
    ref = _spectral_expected(x, w, C, H, lmax)

    def variant(mistake):
        def so3(v, Wt, b):
            outs, s = [], 0
            for l in range(lmax + 1):
                n = 2 * l + 1
                Wl = Wt[0] if mistake == "shared" else Wt[l]
                ob = v[:, s:s + n, :] @ (Wl if mistake == "transposed" and Wl.shape[0] == Wl.shape[1]
                                         else Wl.T)
                if l == 0 or mistake == "bias_all":
                    ob = ob + b.view(1, 1, -1)
                outs.append(ob)
                s += n
            return torch.cat(outs, 1)
        a = F.linear(x[:, 0, :], w["ff.scalar_mlp.0.weight"], w["ff.scalar_mlp.0.bias"])
        gating = a if mistake == "no_silu" else F.silu(a)
        h = so3(x, w["ff.so3_linear_1.weight"], w["ff.so3_linear_1.bias"])
        sg = torch.sigmoid(gating)
        rows = [1, 0] if mistake == "swap_rows" else [0, 1]
        parts, s = [F.silu(h[:, 0:1, :])], 1
        for l in range(1, lmax + 1):
            n = 2 * l + 1
            r = rows[l - 1]
            parts.append(h[:, s:s + n, :] * sg[:, r * H:(r + 1) * H].unsqueeze(1))
            s += n
        return so3(torch.cat(parts, 1), w["ff.so3_linear_2.weight"], w["ff.so3_linear_2.bias"])

    assert (variant(None) - ref).abs().max() < 1e-12
    for mistake in ("no_silu", "swap_rows", "bias_all", "shared"):
        assert (variant(mistake) - ref).abs().max() > 1e-3, mistake


def test_safe_acos_atan2_regularised_gradients_known_values():
    """The regularised derivatives of the Euler angles (geometry.py:87-109): acos' = -1/sqrt(1-x^2)
    with x clamped to [-1 + 1e-7, 1 - 1e-7] and the root clamped at 1e-7; atan2' = (x, -y) / r^2
    with r^2 clamped at 1e-7.  Generic points give the textbook derivatives; the poles give the
    clamped values."""
    x = torch.tensor([0.6, 1.0, -1.0, 0.0], dtype=torch.float64, requires_grad=True)
    (g,) = torch.autograd.grad(G.SafeAcos.apply(x).sum(), x)
    xc = 1 - 1e-7
    pole = -1.0 / math.sqrt(1 - xc * xc)
    ref = torch.tensor([-1.25, pole, pole, -1.0], dtype=torch.float64)
    assert (g - ref).abs().max() < 1e-9 * abs(pole)
    y = torch.tensor([3.0, 0.0, 1e-5, -2.0], dtype=torch.float64, requires_grad=True)
    xx = torch.tensor([4.0, 0.0, 0.0, 0.0], dtype=torch.float64, requires_grad=True)
    gy, gx = torch.autograd.grad(G.SafeAtan2.apply(y, xx).sum(), (y, xx))
    torch.testing.assert_close(gy, torch.tensor([4 / 25, 0.0, 0.0, 0.0], dtype=torch.float64),
                               rtol=0, atol=1e-15)
    torch.testing.assert_close(gx, torch.tensor([-3 / 25, 0.0, -1e-5 / 1e-7, 2.0 / 4.0],
                                                dtype=torch.float64), rtol=1e-12, atol=1e-15)
