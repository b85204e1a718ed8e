"""The Orb-v3 path through the reference's import paths and signatures: orb_weights.OrbWeights,
disjoint.assemble_orb, orb_model.Encoder / AttentionInteractionLayer / EnergyHead /
OrbGraphContext / host_node_features / host_charge_spin_embedding,
orb_forces.energy_and_forces(_batch) and orb_geometry.host_edge_features(_vjp).  The module
route runs the same OrbEngine step as tt_atom.orb, so its results are bit for bit those of
orb.energy_and_forces(_batch); the edge-descriptor functions are checked against the fp64
oracle and against each other (autograd through host_edge_features == host_edge_features_vjp)."""
import numpy as np
import pytest
import torch

from oracle import orb as O
from tt_atom import disjoint, orb, orb_forces, orb_geometry, orb_model, orb_weights
from tt_atom import synthetic as S

pytestmark = pytest.mark.gpu


def _modules(w, cfg, dev, **kw):
    """The reference's construction sequence (orb_calculator.py:54-67)."""
    C, H = cfg["latent_dim"], cfg["mlp_hidden_dim"]
    enc = orb_model.Encoder(w, dev, node_in=cfg["node_embed_size"], edge_in=cfg["edge_embed_size"],
                            latent_dim=C, hidden_dim=H, **kw)
    layers = [orb_model.AttentionInteractionLayer(w, f"gnn_stacks.{i}", dev, latent_dim=C,
                                                  hidden_dim=H, **kw)
              for i in range(cfg["num_message_passing_steps"])]
    # the reference passes the MLP width to the head as well; the head reads its own from the
    # weights
    eh = orb_model.EnergyHead(w, dev, latent_dim=C, hidden_dim=H, **kw)
    return enc, layers, eh


def _bundle(tmp_path, cfg, seed):
    w = S.random_orb_weights(cfg, seed)
    path = tmp_path / "orb.npz"
    orb.save_orb_bundle(path, cfg, w)
    ow = orb_weights.OrbWeights.load(path)
    assert ow.config == cfg
    return ow.weights, ow.config


@pytest.mark.parametrize("precision", [None, "bf16"])
def test_reference_signatures_equal_engine(tmp_path, precision):
    cfg = dict(S.CFG_ORB_TINY)
    w, cfg = _bundle(tmp_path, cfg, 11)
    dev = torch.device("cuda")
    kw = {} if precision is None else {"fast": True}
    enc, layers, eh = _modules(w, cfg, dev, **kw)
    model = orb.OrbModel(w, cfg, precision="f32" if precision is None else precision)
    systems = S.c5_systems(11, K=3, n_min=6, n_max=14, side=5.0)
    bg = disjoint.assemble_orb(systems, cfg["cutoff"], cfg["max_num_neighbors"])
    common = dict(r_max=cfg["cutoff"], num_bases=cfg["num_bases"])

    # one system through orb_forces.energy_and_forces
    one = disjoint.assemble_orb(systems[:1], cfg["cutoff"], cfg["max_num_neighbors"])
    nf = orb_model.host_node_features(w, one.Z)
    raw, F = orb_forces.energy_and_forces(enc, layers, eh, dev, pos=one.pos, senders=one.senders,
                                          receivers=one.receivers, atomic_numbers=one.Z,
                                          node_feat=nf, cell_shift=one.cell_shift, **common)
    r_raw, r_F = orb.energy_and_forces(model, pos=one.pos, senders=one.senders,
                                       receivers=one.receivers, atomic_numbers=one.Z,
                                       cell_shift=one.cell_shift)
    print(f"boundary ({precision}): single raw {raw:.8f} vs {r_raw:.8f}", flush=True)
    assert isinstance(raw, float) and raw == r_raw and torch.equal(F, r_F)
    assert F.dtype == one.pos.dtype and F.shape == (one.pos.shape[0], 3)

    # the batch through orb_forces.energy_and_forces_batch with the segment matrices
    _, seg_mean = bg.segment_matrices()
    rb, Fb = orb_forces.energy_and_forces_batch(
        enc, layers, eh, dev, pos=bg.pos, senders=bg.senders, receivers=bg.receivers,
        atomic_numbers=bg.Z, node_feat=orb_model.host_node_features(w, bg.Z),
        cell_shift=bg.cell_shift, seg_mean=seg_mean, seg_mean_T=seg_mean.T.contiguous(),
        **common)
    r_rb, r_Fb = orb.energy_and_forces_batch(model, pos=bg.pos, senders=bg.senders,
                                             receivers=bg.receivers, atomic_numbers=bg.Z,
                                             natoms=bg.natoms, cell_shift=bg.cell_shift)
    assert rb.dtype == torch.float64 and rb.shape == (bg.K,)
    assert torch.equal(rb, r_rb) and torch.equal(Fb, r_Fb)
    # and against the fp64 oracle at the precision's tolerance
    ref_raw, ref_F = O.energy_and_forces(w, cfg, bg.pos.double(), bg.Z, bg.senders,
                                         bg.receivers, bg.cell_shift.double(), bg.batch,
                                         bg.natoms)
    tol_e, tol_f = (1e-6, 2e-6) if precision is None else (2e-2, 4e-2)
    assert (rb - ref_raw).abs().max() <= tol_e * max(1.0, ref_raw.abs().max().item())
    assert (Fb.double() - ref_F).abs().max() <= tol_f * max(1.0, ref_F.abs().max().item())
    # a seg_mean whose systems are not contiguous node ranges is refused
    with pytest.raises(ValueError):
        orb_forces.energy_and_forces_batch(
            enc, layers, eh, dev, pos=bg.pos, senders=bg.senders, receivers=bg.receivers,
            atomic_numbers=bg.Z, node_feat=orb_model.host_node_features(w, bg.Z),
            cell_shift=bg.cell_shift, seg_mean=seg_mean.flip(1), seg_mean_T=None, **common)


def test_reference_signatures_stress_and_conditioning(tmp_path):
    """compute_stress on a periodic crystal and the charge / spin conditioning (cond_nodes from
    host_charge_spin_embedding): equal to the engine route."""
    dev = torch.device("cuda")
    cfg = dict(S.CFG_ORB_TINY)
    w, cfg = _bundle(tmp_path, cfg, 99)
    enc, layers, eh = _modules(w, cfg, dev)
    pos, Z, cell = S.c4_system(seed=4, reps=2, a=3.61, noise=0.05, Z=29)
    bg = disjoint.assemble_orb([(pos, Z, cell, [True] * 3)], cfg["cutoff"],
                               cfg["max_num_neighbors"], truncate=True)
    raw, F, vir = orb_forces.energy_and_forces(
        enc, layers, eh, dev, pos=bg.pos, senders=bg.senders, receivers=bg.receivers,
        atomic_numbers=bg.Z, node_feat=orb_model.host_node_features(w, bg.Z),
        cell_shift=bg.cell_shift, r_max=cfg["cutoff"], num_bases=cfg["num_bases"],
        compute_stress=True, bucketing=True, max_num_neighbors=cfg["max_num_neighbors"])
    r_raw, r_F, r_vir = orb.energy_and_forces(orb.OrbModel(w, cfg), pos=bg.pos,
                                              senders=bg.senders, receivers=bg.receivers,
                                              atomic_numbers=bg.Z, cell_shift=bg.cell_shift,
                                              compute_stress=True)
    assert raw == r_raw and torch.equal(F, r_F) and torch.equal(vir, r_vir)

    cfg = dict(S.CFG_ORB_TINY, has_charge_spin_cond=True)
    w, cfg = _bundle(tmp_path, cfg, 12)
    enc, layers, eh = _modules(w, cfg, dev)
    one = disjoint.assemble_orb(S.c5_systems(12, K=1, n_min=8, n_max=12, side=5.0),
                                cfg["cutoff"], cfg["max_num_neighbors"])
    n = one.natoms[0]
    cond = orb_model.host_charge_spin_embedding(w, 1.0, 2.0, n, cfg["latent_dim"])
    model = orb.OrbModel(w, cfg)
    assert torch.equal(cond, model.charge_spin_embedding(1.0, 2.0, n).contiguous())
    raw, F = orb_forces.energy_and_forces(
        enc, layers, eh, dev, pos=one.pos, senders=one.senders, receivers=one.receivers,
        atomic_numbers=one.Z, node_feat=orb_model.host_node_features(w, one.Z),
        cell_shift=one.cell_shift, r_max=cfg["cutoff"], num_bases=cfg["num_bases"],
        cond_nodes=cond)
    r_raw, r_F = orb.energy_and_forces(model, pos=one.pos, senders=one.senders,
                                       receivers=one.receivers, atomic_numbers=one.Z,
                                       cell_shift=one.cell_shift, cond_nodes=cond)
    assert raw == r_raw and torch.equal(F, r_F)
    ref_raw, _ = O.energy_and_forces(w, cfg, one.pos.double(), one.Z, one.senders, one.receivers,
                                     one.cell_shift.double(), one.batch, one.natoms,
                                     cond_nodes=cond.double())
    assert abs(raw - float(ref_raw[0])) <= 1e-6 * max(1.0, abs(float(ref_raw[0])))


def test_host_edge_features_and_vjp():
    """host_edge_features (device kernels) against the fp64 oracle; autograd through it (pos
    and strain) against host_edge_features_vjp and the oracle's autograd."""
    g = torch.Generator().manual_seed(7)
    n, E = 30, 300
    pos = 3.0 * torch.randn(n, 3, generator=g)
    s = torch.randint(n, (E,), generator=g)
    r = (s + torch.randint(1, n, (E,), generator=g)) % n
    shift = 0.3 * torch.randn(E, 3, generator=g)
    feat, cut, vec = orb_geometry.host_edge_features(pos, s, r, shift, r_max=6.0, num_bases=8)
    assert feat.device == pos.device and cut.shape == (E, 1) and vec.shape == (E, 3)
    rf, rc, rv = O.edge_features(pos.double(), s, r, shift.double())
    assert (feat.double() - rf).abs().max() < 1e-5
    assert (cut.double() - rc).abs().max() < 1e-6
    assert (vec.double() - rv).abs().max() < 2e-6
    gf, gc = torch.randn(E, 128, generator=g), torch.randn(E, 1, generator=g)
    # closed-form VJP function
    F = orb_geometry.host_edge_features_vjp(vec, s, r, n, gf, gc, r_max=6.0, num_bases=8)
    p64 = pos.double().requires_grad_(True)
    strain = torch.zeros(3, 3, dtype=torch.float64, requires_grad=True)
    f64, c64, _ = O.edge_features(p64, s, r, shift.double(), strain=strain)
    g_pos, g_strain = torch.autograd.grad([f64, c64], [p64, strain], [gf.double(), gc.double()])
    scale = g_pos.abs().max()
    assert (F.double() + g_pos).abs().max() / scale < 1e-5
    # autograd through host_edge_features, on the GPU, with a strain leaf
    pd = pos.cuda().requires_grad_(True)
    st = torch.zeros(3, 3, device="cuda", requires_grad=True)
    f2, c2, _ = orb_geometry.host_edge_features(pd, s.cuda(), r.cuda(), shift.cuda(), r_max=6.0,
                                                num_bases=8, strain=st)
    gp, gs = torch.autograd.grad([f2, c2], [pd, st], [gf.cuda(), gc.cuda()])
    assert (gp.cpu().double() - g_pos).abs().max() / scale < 1e-5
    assert (gs.cpu().double() - g_strain).abs().max() / g_strain.abs().max() < 1e-5
    assert torch.equal(gp.cpu(), -orb_geometry.host_edge_features_vjp(
        vec.cuda(), s, r, n, gf, gc, r_max=6.0, num_bases=8).cpu())
