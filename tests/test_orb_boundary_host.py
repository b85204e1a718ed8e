"""Host-side pieces of the Orb-v3 reference-named boundary (no GPU): import paths, the segment
matrix -> system sizes conversion of orb_forces.energy_and_forces_batch, the bundle loader."""
import numpy as np
import pytest
import torch

from tt_atom import disjoint, orb, orb_forces, orb_geometry, orb_model, orb_weights
from tt_atom import synthetic as S


def test_reference_import_paths():
    for mod, names in ((orb_model, ["Encoder", "AttentionInteractionLayer", "EnergyHead",
                                    "ForceHead", "StressHead", "OrbGraphContext", "MLPNorm",
                                    "RMSNorm", "host_node_features",
                                    "host_charge_spin_embedding", "host_energy_denormalize",
                                    "host_conservative_force_denormalize",
                                    "host_conservative_stress", "host_force_denormalize",
                                    "host_stress_denormalize", "host_zbl_energy"]),
                       (orb_forces, ["energy_and_forces", "energy_and_forces_batch"]),
                       (orb_geometry, ["host_edge_features", "host_edge_features_vjp"]),
                       (orb_weights, ["OrbWeights"]),
                       (disjoint, ["assemble_orb", "OrbBatchedGraph"])):
        for n in names:
            assert hasattr(mod, n), (mod.__name__, n)
    assert orb.OrbWeights is orb_weights.OrbWeights


def test_natoms_from_seg_mean():
    systems = S.c5_systems(3, K=4, n_min=5, n_max=9, side=5.0)
    bg = disjoint.assemble_orb(systems, 6.0, 20)
    _, seg_mean = bg.segment_matrices()
    n = bg.pos.shape[0]
    assert orb_forces._natoms_from_seg_mean(seg_mean, n) == bg.natoms
    with pytest.raises(ValueError):                      # systems out of order
        orb_forces._natoms_from_seg_mean(seg_mean.flip(1), n)
    bad = seg_mean.clone()
    bad[0, -1] = 0.5                                      # a node in two systems
    with pytest.raises(ValueError):
        orb_forces._natoms_from_seg_mean(bad, n)
    with pytest.raises(ValueError):
        orb_forces._natoms_from_seg_mean(seg_mean[:, :-1], n)


def test_host_terms_match_package_functions():
    cfg = dict(S.CFG_ORB_TINY, has_charge_spin_cond=True)
    w = S.random_orb_weights(cfg, 5)
    Z = torch.tensor([1, 6, 8, 8])
    assert torch.equal(orb_model.host_node_features(w, Z), w["atom_emb.embeddings.weight"][Z])
    c = orb_model.host_charge_spin_embedding(w, -1.0, 0.0, 3, cfg["latent_dim"])
    ref = orb.charge_spin_embedding_batch(w, cfg["latent_dim"], [-1.0], [0.0], [3])
    assert torch.equal(c, ref) and c.shape == (3, cfg["latent_dim"])
    e = orb_model.host_energy_denormalize(
        torch.tensor(0.25), Z, 4, running_mean=w["energy_head.normalizer.bn.running_mean"],
        running_var=w["energy_head.normalizer.bn.running_var"],
        ref_weight=w["energy_head.reference.linear.weight"])
    assert torch.equal(e, orb.denormalize_energy(torch.tensor(0.25), Z, 4, w))


def test_bundle_round_trip(tmp_path):
    cfg = dict(S.CFG_ORB_TINY)
    w = S.random_orb_weights(cfg, 1)
    orb.save_orb_bundle(tmp_path / "b.npz", cfg, w)
    ow = orb_weights.OrbWeights.load(tmp_path / "b.npz")
    assert ow.config == cfg
    got = ow.weights
    assert set(got) == set(w)
    assert all(torch.equal(got[k], torch.as_tensor(w[k], dtype=torch.float32)) for k in w)
