"""Host-side logic of the calculator front end (no GPU): Voigt conversion, bundle round trip,
coverage check, neighbour-list cap and configuration generators."""
import numpy as np
import pytest
import torch

from tt_atom import calculator, geometry, synthetic, weights


def test_voigt_order_matches_ase_convention():
    s = np.arange(9, dtype=float).reshape(3, 3)
    v = calculator.full_3x3_to_voigt_6(s)
    assert np.allclose(v, [0, 4, 8, 0.5 * (5 + 7), 0.5 * (2 + 6), 0.5 * (1 + 3)])


def test_bundle_round_trip_and_coverage(tmp_path):
    cfg = dict(synthetic.CFG_UMA_S, sphere_channels=8, hidden_channels=8, edge_channels=8,
               num_distance_basis=8, num_layers=1)
    w, host = synthetic.random_uma_bundle(cfg, 5)
    p = tmp_path / "b.npz"
    weights.save_bundle(p, cfg, w, host, scale={"rmsd": 2.0, "mean": -1.0})
    b = weights.WeightBundle.load(p)
    ok, missing, _ = b.verify_coverage()
    assert ok, missing
    assert b.scale_rmsd == 2.0 and b.scale_mean == -1.0 and b.task == "omol"
    assert torch.equal(b.weights["blocks.0.norm_1.affine_weight"], w["blocks.0.norm_1.affine_weight"])
    assert torch.equal(b.to_m, host["to_m"])


def test_jd_matches_fixture(golden):
    jd = synthetic.jd_matrices()
    for l in range(3):
        assert (jd[l] - golden.w()[f"Jd_{l}"]).abs().max() < 1e-7


def test_gaussian_buffers_match_fixture(golden):
    off, coeff = synthetic.gaussian_buffers(32, 5.0)
    assert (off - golden.host("gauss_offset")).abs().max() < 1e-6
    assert abs(float(coeff) - float(golden.host("gauss_coeff"))) < 1e-4


def test_product_neighbor_list_matches_oracle():
    from oracle import geometry as OG
    pos, Z = synthetic.c1_system()
    pos = torch.from_numpy(pos)
    for cap in (None, 6):
        a = geometry.radius_graph(pos, 5.0, max_neighbors=cap)
        b = OG.neighbor_list(pos, 5.0, max_neighbors=cap)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    p4, _, cell = synthetic.c4_system(reps=2)
    p4, cell = torch.from_numpy(p4), torch.from_numpy(cell)
    a = geometry.radius_graph(p4, 4.0, cell, [True] * 3, max_neighbors=10)
    b = OG.neighbor_list(p4, 4.0, cell, [True] * 3, max_neighbors=10)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_generators_are_seeded_and_sized():
    p1, Z1 = synthetic.c1_system()
    p2, Z2 = synthetic.c1_system()
    assert np.array_equal(p1, p2) and len(Z1) == 24 and set(Z1) <= {1, 6, 7, 8}
    d = np.linalg.norm(p1[:, None] - p1[None], axis=-1) + np.eye(24) * 9
    assert d.min() >= 0.9
    p4, Z4, cell = synthetic.c4_system()
    assert p4.shape == (2048, 3) and np.all(Z4 == 29) and np.allclose(np.diag(cell), 8 * 3.61)
    ei, vec = synthetic.c2_graph()
    assert ei.shape == (2, 204800) and np.all(ei[0] != ei[1]) and np.all(np.diff(ei[1]) >= 0)
    assert np.allclose(np.linalg.norm(vec, axis=1).min(), 0.8, atol=1e-3)


def test_orb_zbl_forces_and_stress_are_derivatives_of_its_energy():
    """Host ZBL pair repulsion: forces = -dE/dpos and stress = dE/dstrain / V by fp64 finite
    differences (orb_model.py:491-585), on a short-contact periodic pair system."""
    import numpy as np
    import torch
    from tt_atom import orb_calculator as OC
    from tt_atom import orb
    radii = np.full(120, 1.1)
    pos = np.array([[0.0, 0.0, 0.0], [1.3, 0.2, 0.1], [0.4, 1.5, 0.3]])
    Z = np.array([6, 8, 1])
    cell = np.eye(3) * 4.0
    bg = orb.assemble_orb([(pos, Z, cell, [True] * 3)], 3.0, 20)
    args = (bg.Z, bg.senders, bg.receivers)
    e, F, s = OC.zbl_energy_forces_stress(*args, bg.pos.double(), bg.cell_shift, radii, cell)
    assert e > 0
    h = 1e-6
    for a, k in ((0, 0), (1, 2), (2, 1)):
        p1, p2 = bg.pos.double().clone(), bg.pos.double().clone()
        p1[a, k] += h
        p2[a, k] -= h
        e1 = OC.zbl_energy_forces_stress(*args, p1, bg.cell_shift, radii)[0]
        e2 = OC.zbl_energy_forces_stress(*args, p2, bg.cell_shift, radii)[0]
        assert abs(-(e1 - e2) / (2 * h) - F[a, k]) < 1e-6 * max(1.0, abs(F[a, k]))
    # stress: strain the positions, the cell and therefore the image shifts together
    eps = np.zeros((3, 3))
    eps[0, 1] = eps[1, 0] = h
    vals = []
    for sgn in (1, -1):
        M = np.eye(3) + sgn * eps
        vals.append(OC.zbl_energy_forces_stress(*args, bg.pos.double() @ torch.tensor(M),
                                                bg.cell_shift.double() @ torch.tensor(M),
                                                radii)[0])
    fd = (vals[0] - vals[1]) / (2 * h) / 2 / 64.0          # d/d eps_01 of a symmetric strain / V
    assert abs(fd - s[5]) < 1e-6 * max(1.0, abs(s[5]))


def test_disjoint_assemble_block_diagonal():
    """disjoint.assemble (disjoint.py:123-159): every edge stays inside its system, edges are the
    per-system graphs offset by the node count, and sys_emb rows follow each system's charge /
    spin."""
    from tt_atom import disjoint
    cfg = dict(synthetic.CFG_UMA_S, sphere_channels=8, hidden_channels=8, edge_channels=8,
               num_distance_basis=8, num_layers=1)
    w, _ = synthetic.random_uma_bundle(cfg, 5)
    mols = [synthetic.c3_system(seed=50 + k, n=n, radius=4.0 + k) for k, n in enumerate((9, 14, 11))]
    systems = [dict(positions=p, numbers=z, charge=float(k), spin=1.0)
               for k, (p, z) in enumerate(mols)]
    bg = disjoint.assemble(systems, 5.0, w, 8, task="omol")
    assert bg.K == 3 and bg.natoms == [9, 14, 11]
    off = 0
    for k, (p, z) in enumerate(mols):
        n = len(z)
        ei, _ = geometry.radius_graph(torch.from_numpy(p).float(), 5.0)
        m = (bg.edge_index[1] >= off) & (bg.edge_index[1] < off + n)
        assert torch.equal(bg.edge_index[:, m], ei + off)
        assert bool(((bg.edge_index[0, m] >= off) & (bg.edge_index[0, m] < off + n)).all())
        se = geometry.csd_embedding(w, torch.tensor([float(k)]), torch.tensor([1.0]), 8,
                                    dataset="omol")
        assert torch.equal(bg.sys_emb[off:off + n], se.expand(n, -1))
        assert bool((bg.batch[off:off + n] == k).all())
        off += n
    seg = bg.segment_matrix()
    assert torch.equal(seg.sum(0), torch.ones(off)) and seg.sum(1).tolist() == [9.0, 14.0, 11.0]


def _np_csr(keys, n):
    ptr = np.zeros(n + 1, np.int64)
    ptr[1:] = np.cumsum(np.bincount(keys, minlength=n))
    return ptr


def test_graph_context_topology_matches_numpy():
    """Destination-sorted edge order, CSR offsets and the src permutation (built with torch on
    the engine's device) equal numpy's stable sorts; malformed edge lists raise."""
    import pytest
    from tt_atom.model import GraphContext
    rng = np.random.default_rng(4)
    N, E = 37, 500
    ei = rng.integers(0, N, size=(2, E))
    ei[:, :60] = 5                                                # repeated keys: stability matters
    Z = rng.integers(1, 9, size=N)
    shift = rng.normal(size=(E, 3)).astype(np.float32)
    g = GraphContext("cpu", edge_index=torch.from_numpy(ei), num_nodes=N,
                     atomic_numbers=torch.from_numpy(Z), edge_cell_shift=torch.from_numpy(shift))
    order = np.argsort(ei[1], kind="stable")
    s, t = ei[0][order], ei[1][order]
    assert np.array_equal(g.order.numpy(), order)
    assert np.array_equal(g.src.numpy(), s) and np.array_equal(g.tgt.numpy(), t)
    assert np.array_equal(g.tgt_ptr.numpy(), _np_csr(t, N))
    assert np.array_equal(g.src_ptr.numpy(), _np_csr(s, N))
    assert np.array_equal(g.src_perm.numpy(), np.argsort(s, kind="stable"))
    assert np.array_equal(g.zsrc.numpy(), Z[s]) and np.array_equal(g.ztgt.numpy(), Z[t])
    assert np.array_equal(g.shift.numpy(), shift[order])
    assert g.max_in_degree == int(np.bincount(t, minlength=N).max())
    assert g.src.dtype == torch.int32 and g.src_perm.dtype == torch.int32
    for bad in (np.array([[0, N], [1, 2]]), np.array([[0, -1], [1, 2]])):
        with pytest.raises(ValueError):
            GraphContext("cpu", edge_index=torch.from_numpy(bad), num_nodes=N,
                         atomic_numbers=torch.from_numpy(Z))


def test_orb_graph_topology_matches_numpy():
    import pytest
    from tt_atom.orb import OrbGraph
    rng = np.random.default_rng(5)
    natoms = [7, 12, 5]
    N = sum(natoms)
    off = np.concatenate([[0], np.cumsum(natoms)])
    snd, rcv = [], []
    for k, n in enumerate(natoms):                                  # edges inside each system
        snd.append(rng.integers(0, n, 40) + off[k])
        rcv.append(rng.integers(0, n, 40) + off[k])
    s, r = np.concatenate(snd), np.concatenate(rcv)
    g = OrbGraph("cpu", senders=torch.from_numpy(s), receivers=torch.from_numpy(r), num_nodes=N,
                 atomic_numbers=torch.ones(N, dtype=torch.long), natoms=natoms)
    order = np.argsort(s, kind="stable")
    s_s, r_s = s[order], r[order]
    assert np.array_equal(g.order.numpy(), order)
    assert np.array_equal(g.send.numpy(), s_s) and np.array_equal(g.recv.numpy(), r_s)
    assert np.array_equal(g.send_ptr.numpy(), _np_csr(s_s, N))
    assert np.array_equal(g.recv_ptr.numpy(), _np_csr(r_s, N))
    assert np.array_equal(g.recv_perm.numpy(), np.argsort(r_s, kind="stable"))
    assert np.array_equal(g.batch.numpy(), np.repeat(np.arange(3), natoms))
    assert np.array_equal(g.seg_ptr.numpy(), off)
    with pytest.raises(ValueError, match="joins two systems"):
        OrbGraph("cpu", senders=torch.tensor([0]), receivers=torch.tensor([8]), num_nodes=N,
                 atomic_numbers=torch.ones(N, dtype=torch.long), natoms=natoms)
    with pytest.raises(ValueError, match="out of range"):
        OrbGraph("cpu", senders=torch.tensor([0]), receivers=torch.tensor([N]), num_nodes=N,
                 atomic_numbers=torch.ones(N, dtype=torch.long), natoms=natoms)


class _Atoms:
    """The three members of ase.Atoms the cache and the front door read."""

    def __init__(self, numbers, pbc=False, info=None):
        self.numbers, self.pbc, self.info = np.asarray(numbers), pbc, dict(info or {})

    def get_atomic_numbers(self):
        return self.numbers

    def get_pbc(self):
        return np.broadcast_to(np.asarray(self.pbc, dtype=bool), (3,))


def test_bundle_cache_key_and_hits(tmp_path):
    """The reference's cache naming: reduced composition (H2O == H4O2, any atom order) hashed as
    sha1("Z:count;...")[:12]; charge, spin, task and an explicit checkpoint each change the name;
    a hit returns the file, a miss raises with the path."""
    import hashlib
    import pytest
    from tt_atom import bundle_cache as BC
    assert BC.reduced_composition([8, 1, 1]) == ((1, 2), (8, 1))
    assert BC.reduced_composition([1, 8, 1, 1, 8, 1]) == ((1, 2), (8, 1))
    assert BC.composition_hash([1, 1, 8]) == hashlib.sha1(b"1:2;8:1").hexdigest()[:12]
    p = BC.bundle_path("uma-s-1", "omol", [8, 1, 1], 0, 1, cache_dir=tmp_path)
    assert p == tmp_path / f"uma-s-1_omol_{hashlib.sha1(b'1:2;8:1').hexdigest()[:12]}_c0_s1.npz"
    assert p == BC.bundle_path("uma-s-1", "omol", [1, 8, 1, 1, 8, 1], 0, 1, cache_dir=tmp_path)
    others = {BC.bundle_path("uma-s-1", "omol", [8, 1, 1], 1, 1, cache_dir=tmp_path),
              BC.bundle_path("uma-s-1", "omol", [8, 1, 1], 0, 2, cache_dir=tmp_path),
              BC.bundle_path("uma-s-1", "omat", [8, 1, 1], 0, 1, cache_dir=tmp_path),
              BC.bundle_path("uma-s-1", "omol", [8, 1, 1], 0, 1, cache_dir=tmp_path,
                             checkpoint=tmp_path / "ckpt.pt")}
    assert p not in others and len(others) == 4
    assert BC.infer_task(_Atoms([1], pbc=True)) == "omat"
    assert BC.infer_task(_Atoms([1], pbc=[True, True, False])) == "omol"
    with pytest.raises(BC.BundleNotCached, match="export_weights"):
        BC.get_or_build(_Atoms([8, 1, 1]), cache_dir=tmp_path)
    p.write_bytes(b"")
    assert BC.get_or_build(_Atoms([1, 8, 1]), cache_dir=tmp_path) == p


def test_orb_weight_cache_and_front_door(tmp_path):
    import pytest
    from tt_atom import auto, calculator, orb_weight_cache as OWC
    assert OWC.weights_path("orb-v3-direct-20-omat", tmp_path) == tmp_path / "direct-20-omat.npz"
    with pytest.raises(ValueError, match="unknown Orb checkpoint"):
        OWC.weights_path("orb-v4", tmp_path)
    with pytest.raises(OWC.WeightsNotCached):
        OWC.get_or_build("orb-v3-conservative-omol", cache_dir=tmp_path)
    assert auto._family("UMA-s-1") == "uma" and auto._family("orb-v3-direct-omol") == "orb"
    with pytest.raises(ValueError, match="unknown model"):
        auto.Calculator(_Atoms([1]), "mace")
    with pytest.raises(ValueError, match="needs `atoms`"):
        auto.Calculator(None, "uma-s-1")
    with pytest.raises(ValueError, match="only to UMA"):
        auto.Calculator(None, "orb-v3-direct-omol", task="omol")
    # a cache hit reaches the calculator class (which needs ase where it is absent); charge and
    # spin from atoms.info win and the resolved values are stamped back
    from tt_atom import bundle_cache as BC
    atoms = _Atoms([8, 1, 1], info={"spin": 3})
    BC.bundle_path("uma-s-1", "omol", [8, 1, 1], 0, 3, cache_dir=tmp_path).write_bytes(b"")
    if not calculator.HAVE_ASE:
        with pytest.raises(ImportError, match="needs ase"):
            auto.Calculator(atoms, "uma-s-1", cache_dir=tmp_path)
        assert atoms.info == {"spin": 3, "charge": 0}


def test_orb_batched_host_terms_equal_per_system():
    """The vectorised host pieces of OrbSession.evaluate_batch against their one-system forms:
    the conditioning embedding bit for bit, the union ZBL energies / forces (mean and sum
    aggregation) and the batched energy normaliser to fp64 rounding."""
    from oracle import orb as O
    from tt_atom import orb, orb_calculator as OC
    cfg = dict(synthetic.CFG_ORB_TINY, has_charge_spin_cond=True)
    w = synthetic.random_orb_weights(cfg, 3)
    charges, spins, natoms = [0.0, 1.0, -2.0], [1.0, 0.0, 3.0], [4, 2, 5]
    emb = orb.charge_spin_embedding_batch(w, cfg["latent_dim"], charges, spins, natoms)
    ref = torch.cat([O.charge_spin_embedding(w, q, s, n) for q, s, n in zip(charges, spins,
                                                                             natoms)])
    assert torch.equal(emb, ref)
    systems = synthetic.ethanol_batch(3) + synthetic.si_batch(2)
    bg = orb.assemble_orb(systems, 6.0, 120)
    radii = np.full(120, 0.9)
    batch = bg.batch.long()
    for agg in ("mean", "sum"):
        e, f = OC.zbl_batch(bg.Z, bg.senders, bg.receivers, bg.pos, bg.cell_shift, batch,
                            bg.natoms, radii, agg)
        off = 0
        for k, n in enumerate(bg.natoms):
            m = (bg.senders >= off) & (bg.senders < off + n)
            ek, fk, _ = OC.zbl_energy_forces_stress(bg.Z[off:off + n], bg.senders[m] - off,
                                                    bg.receivers[m] - off, bg.pos[off:off + n],
                                                    bg.cell_shift[m], radii, aggregation=agg)
            assert abs(e[k] - ek) <= 1e-12 * max(1.0, abs(ek))
            assert np.abs(f[off:off + n] - fk).max() <= 1e-10
            off += n
        assert np.abs(e).max() > 0
    raw = torch.tensor([0.3, -1.2, 0.7, 2.0, -0.4], dtype=torch.float64)
    eb = orb.denormalize_energy_batch(raw, bg.Z, batch, bg.natoms, w)
    off = 0
    for k, n in enumerate(bg.natoms):
        e1 = orb.denormalize_energy(raw[k], bg.Z[off:off + n], n, w)
        assert abs(float(eb[k]) - float(e1)) <= 1e-12 * max(1.0, abs(float(e1)))
        off += n


def test_batch_refused_when_it_does_not_match_the_merged_bundle(tmp_path):
    """A bundle carrying merge inputs (ref@*) refuses a batch whose reduced composition or
    (charge, spin) differs from them (calculator.py:191-218); one without them accepts any."""
    cfg = dict(synthetic.CFG_UMA_S, sphere_channels=8, hidden_channels=8, edge_channels=8,
               num_distance_basis=8, num_layers=1)
    w, host = synthetic.random_uma_bundle(cfg, 5)
    eth = synthetic.ethanol_batch(2)
    pos0, Z0 = eth[0]["positions"], eth[0]["numbers"]
    ref = dict(energy=-1.5, forces=np.zeros((len(Z0), 3)), pos=pos0, atomic_numbers=Z0,
               charge=0.0, spin=1.0)
    p = tmp_path / "merged.npz"
    weights.save_bundle(p, cfg, w, host, reference=ref)
    b = weights.WeightBundle.load(p)
    r = b.reference
    assert r["charge"] == 0.0 and r["spin"] == 1.0 and r["energy"] == -1.5
    assert np.array_equal(r["atomic_numbers"], Z0) and r["cell"] is None
    ok = list(eth)
    calculator.check_batch_matches_bundle(b, ok)
    # water: a different reduced composition
    Zw = np.array([8, 1, 1])
    wrong = ok + [dict(positions=np.zeros((3, 3)), numbers=Zw, charge=0.0, spin=1.0)]
    with pytest.raises(ValueError, match="reduced composition"):
        calculator.check_batch_matches_bundle(b, wrong)
    # twice the molecule has the same reduced composition: accepted
    dbl = dict(positions=np.concatenate([pos0, pos0 + 10.0]), numbers=np.concatenate([Z0, Z0]),
               charge=0.0, spin=1.0)
    calculator.check_batch_matches_bundle(b, ok + [dbl])
    with pytest.raises(ValueError, match="charge, spin"):
        calculator.check_batch_matches_bundle(
            b, ok + [dict(positions=pos0, numbers=Z0, charge=1.0, spin=1.0)])
    with pytest.raises(ValueError, match="charge, spin"):
        calculator.check_batch_matches_bundle(
            b, [dict(positions=pos0, numbers=Z0, charge=0.0, spin=2.0)])
    p2 = tmp_path / "plain.npz"
    weights.save_bundle(p2, cfg, w, host)
    b2 = weights.WeightBundle.load(p2)
    assert b2.reference is None
    calculator.check_batch_matches_bundle(b2, wrong)


def test_assemble_orb_refuses_over_cap_by_default():
    """As the reference (disjoint.py:188-197): a system whose sender or receiver degree exceeds
    max_num_neighbors is refused; truncate=True keeps each sender's nearest ones instead."""
    from tt_atom import orb
    systems = synthetic.c5_systems(K=2)
    with pytest.raises(ValueError, match="max_num_neighbors=20"):
        orb.assemble_orb(systems, 6.0, 20)
    bg = orb.assemble_orb(systems, 6.0, 20, truncate=True)
    assert int(torch.bincount(bg.senders).max()) <= 20
    big = orb.assemble_orb(systems, 6.0, 1000)
    n = big.pos.shape[0]
    deg = max(int(torch.bincount(big.senders, minlength=n).max()),
              int(torch.bincount(big.receivers, minlength=n).max()))
    assert deg > 20
    orb.assemble_orb(systems, 6.0, deg)           # exactly at the cap: accepted
    with pytest.raises(ValueError):
        orb.assemble_orb(systems, 6.0, deg - 1)
    # an uncapped graph within the cap is the same with or without truncation
    same = orb.assemble_orb(systems, 6.0, deg, truncate=True)
    assert torch.equal(same.senders, big.senders) and torch.equal(same.receivers, big.receivers)


def test_radius_graph_device_checks_node_ranges_on_the_host():
    """Bad node ranges raise before anything reaches the device."""
    pos = torch.zeros(4, 3)
    lo = torch.tensor([0, 0, 2, 2])
    hi = torch.tensor([2, 2, 4, 4])
    for bad in ((lo[:3], hi), (lo, hi[:2]), (torch.tensor([0, 0, 2, -1]), hi),
                (lo, torch.tensor([2, 2, 4, 5])), (torch.tensor([0, 3, 2, 2]), hi)):
        with pytest.raises(ValueError, match="node_ranges"):
            geometry.radius_graph_device(pos, 5.0, node_ranges=bad, device="cpu")
