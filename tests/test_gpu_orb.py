"""GPU parity of the Orb-v3 path (HIP kernels through the C ABI) against the CPU oracle."""
import math

import numpy as np
import pytest
import torch

from oracle import orb as O
from tt_atom import orb as orb
from tt_atom import synthetic as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from tt_atom import _native
    _native.load()
    return _native


def _edges(seed, n_nodes=40, n_edges=400, r_hi=6.5):
    g = torch.Generator().manual_seed(seed)
    pos = 3.0 * torch.randn(n_nodes, 3, generator=g)
    s = torch.randint(n_nodes, (n_edges,), generator=g)
    r = (s + torch.randint(1, n_nodes, (n_edges,), generator=g)) % n_nodes
    d = torch.nn.functional.normalize(torch.randn(n_edges, 3, generator=g), dim=1)
    length = 0.5 + (r_hi - 0.5) * torch.rand(n_edges, generator=g)
    shift = d * length[:, None] - (pos[r] - pos[s])           # vectors of controlled length
    return pos, s, r, shift


def test_edge_features_and_vjp(nat):
    pos, s, r, shift = _edges(3)
    E = s.numel()
    dev = "cuda"
    vec, feat, cut = (torch.empty(E, 3, device=dev), torch.empty(E, 128, device=dev),
                      torch.empty(E, device=dev))
    i32 = lambda t: t.to(torch.int32).to(dev)
    nat.orb_edge_features(pos.to(dev), i32(s), i32(r), shift.to(dev), 6.0, 8, vec, feat, cut)
    p64 = pos.double().requires_grad_(True)
    rf, rc, rv = O.edge_features(p64, s, r, shift.double())
    # fp32 rounding of the sine argument n pi r / r_max (up to ~27) bounds the absolute error
    # of the features (values up to ~6) at a few 1e-6
    assert (feat.cpu().double() - rf).abs().max() < 1e-5
    assert (cut.cpu().double() - rc[:, 0]).abs().max() < 1e-6
    assert (vec.cpu().double() - rv).abs().max() < 2e-6
    g = torch.Generator().manual_seed(5)
    gf, gc = torch.randn(E, 128, generator=g), torch.randn(E, generator=g)
    g_vec = torch.empty(E, 3, device=dev)
    nat.orb_edge_features_bwd(vec, gf.to(dev), gc.to(dev), 6.0, 8, g_vec)
    v64 = rv.detach().clone().requires_grad_(True)
    r64 = torch.linalg.norm(v64, dim=1)
    u64 = torch.nn.functional.normalize(v64, dim=1)
    f64 = (O.envelope(r64)[:, None] * (O.bessel(r64)[:, :, None] * O.sph_l3(u64)[:, None, :])
           .reshape(E, -1))
    ref = torch.autograd.grad([f64, O.envelope(r64)], v64, [gf.double(), gc.double()])[0]
    err = (g_vec.cpu().double() - ref).abs().max() / ref.abs().max()
    assert err < 1e-5, err


def test_row_kernels(nat):
    g = torch.Generator().manual_seed(7)
    R, C = 300, 256
    dev = "cuda"
    h, w, x = (torch.randn(R, C, generator=g), 1 + 0.1 * torch.randn(C, generator=g),
               torch.randn(R, C, generator=g))
    aw, ab = 0.1 * torch.randn(2 * C, generator=g), torch.randn(2, generator=g)
    u, xn, inv, sig = (torch.empty(R, C, device=dev), torch.empty(R, C, device=dev),
                       torch.empty(R, device=dev), torch.empty(R, 2, device=dev))
    nat.rms_residual(h.to(dev), w.to(dev), x.to(dev), u, xn, inv, aw.to(dev), ab.to(dev), sig)
    y = O.rmsnorm(h.double(), w.double())
    assert (u.cpu().double() - y).abs().max() < 2e-6
    assert (xn.cpu().double() - (x.double() + y)).abs().max() < 4e-6
    xs = x.double() + y
    sr = torch.sigmoid(xs @ aw[:C].double() + ab[0])
    ss = torch.sigmoid(xs @ aw[C:].double() + ab[1])
    assert (sig.cpu().double() - torch.stack([sr, ss], 1)).abs().max() < 2e-6
    # RMSNorm backward vs autograd
    gy = torch.randn(R, C, generator=g)
    hd = h.double().requires_grad_(True)
    ref = torch.autograd.grad(O.rmsnorm(hd, w.double()), hd, gy.double())[0]
    gh = torch.empty(R, C, device=dev)
    nat.rms_bwd(gy.to(dev), h.to(dev), w.to(dev), inv, gh)
    assert (gh.cpu().double() - ref).abs().max() < 5e-6


def _tiny_batch(K=3, seed=11, cfg=None, n_min=6, n_max=14, side=5.0):
    cfg = dict(S.CFG_ORB_TINY if cfg is None else cfg)
    w = S.random_orb_weights(cfg, seed + S.WEIGHT_SEED_OFFSET)
    systems = S.c5_systems(seed, K=K, n_min=n_min, n_max=n_max, side=side)
    bg = orb.assemble_orb(systems, cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
    return cfg, w, systems, bg


def _oracle(cfg, w, bg, dtype=torch.float64, **kw):
    return O.energy_and_forces(w, cfg, bg.pos.to(dtype), bg.Z, bg.senders, bg.receivers,
                               bg.cell_shift.to(dtype), bg.batch, bg.natoms, **kw)


def _check(cfg, w, bg, raw, F, tol_e=1e-6, tol_f=1e-4, oracle_dtype=torch.float64):
    ref_raw, ref_F = _oracle(cfg, w, bg, dtype=oracle_dtype)
    ref_raw, ref_F = ref_raw.double(), ref_F.double()
    off = 0
    for k, n in enumerate(bg.natoms):
        e = float(orb.denormalize_energy(raw[k], bg.Z[off:off + n], n, w))
        e_ref = float(O.denormalize_energy(ref_raw[k], bg.Z[off:off + n], n,
                                           w["energy_head.normalizer.bn.running_mean"],
                                           w["energy_head.normalizer.bn.running_var"],
                                           w["energy_head.reference.linear.weight"]))
        assert abs(e - e_ref) <= tol_e * max(1.0, abs(e_ref)), (k, e, e_ref)
        f = orb.denormalize_forces(F[off:off + n], n, w)
        f_ref = O.denormalize_forces(ref_F[off:off + n], n,
                                     w["energy_head.normalizer.bn.running_var"])
        assert (f - f_ref).abs().max() <= tol_f, (k, (f - f_ref).abs().max())
        off += n


def test_orb_tiny_batch_matches_oracle(nat):
    cfg, w, _, bg = _tiny_batch()
    model = orb.OrbModel(w, cfg)
    raw, F = orb.energy_and_forces_batch(model, pos=bg.pos, senders=bg.senders,
                                         receivers=bg.receivers, atomic_numbers=bg.Z,
                                         natoms=bg.natoms, cell_shift=bg.cell_shift)
    _check(cfg, w, bg, raw, F)


def test_orb_conditioning_and_batch_consistency(nat):
    cfg = dict(S.CFG_ORB_TINY, has_charge_spin_cond=True)
    cfg, w, systems, bg = _tiny_batch(K=2, seed=12, cfg=cfg)
    model = orb.OrbModel(w, cfg)
    cond = torch.cat([model.charge_spin_embedding(1.0, 2.0, bg.natoms[0]),
                      model.charge_spin_embedding(0.0, 1.0, bg.natoms[1])])
    raw, F = orb.energy_and_forces_batch(model, pos=bg.pos, senders=bg.senders,
                                         receivers=bg.receivers, atomic_numbers=bg.Z,
                                         natoms=bg.natoms, cell_shift=bg.cell_shift,
                                         cond_nodes=cond)
    ref_raw, ref_F = _oracle(cfg, w, bg, cond_nodes=cond.double())
    assert (raw - ref_raw).abs().max() < 1e-6 * max(1.0, ref_raw.abs().max().item())
    assert (F.double() - ref_F).abs().max() < 2e-6
    # each system alone gives the same result as inside the batch
    off = 0
    for k, sysk in enumerate(systems):
        one = orb.assemble_orb([sysk], cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
        n = bg.natoms[k]
        r1, F1 = orb.energy_and_forces_batch(model, pos=one.pos, senders=one.senders,
                                             receivers=one.receivers, atomic_numbers=one.Z,
                                             natoms=one.natoms, cell_shift=one.cell_shift,
                                             cond_nodes=cond[off:off + n])
        assert abs(float(r1[0]) - float(raw[k])) < 1e-6 * max(1.0, abs(float(raw[k])))
        assert (F1 - F[off:off + n]).abs().max() < 2e-6
        off += n


def test_orb_periodic_stress_matches_oracle(nat):
    cfg = dict(S.CFG_ORB_TINY)
    w = S.random_orb_weights(cfg, 99)
    pos, Z, cell = S.c4_system(seed=4, reps=2, a=3.61, noise=0.05, Z=29)
    bg = orb.assemble_orb([(pos, Z, cell, [True] * 3)], cfg["cutoff"],
                          cfg["max_num_neighbors"], truncate=True)
    model = orb.OrbModel(w, cfg)
    raw, F, vir = orb.energy_and_forces(model, pos=bg.pos, senders=bg.senders,
                                        receivers=bg.receivers, atomic_numbers=bg.Z,
                                        cell_shift=bg.cell_shift, compute_stress=True)
    r_raw, r_F, r_vir = _oracle(cfg, w, bg, compute_stress=True)
    n = bg.natoms[0]
    assert abs(raw - float(r_raw[0])) < 1e-6 * max(1.0, abs(float(r_raw[0])))
    s = orb.denormalize_stress(vir, n, cell, w)
    s_ref = orb.denormalize_stress(r_vir, n, cell, w)
    assert (s - s_ref).abs().max() < 1e-5, (s, s_ref)
    f = orb.denormalize_forces(F, n, w)
    f_ref = orb.denormalize_forces(r_F, n, w)
    assert (f - f_ref).abs().max() < 1e-4


def test_orb_c5_architecture_reduced_batch(nat):
    """C5 architecture (latent 256, hidden 1024, 5 layers, cap 20) on 8 of its molecules."""
    cfg = dict(S.CFG_ORB_C5)
    w = S.random_orb_weights(cfg, S.SEEDS["C5"] + S.WEIGHT_SEED_OFFSET)
    systems = S.c5_systems()[:8]
    bg = orb.assemble_orb(systems, cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
    model = orb.OrbModel(w, cfg)
    raw, F = orb.energy_and_forces_batch(model, pos=bg.pos, senders=bg.senders,
                                         receivers=bg.receivers, atomic_numbers=bg.Z,
                                         natoms=bg.natoms, cell_shift=bg.cell_shift)
    _check(cfg, w, bg, raw, F)
    # a second call on the same engine inputs is bitwise identical (deterministic reductions)
    raw2, F2 = orb.energy_and_forces_batch(model, pos=bg.pos, senders=bg.senders,
                                           receivers=bg.receivers, atomic_numbers=bg.Z,
                                           natoms=bg.natoms, cell_shift=bg.cell_shift)
    assert torch.equal(raw, raw2) and torch.equal(F, F2)


def test_orb_c5_full_batch(nat):
    """The full C5 workload (256 molecules, 10,150 atoms, E = 196,555) against the fp32 oracle."""
    cfg = dict(S.CFG_ORB_C5)
    w = S.random_orb_weights(cfg, S.SEEDS["C5"] + S.WEIGHT_SEED_OFFSET)
    bg = orb.assemble_orb(S.c5_systems(), cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
    model = orb.OrbModel(w, cfg)
    raw, F = orb.energy_and_forces_batch(model, pos=bg.pos, senders=bg.senders,
                                         receivers=bg.receivers, atomic_numbers=bg.Z,
                                         natoms=bg.natoms, cell_shift=bg.cell_shift)
    # the fp64 oracle of the whole batch would hold ~50 GB of saved activations
    _check(cfg, w, bg, raw, F, oracle_dtype=torch.float32)


# bf16 operands (8 significant bits, relative rounding 2^-9 per operand) in every edge- and
# node-level product of the 5-layer, 1024-wide C5 network, with fp32 accumulation: the error of
# the raw energy and of the forces is a few 1e-3 of their magnitude, against ~1e-7 for the fp32
# arithmetic.  Stated bounds: raw energy within 2e-2 of max(1, |raw|) per system, forces within
# 4e-2 of the largest |F| of the batch (both relative, vs the fp64 oracle).
BF16_TOL_RAW, BF16_TOL_F = 2e-2, 4e-2


def _bf16_errors(cfg, w, bg, raw, F, oracle_dtype=torch.float64):
    ref_raw, ref_F = _oracle(cfg, w, bg, dtype=oracle_dtype)
    ref_raw, ref_F = ref_raw.double(), ref_F.double()
    e_raw = ((raw.double() - ref_raw).abs() / ref_raw.abs().clamp_min(1.0)).max().item()
    e_f = (F.double() - ref_F).abs().max().item() / ref_F.abs().max().item()
    return e_raw, e_f


def test_orb_c5_bf16_matches_oracle(nat):
    """C5 architecture with bf16 GEMM operands (BASELINE configs[4] 'fp32/bf16') on 8 of its
    molecules against the fp64 oracle, within the stated bf16 bounds; the fp32 default on the
    same batch is checked at its own tolerance alongside, and bf16 must actually differ from it
    (the bf16 kernels ran)."""
    cfg = dict(S.CFG_ORB_C5)
    w = S.random_orb_weights(cfg, S.SEEDS["C5"] + S.WEIGHT_SEED_OFFSET)
    bg = orb.assemble_orb(S.c5_systems()[:8], cfg["cutoff"], cfg["max_num_neighbors"],
                          truncate=True)
    kw = dict(pos=bg.pos, senders=bg.senders, receivers=bg.receivers, atomic_numbers=bg.Z,
              natoms=bg.natoms, cell_shift=bg.cell_shift)
    raw16, F16 = orb.energy_and_forces_batch(orb.OrbModel(w, cfg, precision="bf16"), **kw)
    raw32, F32 = orb.energy_and_forces_batch(orb.OrbModel(w, cfg), **kw)
    e_raw, e_f = _bf16_errors(cfg, w, bg, raw16, F16)
    print(f"C5 bf16 (8 molecules, E = {bg.senders.numel()}): raw energy rel {e_raw:.2e}, "
          f"forces rel {e_f:.2e}", flush=True)
    assert e_raw < BF16_TOL_RAW and e_f < BF16_TOL_F, (e_raw, e_f)
    assert not torch.equal(F16, F32)
    _check(cfg, w, bg, raw32, F32)


def test_orb_c5_bf16_full_batch_properties(nat):
    """The full C5 batch (256 molecules) in bf16: (i) the first 128 molecules as a batch of their
    own give the same per-system results as inside the full batch (every kernel is row-local and
    every reduction runs in a fixed order, so the slices agree to fp32 rounding; the sub-batch
    has at least 4096 nodes so that its node-level products take the same bf16 kernel as the full
    batch's -- smaller products run on the fp32 kernel); (ii) a rigid translation of every
    molecule leaves the energies unchanged and the forces unchanged within the bf16 bounds;
    (iii) the forces of every molecule sum to zero within bf16 rounding."""
    cfg = dict(S.CFG_ORB_C5)
    w = S.random_orb_weights(cfg, S.SEEDS["C5"] + S.WEIGHT_SEED_OFFSET)
    systems = S.c5_systems()
    model = orb.OrbModel(w, cfg, precision="bf16")

    def run(sys_list):
        bg = orb.assemble_orb(sys_list, cfg["cutoff"], cfg["max_num_neighbors"], truncate=True)
        raw, F = orb.energy_and_forces_batch(model, pos=bg.pos, senders=bg.senders,
                                             receivers=bg.receivers, atomic_numbers=bg.Z,
                                             natoms=bg.natoms, cell_shift=bg.cell_shift)
        return bg, raw.double(), F.double()

    K = 128
    bg, raw, F = run(systems)
    bgK, rawK, FK = run(systems[:K])
    nK = sum(bgK.natoms)
    assert nK >= 4096, nK
    d_raw = ((raw[:K] - rawK).abs() / rawK.abs().clamp_min(1.0)).max().item()
    d_f = (F[:nK] - FK).abs().max().item() / FK.abs().max().item()
    print(f"C5 bf16 full batch vs first {K} ({nK} atoms): raw rel {d_raw:.2e}, forces rel "
          f"{d_f:.2e} (exact: {torch.equal(raw[:K], rawK) and torch.equal(F[:nK], FK)})",
          flush=True)
    assert d_raw < 1e-5 and d_f < 1e-4, (d_raw, d_f)
    shift = np.array([3.7, -1.2, 0.55], np.float32)
    _, raw_t, F_t = run([(p + shift, z) for p, z in systems])
    t_raw = ((raw_t - raw).abs() / raw.abs().clamp_min(1.0)).max().item()
    t_f = (F_t - F).abs().max().item() / F.abs().max().item()
    print(f"C5 bf16 translation: raw rel {t_raw:.2e}, forces rel {t_f:.2e}", flush=True)
    assert t_raw < BF16_TOL_RAW and t_f < BF16_TOL_F, (t_raw, t_f)
    net = torch.zeros(len(bg.natoms), 3, dtype=torch.float64).index_add_(0, bg.batch.long(), F)
    net_rel = net.abs().max().item() / F.abs().max().item()
    print(f"C5 bf16 net force per molecule: {net_rel:.2e} of max |F|", flush=True)
    assert net_rel < BF16_TOL_F


def test_orb_session_single_and_batch(nat, tmp_path):
    """OrbSession (the array-level core of OrbCalculator): a saved bundle round trip, one system
    against the oracle, and evaluate_batch == per-system evaluate (ZBL on, with a synthetic
    covalent-radius table, since ase is absent)."""
    from tt_atom import orb_calculator as OC
    cfg = dict(S.CFG_ORB_TINY)
    w = S.random_orb_weights(cfg, 31)
    path = tmp_path / "orb.npz"
    orb.save_orb_bundle(path, cfg, w)
    systems = S.c5_systems(13, K=3, n_min=6, n_max=12, side=5.0)
    radii = np.full(120, 0.45)
    sess = OC.OrbSession(str(path), pair_repulsion=True, covalent_radii=radii)
    res = [sess.evaluate(p, z) for p, z in systems]
    # oracle: raw GNN energy / forces + the same host ZBL
    for (p, z), r in zip(systems, res):
        bg = orb.assemble_orb([(p, z)], cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
        raw, F = _oracle(cfg, w, bg)
        n = bg.natoms[0]
        e_z, f_z, _ = OC.zbl_energy_forces_stress(bg.Z, bg.senders, bg.receivers, bg.pos,
                                                  bg.cell_shift, radii)
        e_ref = float(O.denormalize_energy(raw[0], bg.Z, n,
                                           w["energy_head.normalizer.bn.running_mean"],
                                           w["energy_head.normalizer.bn.running_var"],
                                           w["energy_head.reference.linear.weight"])) + e_z
        f_ref = O.denormalize_forces(F, n, w["energy_head.normalizer.bn.running_var"]).numpy() + f_z
        assert abs(r["energy"] - e_ref) <= 1e-6 * max(1.0, abs(e_ref))
        assert np.abs(r["forces"] - f_ref).max() <= 1e-4
    batch = sess.evaluate_batch(systems)
    for k, r in enumerate(res):
        assert abs(batch["energy"][k] - r["energy"]) <= 1e-6 * max(1.0, abs(r["energy"]))
        assert np.abs(batch["forces"][k] - r["forces"]).max() <= 2e-5


def test_orb_session_systems_without_edges(nat, tmp_path):
    """A system with no edge inside the cutoff (one atom; two atoms 20 A apart) is refused with
    ValueError, alone and inside a batch, as the reference's batch assembly refuses it
    (batch.py:171-174, disjoint.py:139-140); the session stays usable."""
    from tt_atom import orb_calculator as OC
    cfg = dict(S.CFG_ORB_TINY)
    w = S.random_orb_weights(cfg, 32)
    path = tmp_path / "orb.npz"
    orb.save_orb_bundle(path, cfg, w)
    sess = OC.OrbSession(str(path), pair_repulsion=False)
    one = (np.zeros((1, 3)), np.array([8]))
    two = (np.array([[0.0, 0.0, 0.0], [20.0, 0.0, 0.0]]), np.array([6, 1]))
    for p, z in (one, two):
        with pytest.raises(ValueError, match="no edges"):
            sess.evaluate(p, z)
    mol = S.c5_systems(14, K=1, n_min=6, n_max=8, side=5.0)[0]
    with pytest.raises(ValueError, match="no edges"):
        sess.evaluate_batch([mol, two])
    assert np.isfinite(sess.evaluate(*mol)["energy"])


def test_orb_step_graph_replays_match_eager():
    """OrbEngine: graph replays equal the eager kernel sequence bit for bit, across eager work in
    between and after a change of positions."""
    from tt_atom import orb, synthetic
    cfg = dict(synthetic.CFG_ORB_TINY)
    w = synthetic.random_orb_weights(cfg, 7)
    systems = synthetic.c5_systems(K=4)
    bg = orb.assemble_orb(systems, cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
    model = orb.OrbModel(w, cfg)
    graph = orb.OrbGraph(model.device, senders=bg.senders, receivers=bg.receivers,
                         num_nodes=bg.pos.shape[0], atomic_numbers=bg.Z, cell_shift=bg.cell_shift,
                         natoms=bg.natoms)
    eng = orb.OrbEngine(model, graph)
    p0 = bg.pos.to(model.device)
    eng.step(p0, eager=True)
    raw0, F0 = eng.raw.clone(), eng.forces.clone()
    for _ in range(3):
        eng.step(p0)
        torch.cuda.synchronize()
        assert torch.equal(eng.raw, raw0) and torch.equal(eng.forces, F0)
        torch.randn(1 << 20, device=model.device).mul_(3.0).sum().item()
    p1 = p0 + 0.01 * torch.randn_like(p0)
    eng.step(p1, eager=True)
    raw1, F1 = eng.raw.clone(), eng.forces.clone()
    eng.step(p1)
    torch.cuda.synchronize()
    assert torch.equal(eng.raw, raw1) and torch.equal(eng.forces, F1)
    assert not torch.equal(raw1, raw0)


# ----------------------------------------------------------------------------- direct heads
def _direct_check(cfg, w, bg, raw, F, S_raw, oracle_dtype=torch.float64):
    """Denormalised energies within 1e-6 relative, forces within 1e-4 eV/A and the stress head
    within 1e-5 eV/A^3 of the oracle; every system's net force is zero."""
    ref_e, ref_f, ref_s = O.direct_forward(w, cfg, bg.pos.to(oracle_dtype), bg.Z, bg.senders,
                                           bg.receivers, bg.cell_shift.to(oracle_dtype),
                                           bg.batch, bg.natoms,
                                           compute_stress=S_raw is not None)
    off = 0
    for k, n in enumerate(bg.natoms):
        e = float(orb.denormalize_energy(raw[k], bg.Z[off:off + n], n, w))
        e_ref = float(orb.denormalize_energy(ref_e[k].double(), bg.Z[off:off + n], n, w))
        assert abs(e - e_ref) <= 1e-6 * max(1.0, abs(e_ref)), (k, e, e_ref)
        f = orb.denormalize_direct_forces(F[off:off + n].double(), w)
        f_ref = O.denormalize_direct_forces(ref_f[off:off + n],
                                            w["forces_head.normalizer.bn.running_mean"],
                                            w["forces_head.normalizer.bn.running_var"])
        assert (f - f_ref).abs().max() <= 1e-4, (k, (f - f_ref).abs().max())
        assert F[off:off + n].double().sum(0).abs().max() < 1e-5
        off += n
    if S_raw is not None:
        s = orb.denormalize_direct_stress(S_raw.double(), w)
        s_ref = O.denormalize_direct_stress(
            ref_s, w["stress_head.diag_normalizer.bn.running_mean"],
            w["stress_head.diag_normalizer.bn.running_var"],
            w["stress_head.offdiag_normalizer.bn.running_mean"],
            w["stress_head.offdiag_normalizer.bn.running_var"])
        assert (s - s_ref).abs().max() <= 1e-5, (s - s_ref).abs().max()


def _direct_engine(cfg, w, bg, use_graph=True):
    model = orb.OrbModel(w, cfg)
    graph = orb.OrbGraph(model.device, senders=bg.senders, receivers=bg.receivers,
                         num_nodes=bg.pos.shape[0], atomic_numbers=bg.Z, cell_shift=bg.cell_shift,
                         natoms=bg.natoms)
    return model, orb.OrbEngine(model, graph, use_graph=use_graph)


@pytest.mark.parametrize("arch", ["tiny", "c5"])
def test_orb_direct_heads_match_oracle(nat, arch):
    """Direct checkpoint: forward + ForceHead (per-system net-force removal) + StressHead on a
    batch, against the fp64 oracle; graph replays equal the eager step bit for bit."""
    if arch == "tiny":
        cfg = dict(S.CFG_ORB_TINY)
        systems = S.c5_systems(21, K=3, n_min=6, n_max=14, side=5.0)
    else:
        cfg = dict(S.CFG_ORB_C5)
        systems = S.c5_systems()[:8]
    w = S.random_orb_weights(cfg, 41, direct=True)
    bg = orb.assemble_orb(systems, cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
    model, eng = _direct_engine(cfg, w, bg)
    assert model.is_direct and model.has_stress_head
    p = bg.pos.to(model.device)
    raw, F, S_raw = eng.run(p, compute_stress=True, eager=True)
    F, S_raw = F.detach().cpu().clone(), S_raw.detach().cpu().clone()
    _direct_check(cfg, w, bg, raw, F, S_raw)
    for _ in range(3):                                   # capture, then replays
        raw2, F2, S2 = eng.run(p, compute_stress=True)
        torch.cuda.synchronize()
        assert torch.equal(raw2, raw) and torch.equal(F2.cpu(), F) and torch.equal(S2.cpu(), S_raw)
    raw3, F3, none = eng.run(p)                          # the variant without the stress head
    assert none is None and torch.equal(raw3, raw) and torch.equal(F3.cpu(), F)


def test_orb_direct_session(nat, tmp_path):
    """OrbSession on a direct bundle: periodic crystal with stress (ZBL sum-aggregated) against
    the oracle, evaluate_batch == evaluate per system, and a direct checkpoint without a stress
    head refuses an explicit stress request."""
    from tt_atom import orb_calculator as OC
    cfg = dict(S.CFG_ORB_TINY)
    w = S.random_orb_weights(cfg, 43, direct=True)
    path = tmp_path / "orb_direct.npz"
    orb.save_orb_bundle(path, cfg, w)
    radii = np.full(120, 0.6)
    sess = OC.OrbSession(str(path), pair_repulsion=True, covalent_radii=radii,
                         truncate_neighbors=True)
    assert sess.is_direct and sess.zbl_aggregation == "sum"
    pos, Z, cell = S.c4_system(seed=4, reps=2, a=3.61, noise=0.05, Z=29)
    r = sess.evaluate(pos, Z, cell=cell, pbc=[True] * 3, properties=("energy", "forces", "stress"))
    bg = orb.assemble_orb([(pos, Z, cell, [True] * 3)], cfg["cutoff"],
                          cfg["max_num_neighbors"], truncate=True)
    e_raw, f_raw, s_raw = O.direct_forward(w, cfg, bg.pos.double(), bg.Z, bg.senders,
                                           bg.receivers, bg.cell_shift.double(), bg.batch,
                                           bg.natoms, compute_stress=True)
    n = bg.natoms[0]
    e_z, f_z, s_z = OC.zbl_energy_forces_stress(bg.Z, bg.senders, bg.receivers, bg.pos,
                                                bg.cell_shift, radii, cell, aggregation="sum")
    e_ref = float(orb.denormalize_energy(e_raw[0], bg.Z, n, w)) + e_z
    f_ref = O.denormalize_direct_forces(f_raw, w["forces_head.normalizer.bn.running_mean"],
                                        w["forces_head.normalizer.bn.running_var"]).numpy() + f_z
    s_ref = O.denormalize_direct_stress(
        s_raw[0], w["stress_head.diag_normalizer.bn.running_mean"],
        w["stress_head.diag_normalizer.bn.running_var"],
        w["stress_head.offdiag_normalizer.bn.running_mean"],
        w["stress_head.offdiag_normalizer.bn.running_var"]).numpy() + s_z
    assert abs(r["energy"] - e_ref) <= 1e-6 * max(1.0, abs(e_ref))
    assert np.abs(r["forces"] - f_ref).max() <= 1e-4
    assert np.abs(r["stress"] - s_ref).max() <= 1e-5
    systems = S.c5_systems(17, K=3, n_min=6, n_max=12, side=5.0)
    res = [sess.evaluate(p, z) for p, z in systems]
    batch = sess.evaluate_batch(systems)
    for k, rk in enumerate(res):
        assert abs(batch["energy"][k] - rk["energy"]) <= 1e-6 * max(1.0, abs(rk["energy"]))
        assert np.abs(batch["forces"][k] - rk["forces"]).max() <= 2e-5
    w_ns = {k: v for k, v in w.items() if not k.startswith("stress_head.")}
    path2 = tmp_path / "orb_direct_nostress.npz"
    orb.save_orb_bundle(path2, cfg, w_ns)
    sess2 = OC.OrbSession(str(path2), pair_repulsion=False, truncate_neighbors=True)
    with pytest.raises(ValueError, match="stress_head"):
        sess2.evaluate(pos, Z, cell=cell, pbc=[True] * 3, properties=("energy", "stress"))
    r2 = sess2.evaluate(pos, Z, cell=cell, pbc=[True] * 3)     # implicit stress: left out
    assert "stress" not in r2


def test_segment_center(nat):
    """Per-system centring kernel: ragged systems, a one-row system, C = 3 and C = 16."""
    g = torch.Generator().manual_seed(3)
    sizes = [1, 5, 64, 65, 130, 7]
    ptr = torch.tensor([0] + list(np.cumsum(sizes)), dtype=torch.int32)
    N = int(ptr[-1])
    for C in (3, 16):
        x = torch.randn(N, C, generator=g)
        out = torch.empty(N, C, device="cuda")
        nat.segment_center(x.cuda(), ptr.cuda(), out)
        torch.cuda.synchronize()
        ref = torch.cat([xs - xs.double().mean(0).float() for xs in torch.split(x, sizes)])
        assert (out.cpu() - ref).abs().max() < 1e-6
        xi = x.cuda()
        nat.segment_center(xi, ptr.cuda(), xi)                  # in place
        assert torch.equal(xi, out)


def test_orb_c5_full_batch_translation(nat):
    """The full C5 batch: translating every molecule by its own vector leaves every energy and
    force unchanged (fp32 resolution) and each molecule's forces sum to zero."""
    cfg = dict(S.CFG_ORB_C5)
    w = S.random_orb_weights(cfg, S.SEEDS["C5"] + S.WEIGHT_SEED_OFFSET)
    bg = orb.assemble_orb(S.c5_systems(), cfg["cutoff"], cfg["max_num_neighbors"],
                              truncate=True)
    model = orb.OrbModel(w, cfg)
    graph = orb.OrbGraph(model.device, senders=bg.senders, receivers=bg.receivers,
                         num_nodes=bg.pos.shape[0], atomic_numbers=bg.Z, cell_shift=bg.cell_shift,
                         natoms=bg.natoms)
    eng = orb.OrbEngine(model, graph, use_graph=False)
    raw0, F0, _ = eng.run(bg.pos.to(model.device))
    F0 = F0.cpu().double()
    g = torch.Generator().manual_seed(8)
    shift = (torch.rand(bg.K, 3, generator=g, dtype=torch.float64) - 0.5) * 20.0
    batch = bg.batch.long()
    raw1, F1, _ = eng.run((bg.pos.double() + shift[batch]).float().to(model.device))
    F1 = F1.cpu().double()
    assert (raw1 - raw0).abs().max() <= 2e-6 * max(1.0, float(raw0.abs().max()))
    assert (F1 - F0).abs().max() <= 1e-4 * max(1.0, float(F0.abs().max()))
    sums = torch.zeros(bg.K, 3, dtype=torch.float64).index_add_(0, batch, F0)
    assert sums.abs().max() <= 1e-4 * max(1.0, float(F0.abs().max()))
