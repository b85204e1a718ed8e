"""The UMA array-level calculator core (``calculator.Session``, the engine of TTAtomCalculator)
on the MI355X: a saved bundle round trip, one system against the oracle with the energy
normaliser, and ``evaluate_batch`` (one disjoint-union step) against per-system ``evaluate``."""
import numpy as np
import pytest
import torch

from oracle import forces as OF
from tt_atom import calculator, geometry, synthetic, weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def session(tmp_path_factory):
    cfg = dict(synthetic.CFG_UMA_S, sphere_channels=32, hidden_channels=32, edge_channels=32,
               num_distance_basis=32, num_layers=2, task="omol")
    w, host = synthetic.random_uma_bundle(cfg, 77)
    p = tmp_path_factory.mktemp("b") / "b.npz"
    weights.save_bundle(p, cfg, w, host, scale={"rmsd": 1.7, "mean": -0.3})
    return cfg, w, host, calculator.Session(str(p))


def _molecules():
    return [synthetic.c3_system(seed=40 + k, n=n, radius=17.0 * (n / 2048) ** (1 / 3))
            for k, n in enumerate((24, 31, 47, 18))]


def test_session_single_system_matches_oracle(session):
    cfg, w, host, sess = session
    pos, Z = _molecules()[2]
    res = sess.evaluate(pos, Z, charge=0.0, spin=1.0)
    pos_t, Z_t = torch.from_numpy(pos).float(), torch.from_numpy(Z).long()
    ei, _ = geometry.radius_graph(pos_t, cfg["cutoff"])
    se = geometry.csd_embedding(w, torch.tensor([0.0]), torch.tensor([1.0]),
                                dataset="omol").expand(len(Z), -1).contiguous()
    E0, F0 = OF.energy_and_forces(OF.Model(w, cfg, host), pos_t, Z_t, ei, se)
    assert abs(res["energy"] - (1.7 * E0 - 0.3)) <= 1e-6 * max(1.0, abs(1.7 * E0))
    assert np.abs(res["forces"] - 1.7 * F0.double().numpy()).max() <= 1e-4


def test_session_evaluate_batch_equals_per_system(session):
    cfg, w, host, sess = session
    mols = _molecules()
    pos_p, Z_p, cell = synthetic.c4_system(seed=4, reps=2)
    systems = [dict(positions=p, numbers=z) for p, z in mols[:2]]
    systems.append(dict(positions=pos_p, numbers=Z_p, cell=cell, pbc=[True] * 3))
    systems += [dict(positions=p, numbers=z, charge=1.0, spin=2.0) for p, z in mols[2:]]
    out = sess.evaluate_batch(systems)
    assert out["energy"].shape == (len(systems),) and len(out["forces"]) == len(systems)
    for k, s in enumerate(systems):
        one = sess.evaluate(s["positions"], s["numbers"], cell=s.get("cell"), pbc=s.get("pbc"),
                            charge=s.get("charge", 0.0), spin=s.get("spin", 0.0))
        assert abs(out["energy"][k] - one["energy"]) <= 1e-6 * max(1.0, abs(one["energy"])), k
        assert np.abs(out["forces"][k] - one["forces"]).max() <= 1e-5, k
    # a second call on the same batch replays the kept engine: identical results
    again = sess.evaluate_batch(systems)
    assert np.array_equal(again["energy"], out["energy"])
    assert all(np.array_equal(a, b) for a, b in zip(again["forces"], out["forces"]))


def test_session_batch_of_identical_copies(session):
    """K copies of one molecule give K identical energies and force blocks (reference
    test_batch.py::test_batched_identical_copies)."""
    cfg, w, host, sess = session
    pos, Z = _molecules()[1]
    out = sess.evaluate_batch([dict(positions=pos, numbers=Z)] * 5)
    assert np.all(out["energy"] == out["energy"][0])
    assert all(np.array_equal(f, out["forces"][0]) for f in out["forces"])


def test_session_new_engine_on_cell_change(session):
    """Same atoms, same edge set, a strained cell: the image shifts change, so the kept engine
    must not be reused (reference test_trace.py::test_traced_recaptures_on_cell_shift_change);
    the result equals a fresh session's."""
    cfg, w, host, sess = session
    pos, Z, cell = synthetic.c4_system(seed=4, reps=2)
    r1 = sess.evaluate(pos, Z, cell=cell, pbc=[True] * 3)
    cell2 = cell * 1.01
    r2 = sess.evaluate(pos, Z, cell=cell2, pbc=[True] * 3)
    assert r1["energy"] != r2["energy"]
    fresh = calculator.Session(sess.bundle).evaluate(pos, Z, cell=cell2, pbc=[True] * 3)
    assert r2["energy"] == fresh["energy"] and np.array_equal(r2["forces"], fresh["forces"])
    assert np.array_equal(r2["stress"], fresh["stress"])


def test_session_systems_without_edges(session):
    """A system with no edge inside the cutoff (one atom; two atoms 20 A apart) is refused with
    ValueError, alone and inside a batch, as the reference's calculator and disjoint assembly
    refuse it (calculator.py:132-133, disjoint.py:139-140)."""
    cfg, w, host, sess = session
    one = (np.zeros((1, 3)), np.array([8]))
    two = (np.array([[0.0, 0.0, 0.0], [20.0, 0.0, 0.0]]), np.array([6, 1]))
    for pos, Z in (one, two):
        with pytest.raises(ValueError, match="no edges"):
            sess.evaluate(pos, Z, charge=0.0, spin=1.0)
    mol = _molecules()[0]
    with pytest.raises(ValueError, match="no edges"):
        sess.evaluate_batch([dict(positions=mol[0], numbers=mol[1]),
                             dict(positions=two[0], numbers=two[1])])
    # the session stays usable
    assert np.isfinite(sess.evaluate(mol[0], mol[1])["energy"])
