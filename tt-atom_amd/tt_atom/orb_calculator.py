"""``OrbCalculator`` -- ASE calculator over the MI355X Orb-v3 step (reference orb_calculator.py:25-327).

``OrbSession`` holds one Orb-v3 checkpoint on one GPU and evaluates arrays (one system,
``evaluate``) or a disjoint-union batch (``evaluate_batch``) as the reference's ``calculate`` /
``evaluate_batch`` do: neighbour list (senders = tgt, receivers = src), node embedding and
optional charge/spin conditioning, then
  * conservative checkpoints: one device forward + backward, the energy normaliser
    ``E = (raw sigma + mu) n + sum ref[Z]``, ``F = raw_F sigma n`` and
    ``stress = virial sigma n / V`` (orb_model.py:459-600), ZBL mean-aggregated;
  * direct checkpoints (a ``forces_head`` in the weights): the device forward and the force /
    stress heads, ``F = raw_F sigma_F + mu_F`` and the two-normaliser Voigt stress
    (orb_model.py:438-457), ZBL sum-aggregated (orb_calculator.py:124-185);
plus the ZBL pair repulsion (orb_model.py:491-585) when enabled.  The step engine is kept while
the graph is unchanged.
``OrbCalculator`` adapts it to ASE; ``ase`` is optional and only that class (and the default ZBL
radius table) needs it.
"""
from __future__ import annotations

import numpy as np
import torch

from . import orb
from .calculator import full_3x3_to_voigt_6

try:  # ASE is optional
    from ase.calculators.calculator import Calculator as _AseCalculator
    from ase.calculators.calculator import all_changes as _all_changes
    HAVE_ASE = True
except ImportError:  # pragma: no cover - exercised where ase is absent
    _AseCalculator = object
    _all_changes = ()
    HAVE_ASE = False


# ----------------------------------------------------------------------------- ZBL (host)
# Universal ZBL screening function and the Orb pair-repulsion envelope (orb_model.py:491-538);
# the constants are the physical ones and are kept as published.
_ZBL_C = (0.1818, 0.5099, 0.2802, 0.02817)
_ZBL_D = (3.2, 0.9423, 0.4028, 0.2016)
_ZBL_A_EXP, _ZBL_A_PRE, _BOHR, _COULOMB = 0.300, 0.4543, 0.529, 14.3996


def _zbl_pairs(Z, senders, receivers, vectors, covalent_radii, p=6):
    """Per-edge ZBL pair energies (fp64, differentiable in ``vectors``).  Orb's atomic-number
    embedding is indexed by the stored number and its ZBL basis adds one to it
    (orb_model.py:507-510); that convention is kept.  The envelope is zero from the sum of the
    covalent radii on, so only the pairs inside it are evaluated (the others are exact zeros)."""
    Zu = Z[senders].double() + 1
    Zv = Z[receivers].double() + 1
    rad = torch.as_tensor(covalent_radii, dtype=torch.float64)
    r_max = rad[Zu.long()] + rad[Zv.long()]
    vec = vectors.double()
    with torch.no_grad():
        near = torch.nonzero(torch.linalg.norm(vec, dim=1) < r_max).reshape(-1)
    out = torch.zeros(vec.shape[0], dtype=torch.float64)
    if near.numel() == 0:
        return out + 0.0 * vec.sum()                   # keeps the graph for autograd callers
    Zu, Zv, r_max = Zu[near], Zv[near], r_max[near]
    a = _ZBL_A_PRE * _BOHR / (Zu ** _ZBL_A_EXP + Zv ** _ZBL_A_EXP)
    x = torch.linalg.norm(vec[near], dim=1)
    phi = sum(c * torch.exp(-d * x / a) for c, d in zip(_ZBL_C, _ZBL_D))
    q = x / r_max
    env = (1.0 - (p + 1) * (p + 2) / 2.0 * q ** p + p * (p + 2) * q ** (p + 1)
           - p * (p + 1) / 2.0 * q ** (p + 2))
    return out.index_put((near,), 0.5 * _COULOMB * Zu * Zv / x * phi * env)


def zbl_energy(Z, senders, receivers, vectors, covalent_radii, p=6, aggregation="mean"):
    """Pair repulsion of one system: per-edge energies summed onto senders, then the mean or the
    sum over nodes (orb_model.py:491-538)."""
    v = _zbl_pairs(Z, senders, receivers, vectors, covalent_radii, p)
    per_node = torch.zeros(Z.shape[0], dtype=torch.float64).index_add_(0, senders, v)
    if aggregation == "mean":
        return per_node.mean()
    if aggregation == "sum":
        return per_node.sum()
    raise ValueError(f"aggregation must be 'mean' or 'sum', got {aggregation!r}")


def zbl_energy_forces_stress(Z, senders, receivers, pos, shift, covalent_radii, cell=None,
                             aggregation="mean"):
    """(energy, forces [N,3], Voigt stress or None) of the pair repulsion by host autograd
    (orb_model.py:541-585)."""
    pos = torch.as_tensor(pos, dtype=torch.float64).detach().clone().requires_grad_(True)
    strain = torch.zeros(3, 3, dtype=torch.float64, requires_grad=cell is not None)
    v = pos[receivers] - pos[senders]
    if shift is not None:
        v = v + torch.as_tensor(shift, dtype=torch.float64)
    if cell is not None:
        v = v @ (torch.eye(3, dtype=torch.float64) + 0.5 * (strain + strain.T))
    e = zbl_energy(Z, senders, receivers, v, covalent_radii, aggregation=aggregation)
    ins = [pos] if cell is None else [pos, strain]
    g = torch.autograd.grad(e, ins)
    stress = None
    if cell is not None:
        vol = abs(float(np.linalg.det(np.asarray(cell, dtype=np.float64).reshape(3, 3))))
        stress = full_3x3_to_voigt_6(g[1].numpy() / vol)
    return float(e.detach()), (-g[0]).numpy(), stress


def zbl_batch(Z, senders, receivers, pos, shift, batch, natoms, covalent_radii,
              aggregation="mean", p=6):
    """Pair repulsion of every system of a disjoint union: (energies [K], forces [N, 3]), fp64.
    The union's edges never join two systems, so each atom's force comes from its own system (as
    orb_calculator.py:296-327 computes the union's ZBL once).  The force is the closed-form
    derivative of the pair energy of ``_zbl_pairs``, E(x) = k Zu Zv / (2x) * phi(x) * env(x / r)
    with phi = sum_i c_i exp(-d_i x / a) and env the degree-p polynomial envelope, taken only
    over the pairs inside the envelope -- the host autograd of zbl_energy_forces_stress, without
    building a graph per call (same values to fp64 rounding)."""
    if aggregation not in ("mean", "sum"):
        raise ValueError(f"aggregation must be 'mean' or 'sum', got {aggregation!r}")
    Zn = np.asarray(Z, dtype=np.int64)
    s_i, r_i = np.asarray(senders, dtype=np.int64), np.asarray(receivers, dtype=np.int64)
    P = np.asarray(pos, dtype=np.float64)
    v = P[r_i] - P[s_i]
    if shift is not None:
        v = v + np.asarray(shift, dtype=np.float64)
    rad = np.asarray(covalent_radii, dtype=np.float64)
    Zu, Zv = Zn[s_i] + 1, Zn[r_i] + 1
    r_max = rad[Zu] + rad[Zv]
    x_all = np.sqrt((v * v).sum(1))
    near = np.nonzero(x_all < r_max)[0]
    K = len(natoms)
    b = np.asarray(batch, dtype=np.int64)
    w_sys = 1.0 / np.asarray(natoms, dtype=np.float64) if aggregation == "mean" else np.ones(K)
    e_sys = np.zeros(K)
    F = np.zeros_like(P)
    if near.size:
        zu, zv, rm, x = Zu[near].astype(np.float64), Zv[near].astype(np.float64), r_max[near], \
            x_all[near]
        a = _ZBL_A_PRE * _BOHR / (zu ** _ZBL_A_EXP + zv ** _ZBL_A_EXP)
        ex = [np.exp(-d * x / a) for d in _ZBL_D]
        phi = sum(c * e for c, e in zip(_ZBL_C, ex))
        dphi = sum(-c * d / a * e for c, d, e in zip(_ZBL_C, _ZBL_D, ex))
        q = x / rm
        env = (1.0 - (p + 1) * (p + 2) / 2.0 * q ** p + p * (p + 2) * q ** (p + 1)
               - p * (p + 1) / 2.0 * q ** (p + 2))
        denv = (-(p + 1) * (p + 2) / 2.0 * p * q ** (p - 1) + p * (p + 2) * (p + 1) * q ** p
                - p * (p + 1) / 2.0 * (p + 2) * q ** (p + 1)) / rm
        pre = 0.5 * _COULOMB * zu * zv
        e = pre / x * phi * env
        de = pre * (-phi * env / (x * x) + (dphi * env + phi * denv) / x)
        sys_e = b[s_i[near]]
        e_sys = np.bincount(sys_e, weights=e, minlength=K) * w_sys
        g = (w_sys[sys_e] * de / x)[:, None] * v[near]        # dE_sys / dv per pair
        n = P.shape[0]
        for c in range(3):
            F[:, c] = (np.bincount(s_i[near], weights=g[:, c], minlength=n)
                       - np.bincount(r_i[near], weights=g[:, c], minlength=n))
    return e_sys, F


def _default_radii():
    try:
        from ase.data import covalent_radii
    except ImportError as exc:  # pragma: no cover
        raise RuntimeError("the ZBL pair repulsion needs a covalent-radius table: install ase, "
                           "pass covalent_radii=..., or pair_repulsion=False") from exc
    return np.asarray(covalent_radii, dtype=np.float64)


# ----------------------------------------------------------------------------- session
class OrbSession:
    """One Orb-v3 checkpoint, conservative or direct, on one GPU (orb_calculator.py:26-73)."""

    def __init__(self, weights, device=None, device_id=0, precision="f32", pair_repulsion=True,
                 covalent_radii=None, neighbor_list="device", truncate_neighbors=False):
        """``truncate_neighbors=False`` refuses a system with an atom over the checkpoint's
        ``max_num_neighbors`` as the reference does (orb_calculator.py:110-125); True keeps each
        atom's nearest ones instead (``orb.assemble_orb(truncate=True)``)."""
        if isinstance(weights, str):
            weights = orb.OrbWeights.load(weights)
        self.cfg = dict(weights.config)
        self._w = weights.weights
        dev = torch.device(device) if device is not None else torch.device(f"cuda:{device_id}")
        self.model = orb.OrbModel(self._w, self.cfg, dev, precision=precision)
        self.r_max = float(self.cfg["cutoff"])
        self.max_num_neighbors = int(self.cfg["max_num_neighbors"])
        self.task = self.task_name = self.cfg.get("task", "omat")
        self.pair_repulsion = pair_repulsion
        self._radii = covalent_radii
        self.neighbor_list = neighbor_list
        self.truncate_neighbors = bool(truncate_neighbors)
        self.is_direct = self.model.is_direct
        self.zbl_aggregation = "sum" if self.is_direct else "mean"
        self._engine, self._key = None, None

    def _radii_table(self):
        if self._radii is None:
            self._radii = _default_radii()
        return self._radii

    def _run(self, bg, compute_stress):
        N = int(bg.pos.shape[0])
        # the conditioning enters through (charge, spin) per system, so those values (not the
        # embedding tensors) are part of the engine key
        cond_key = ((tuple(bg.charges), tuple(bg.spins)) if self.model.has_cond else None)
        key = (bg.senders.numel(), tuple(bg.natoms), cond_key)
        same = (self._engine is not None and self._key[0] == key
                and torch.equal(self._key[1], bg.senders) and torch.equal(self._key[2], bg.receivers)
                and torch.equal(self._key[3], bg.cell_shift) and torch.equal(self._key[4], bg.Z))
        if not same:
            graph = orb.OrbGraph(self.model.device, senders=bg.senders, receivers=bg.receivers,
                                 num_nodes=N, atomic_numbers=bg.Z, cell_shift=bg.cell_shift,
                                 natoms=bg.natoms)
            cond = self._cond(bg) if self.model.has_cond else None
            self._engine = orb.OrbEngine(self.model, graph, cond)
            self._key = (key, bg.senders.clone(), bg.receivers.clone(), bg.cell_shift.clone(),
                         bg.Z.clone())
        p = torch.as_tensor(bg.pos, dtype=torch.float32).to(self.model.device)
        raw, F, vir = self._engine.run(p, compute_stress)
        return raw, F.detach().cpu().double(), (None if vir is None else vir.detach().cpu().double())

    def _cond(self, bg):
        return self.model.charge_spin_embedding_batch(bg.charges, bg.spins, bg.natoms)

    def evaluate(self, positions, numbers, cell=None, pbc=None, charge=0.0, spin=0.0,
                 properties=("energy", "forces")):
        """One system (orb_calculator.py:89-215): energy, free_energy, forces[, stress]."""
        pbc_a = np.zeros(3, bool) if pbc is None else np.asarray(pbc, dtype=bool).reshape(-1)
        if pbc_a.size == 1:
            pbc_a = np.repeat(pbc_a, 3)
        cell_a = np.asarray(cell, dtype=np.float64).reshape(3, 3) \
            if (cell is not None and pbc_a.any()) else None
        system = dict(positions=positions, numbers=numbers, cell=cell_a,
                      pbc=pbc_a if cell_a is not None else None, charge=charge, spin=spin)
        bg = orb.assemble_orb([system], self.r_max, self.max_num_neighbors, self.neighbor_list,
                              truncate=self.truncate_neighbors)
        explicit_stress = "stress" in properties
        want_stress = cell_a is not None and (explicit_stress or bool(pbc_a.all()))
        if self.is_direct and not self.model.has_stress_head:
            if explicit_stress:
                raise ValueError("stress requested but this direct checkpoint carries no "
                                 "stress_head weights")
            want_stress = False          # a periodic system that did not ask for stress
        raw, F_raw, s_raw = self._run(bg, want_stress)
        n = bg.natoms[0]
        E = float(orb.denormalize_energy(raw[0], bg.Z, n, self._w))
        stress = None
        if self.is_direct:
            F = orb.denormalize_direct_forces(F_raw, self._w).numpy()
            if want_stress:
                stress = orb.denormalize_direct_stress(s_raw[0], self._w).numpy()
        else:
            F = orb.denormalize_forces(F_raw, n, self._w).numpy()
            if want_stress:
                stress = orb.denormalize_stress(s_raw, n, torch.as_tensor(cell_a),
                                                self._w).numpy()
        if self.pair_repulsion:
            e_z, f_z, s_z = zbl_energy_forces_stress(bg.Z, bg.senders, bg.receivers, bg.pos,
                                                     bg.cell_shift, self._radii_table(),
                                                     cell_a if want_stress else None,
                                                     aggregation=self.zbl_aggregation)
            E, F = E + e_z, F + f_z
            if stress is not None:
                stress = stress + s_z
        res = {"energy": E, "free_energy": E, "forces": F}
        if stress is not None:
            res["stress"] = stress
        return res

    def evaluate_batch(self, systems, properties=("energy", "forces")):
        """Disjoint-union batch in one device step (orb_calculator.py:217-327):
        ``dict(energy=ndarray[K], forces=list[ndarray[N_k, 3]] or None)``."""
        want_forces = "forces" in properties
        bg = orb.assemble_orb(systems, self.r_max, self.max_num_neighbors, self.neighbor_list,
                              truncate=self.truncate_neighbors)
        raw, F_raw, _ = self._run(bg, False)
        batch = bg.batch.long()
        n_of = torch.as_tensor(bg.natoms, dtype=torch.float64)
        E = orb.denormalize_energy_batch(raw, bg.Z, batch, bg.natoms, self._w).numpy()
        if self.is_direct:
            F = orb.denormalize_direct_forces(F_raw, self._w).numpy()
        else:
            F = orb.denormalize_forces(F_raw, n_of[batch][:, None], self._w).numpy()
        if self.pair_repulsion:
            e_z, f_z = zbl_batch(bg.Z, bg.senders, bg.receivers, bg.pos, bg.cell_shift, batch,
                                 bg.natoms, self._radii_table(), self.zbl_aggregation)
            E, F = E + e_z, F + f_z
        forces = np.split(F, np.cumsum(bg.natoms)[:-1]) if want_forces else None
        return dict(energy=np.asarray(E, dtype=np.float64), forces=forces)


class OrbCalculator(_AseCalculator):
    """ASE calculator (orb_calculator.py:25-215)."""

    implemented_properties = ["energy", "free_energy", "forces", "stress"]

    def __init__(self, weights, device=None, device_id=0, fast=False, bucketing=False,
                 precision="f32", **kwargs):
        if not HAVE_ASE:
            raise ImportError("OrbCalculator needs ase; tt_atom.orb_calculator.OrbSession "
                              "evaluates arrays without it")
        # fast=True (the reference's bf8 weights, orb_calculator.py:26-73) selects bf16 GEMM
        # operands, as the Orb modules and the UMA calculator do
        if fast:
            precision = "bf16"
        super().__init__(**kwargs)
        # bucketing pads edge counts so ttnn reuses compiled shapes; the HIP kernels are shape-
        # generic, so it changes nothing here
        self.session = OrbSession(weights, device=device, device_id=device_id,
                                  precision=precision)
        self.task = self.task_name = self.session.task

    @classmethod
    def from_checkpoint(cls, checkpoint="orb-v3-conservative-inf-omat", refenv=None,
                        cache_dir=None, device=None, device_id=0, fast=False, **kwargs):
        """Calculator from the per-checkpoint weight cache (orb_calculator.py:75-86)."""
        from . import orb_weight_cache
        path = orb_weight_cache.get_or_build(checkpoint, refenv=refenv, cache_dir=cache_dir)
        return cls(str(path), device=device, device_id=device_id, fast=fast, **kwargs)

    def calculate(self, atoms=None, properties=("energy", "forces"),
                  system_changes=_all_changes):
        super().calculate(atoms, properties, system_changes)
        pbc = np.asarray(atoms.get_pbc())
        res = self.session.evaluate(atoms.get_positions(), atoms.get_atomic_numbers(),
                                    cell=np.asarray(atoms.get_cell()) if pbc.any() else None,
                                    pbc=pbc, charge=float(atoms.info.get("charge", 0.0)),
                                    spin=float(atoms.info.get("spin", 0.0)),
                                    properties=properties)
        self.results.update(res)

    def evaluate_batch(self, systems, properties=("energy", "forces")):
        return self.session.evaluate_batch(systems, properties)
