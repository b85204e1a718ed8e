"""``TTAtomCalculator`` -- ASE calculator over the MI355X step (reference calculator.py:22-166,
ase_base.py:18-54).

``Session`` holds one bundle on one GPU and evaluates arrays (positions, numbers, cell, pbc,
charge, spin) exactly as the reference's ``calculate`` does: neighbour list, system embedding,
energy + forces (+ stress when a cell is periodic or stress is requested), then the per-task
energy normalizer ``E = rmsd * E_raw + mean + sum(refs[Z])``, ``F = rmsd * F_raw`` and
``stress = rmsd * virial / V`` in ASE's Voigt order.  The step engine is kept while the neighbour
list and cell shifts are unchanged (the reference's trace re-capture rule, calculator.py:256-277).
``TTAtomCalculator`` adapts it to ASE; ``ase`` is optional and only that class needs it.
"""
from __future__ import annotations

import numpy as np
import torch

from . import geometry, model, trace
from .weights import WeightBundle

try:  # ASE is optional: only the ASE adapter class needs it
    from ase.calculators.calculator import Calculator as _AseCalculator
    from ase.calculators.calculator import all_changes as _all_changes
    HAVE_ASE = True
except ImportError:  # pragma: no cover - exercised where ase is absent
    _AseCalculator = object
    _all_changes = ()
    HAVE_ASE = False


def check_batch_matches_bundle(bundle, systems):
    """Refuse a batch that a merged bundle was not built for (calculator.py:191-218): a merged
    uma-s-1 bundle bakes the MoLE expert routing for one reduced composition and one
    (charge, spin), so every system must share those of the bundle's merge inputs (``ref@*``).
    Bundles without merge inputs (random-init weights) accept any batch."""
    ref = bundle.reference if hasattr(bundle, "reference") else None
    if ref is None:
        return
    from .bundle_cache import reduced_composition
    from .orb import _fields
    want_comp = reduced_composition(ref["atomic_numbers"])
    want_cs = (float(ref["charge"]), float(ref["spin"]))
    for k, system in enumerate(systems):
        _, Z, _, _, charge, spin = _fields(system)
        if reduced_composition(np.asarray(Z)) != want_comp:
            raise ValueError(
                f"batched system {k} has a different reduced composition than this bundle: a "
                "merged bundle bakes the MoLE routing for one reduced composition, so every "
                "system of a batch must share it; evaluate other compositions with their own "
                "bundle")
        if (float(charge), float(spin)) != want_cs:
            raise ValueError(
                f"batched system {k} has (charge, spin)=({float(charge)}, {float(spin)}) but "
                f"this bundle was merged for {want_cs}; every system of a batch must share it")


def full_3x3_to_voigt_6(s):
    """ASE's Voigt order (xx, yy, zz, yz, xz, xy) with symmetrised off-diagonals."""
    s = np.asarray(s, dtype=np.float64).reshape(3, 3)
    return np.array([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]),
                     0.5 * (s[0, 2] + s[2, 0]), 0.5 * (s[0, 1] + s[1, 0])])


class Session:
    """One bundle on one GPU; evaluates systems given as arrays."""

    def __init__(self, bundle, task_name=None, device=None, gamma=0.0, max_neighbors=None,
                 neighbor_list="device", precision="f32", fast=False):
        if neighbor_list not in ("host", "device"):
            raise ValueError("neighbor_list must be 'host' or 'device'")
        self.neighbor_list = neighbor_list
        if isinstance(bundle, str):
            bundle = WeightBundle.load(bundle)
        self.bundle = bundle
        self.cfg = dict(bundle.config)
        if task_name is not None and task_name != bundle.task:
            raise ValueError(f"task_name={task_name!r} does not match this bundle's task "
                             f"{bundle.task!r}")
        self.task = bundle.task
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        w = bundle.weights
        self._w = w
        self.C = self.cfg["sphere_channels"]
        self.backbone = model.Backbone(w, self.device, self.cfg, bundle.to_grid_mat,
                                       bundle.from_grid_mat, precision=precision, fast=fast)
        self.geo = geometry.HostGeometry(w, self.cfg, bundle.to_m, bundle.gauss_offset,
                                         bundle.gauss_coeff, gamma=gamma,
                                         coefficient_index=bundle.coefficient_index,
                                         device=self.device)
        self.max_neighbors = max_neighbors if max_neighbors is not None else \
            self.cfg.get("max_neighbors_cap")
        self.scale_rmsd, self.scale_mean = bundle.scale_rmsd, bundle.scale_mean
        self.elem_refs = bundle.elem_refs
        self._engine = None
        self._key = None

    def _engine_for(self, Z, edge_index, shift, sys_emb):
        key = (tuple(Z.tolist()), edge_index.shape[1], shift is not None)
        same = (self._engine is not None and self._key[0] == key
                and torch.equal(self._key[1], edge_index)
                and ((shift is None and self._key[2] is None) or
                     (shift is not None and self._key[2] is not None
                      and torch.equal(self._key[2], shift)))
                and torch.equal(self._key[3], sys_emb))
        if not same:
            self._engine = trace.TracedEngine(self.backbone, self.geo, Z, edge_index, sys_emb,
                                              edge_cell_shift=shift)
            self._key = (key, edge_index.clone(), None if shift is None else shift.clone(),
                         sys_emb.clone())
        return self._engine

    def evaluate(self, positions, numbers, cell=None, pbc=None, charge=0.0, spin=0.0,
                 properties=("energy", "forces")):
        pos = torch.as_tensor(np.asarray(positions), dtype=torch.float32)
        Z = torch.as_tensor(np.asarray(numbers), dtype=torch.long)
        pbc = np.zeros(3, bool) if pbc is None else np.asarray(pbc, dtype=bool).reshape(-1)
        if pbc.size == 1:
            pbc = np.repeat(pbc, 3)
        cell_t = torch.as_tensor(np.asarray(cell), dtype=torch.float32).reshape(3, 3) \
            if (cell is not None and pbc.any()) else None
        nl = geometry.radius_graph_device if self.neighbor_list == "device" else \
            geometry.radius_graph
        ei, shift = nl(pos, self.cfg["cutoff"], cell=cell_t,
                       pbc=pbc if cell_t is not None else None, max_neighbors=self.max_neighbors)
        if ei.shape[1] == 0:
            raise ValueError("no edges within cutoff -- system too sparse for this model")
        sys_emb = geometry.csd_embedding(self._w, torch.tensor([float(charge)]),
                                         torch.tensor([float(spin)]), self.C,
                                         dataset=self.task)[torch.zeros(len(Z), dtype=torch.long)]
        want_stress = cell_t is not None and ("stress" in properties or bool(pbc.all()))
        eng = self._engine_for(Z, ei, shift if cell_t is not None else None, sys_emb)
        out = eng(pos, compute_stress=want_stress)
        E = self.scale_rmsd * out[0] + self.scale_mean
        if self.elem_refs is not None:
            E += float(self.elem_refs[Z].sum())
        F = (self.scale_rmsd * out[1]).detach().cpu().numpy().astype(np.float64)
        res = {"energy": float(E), "free_energy": float(E),
               "energies": np.full(len(Z), float(E) / len(Z)), "forces": F}
        if want_stress:
            vol = abs(float(np.linalg.det(cell_t.double().numpy())))
            res["stress"] = full_3x3_to_voigt_6(
                self.scale_rmsd * out[2].detach().cpu().double().numpy() / vol)
        return res


    def evaluate_batch(self, systems, properties=("energy", "forces")):
        """K systems in one device step (calculator.py:168-236): ``dict(energy=ndarray[K],
        forces=list[ndarray[N_k, 3]] or None)`` with the per-system energy normaliser applied.
        The step engine (and its HIP graph) is kept while the batch topology is unchanged."""
        from . import disjoint
        check_batch_matches_bundle(self.bundle, systems)
        bg = disjoint.assemble(systems, self.cfg["cutoff"], self._w, self.C, task=self.task,
                               max_neighbors=self.max_neighbors, neighbor_list=self.neighbor_list)
        periodic = bool(bg.cell_shift.abs().sum() > 0)
        eng = self._engine_for(bg.Z, bg.edge_index, bg.cell_shift if periodic else None,
                               bg.sys_emb)
        eng.run(bg.pos)
        E_raw = eng.segment_energies(bg.natoms).cpu().double()
        want_forces = "forces" in properties
        F_all = eng.forces.detach().cpu().double() if want_forces else None
        energies, forces, off = [], [], 0
        for k, n in enumerate(bg.natoms):
            Ek = self.scale_rmsd * float(E_raw[k]) + self.scale_mean
            if self.elem_refs is not None:
                Ek += float(self.elem_refs[bg.Z[off:off + n]].sum())
            energies.append(Ek)
            if want_forces:
                forces.append((self.scale_rmsd * F_all[off:off + n]).numpy())
            off += n
        return dict(energy=np.array(energies), forces=forces if want_forces else None)


class TTAtomCalculator(_AseCalculator):
    """ASE calculator (reference calculator.py:22-166)."""

    implemented_properties = ["energy", "energies", "free_energy", "forces", "stress"]

    def __init__(self, bundle, task_name=None, device=None, device_id=0, gamma=0.0, fast=False,
                 trace=False, max_neighbors=None, **kwargs):
        if not HAVE_ASE:
            raise ImportError("TTAtomCalculator needs ase; tt_atom.calculator.Session evaluates "
                              "arrays without it")
        super().__init__(**kwargs)
        dev = device if device is not None else torch.device(f"cuda:{device_id}")
        # fast=True: bf16 GEMM operands (model.Backbone), as OrbCalculator does
        self.session = Session(bundle, task_name=task_name, device=dev, gamma=gamma,
                               max_neighbors=max_neighbors, fast=fast)
        self.task = self.task_name = self.session.task

    @classmethod
    def from_uma(cls, model="uma-s-1", task_name="omol", atoms=None, charge=0, spin=1,
                 refenv=None, checkpoint=None, cache_dir=None, device=None, device_id=0,
                 fast=False, trace=False, **kwargs):
        """Calculator for ``atoms`` from the composition-keyed bundle cache (calculator.py:68-110):
        charge / spin in ``atoms.info`` win over the arguments and are stamped back onto the
        atoms, so the bundle's merged routing and the runtime system embedding agree."""
        from . import bundle_cache
        if atoms is None:
            raise ValueError("from_uma needs `atoms`: the merged bundle is chosen by the reduced "
                             "composition, charge, spin and task")
        charge = atoms.info.get("charge", charge)
        spin = atoms.info.get("spin", spin)
        atoms.info.setdefault("charge", charge)
        atoms.info.setdefault("spin", spin)
        path = bundle_cache.get_or_build(atoms, model=model, task=task_name, charge=charge,
                                         spin=spin, refenv=refenv, checkpoint=checkpoint,
                                         cache_dir=cache_dir)
        return cls(str(path), task_name=task_name, device=device, device_id=device_id,
                   fast=fast, trace=trace, **kwargs)

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
