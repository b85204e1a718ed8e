"""Weight bundles in the reference's ``.npz`` layout (bundle.py:18-37, weights.py:19-136).

Keys: ``config`` (JSON bytes), ``w@<state_dict key>`` weights, ``host@<name>`` fixed buffers
(to_m, gauss_offset, gauss_coeff, to_grid_mat, from_grid_mat), optional ``scale@rmsd``,
``scale@mean``, ``scale@elem_refs`` energy normalizer.  Loading never unpickles
(``allow_pickle=False``)."""
from __future__ import annotations

import json
import pathlib

import numpy as np
import torch


class NpzBundle:
    def __init__(self, npz):
        self._d = npz
        self.config = json.loads(bytes(npz["config"]).decode())

    @classmethod
    def load(cls, path):
        return cls(np.load(pathlib.Path(path), allow_pickle=False))

    def _t(self, key):
        return torch.from_numpy(np.array(self._d[key]))

    def has(self, key):
        return key in self._d.files if hasattr(self._d, "files") else key in self._d

    def keys(self):
        return list(self._d.files) if hasattr(self._d, "files") else list(self._d)

    @property
    def weights(self):
        return {k[2:]: self._t(k).float() for k in self.keys() if k.startswith("w@")}


class WeightBundle(NpzBundle):
    def buffer(self, name):
        return self._t(f"host@{name}").float()

    @property
    def task(self):
        return self.config.get("task", "omat")

    @property
    def scale_rmsd(self):
        return float(self._d["scale@rmsd"][0]) if self.has("scale@rmsd") else 1.0

    @property
    def scale_mean(self):
        return float(self._d["scale@mean"][0]) if self.has("scale@mean") else 0.0

    @property
    def elem_refs(self):
        return self._t("scale@elem_refs").double() if self.has("scale@elem_refs") else None

    @property
    def reference(self):
        """The merge inputs a merged bundle carries (``ref@*`` keys, weights.py:45-60): the
        system the MoLE routing was baked for (positions, numbers, charge, spin, optional cell /
        pbc) and its fairchem energy / forces, or None for bundles without them (random-init
        bundles)."""
        if not self.has("ref@energy"):
            return None
        d = self._d
        return dict(
            energy=float(d["ref@energy"][0]), forces=np.array(d["ref@forces"]),
            pos=np.array(d["ref@pos"]), atomic_numbers=np.array(d["ref@atomic_numbers"]),
            charge=float(d["ref@charge"][0]), spin=float(d["ref@spin"][0]),
            cell=np.array(d["ref@cell"]) if self.has("ref@cell") else None,
            pbc=np.array(d["ref@pbc"]) if self.has("ref@pbc") else None)

    @property
    def to_m(self):
        return self.buffer("to_m")

    @property
    def coefficient_index(self):
        return self._t("host@coefficient_index").long() if self.has("host@coefficient_index") else None

    @property
    def gauss_offset(self):
        return self.buffer("gauss_offset")

    @property
    def gauss_coeff(self):
        return self.buffer("gauss_coeff")

    @property
    def to_grid_mat(self):
        return self.buffer("to_grid_mat") if self.has("host@to_grid_mat") else None

    @property
    def from_grid_mat(self):
        return self.buffer("from_grid_mat") if self.has("host@from_grid_mat") else None

    def expected_keys(self):
        """Weight keys the modules consume (weights.py:90-130)."""
        cfg = self.config
        keys = ["sphere_embedding.weight", "source_embedding.weight", "target_embedding.weight",
                "mix_csd.weight", "mix_csd.bias"]
        if cfg.get("chg_spin_emb_type", "pos_emb") == "rand_emb":
            keys += ["charge_embedding.rand_emb.weight", "spin_embedding.rand_emb.weight"]
        else:
            keys += ["charge_embedding.W", "spin_embedding.W"]
        keys += [f"Jd_{l}" for l in range(cfg["lmax"] + 1)]
        for i in (0, 1, 3, 4, 6):
            keys += [f"edge_degree_embedding.rad_func.net.{i}.weight",
                     f"edge_degree_embedding.rad_func.net.{i}.bias"]
        for li in range(cfg["num_layers"]):
            p = f"blocks.{li}"
            keys += [f"{p}.norm_1.affine_weight", f"{p}.norm_1.affine_bias",
                     f"{p}.norm_2.affine_weight", f"{p}.norm_2.affine_bias"]
            for c in (1, 2):
                keys += [f"{p}.edge_wise.so2_conv_{c}.fc_m0.weight",
                         f"{p}.edge_wise.so2_conv_{c}.fc_m0.bias"]
                keys += [f"{p}.edge_wise.so2_conv_{c}.so2_m_conv.{m - 1}.fc.weight"
                         for m in range(1, cfg["mmax"] + 1)]
            for i in (0, 1, 3, 4, 6):
                keys += [f"{p}.edge_wise.so2_conv_1.rad_func.net.{i}.weight",
                         f"{p}.edge_wise.so2_conv_1.rad_func.net.{i}.bias"]
            if cfg.get("ff_type", "grid") == "spectral":
                keys += [f"{p}.atom_wise.{n}" for n in (
                    "scalar_mlp.0.weight", "scalar_mlp.0.bias", "so3_linear_1.weight",
                    "so3_linear_1.bias", "so3_linear_2.weight", "so3_linear_2.bias")]
            else:
                keys += [f"{p}.atom_wise.grid_mlp.{gi}.weight" for gi in (0, 2, 4)]
        keys += ["norm.affine_weight", "norm.affine_bias"]
        keys += [f"energy_block.{i}.{t}" for i in (0, 2, 4) for t in ("weight", "bias")]
        return keys

    def verify_coverage(self):
        w = self.weights
        missing = [k for k in self.expected_keys() if k not in w]
        return (len(missing) == 0, missing, len(w))


def save_bundle(path, cfg, weights, host, scale=None, reference=None):
    """Write a bundle in the same layout the loader reads; ``reference`` (a dict with the keys
    of ``WeightBundle.reference``) is stored as the ``ref@*`` merge inputs."""
    d = {"config": np.frombuffer(json.dumps(cfg).encode(), dtype=np.uint8)}
    for k, v in weights.items():
        d[f"w@{k}"] = np.asarray(torch.as_tensor(v).detach().cpu().float().numpy())
    for k, v in host.items():
        if v is not None:
            d[f"host@{k}"] = np.asarray(torch.as_tensor(v).detach().cpu().numpy())
    for k, v in (scale or {}).items():
        d[f"scale@{k}"] = np.asarray(v, dtype=np.float64).reshape(-1)
    for k, v in (reference or {}).items():
        if v is None:
            continue
        if k in ("energy", "charge", "spin"):
            v = np.asarray([v], dtype=np.float64)
        d[f"ref@{k}"] = np.asarray(v)
    np.savez(pathlib.Path(path), **d)
