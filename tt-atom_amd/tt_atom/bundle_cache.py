"""Composition-keyed UMA bundle cache (reference bundle_cache.py:1-188), cache hits only.

UMA's mixture-of-linear-experts routing is merged into the weights for one (reduced composition,
charge, spin, task), so a merged ``.npz`` bundle serves exactly one such key.  The cache path is
the reference's own naming, so a bundle directory the reference built (``$TT_ATOM_CACHE`` or
``~/.cache/tt_atom/bundles``) is found and loaded as is.  Building a missing bundle needs the
reference environment (fairchem and the gated UMA checkpoint, fetched over the network); that is
not part of this build, so a miss raises ``BundleNotCached`` naming the file to provide.
"""
from __future__ import annotations

import hashlib
import math
import os
import pathlib
from collections import Counter
from functools import reduce

import numpy as np

CACHE_DIR = pathlib.Path(
    os.environ.get("TT_ATOM_CACHE", pathlib.Path.home() / ".cache" / "tt_atom" / "bundles"))


class BundleNotCached(RuntimeError):
    """The merged bundle for this key is not in the cache directory."""


def _numbers(atoms_or_numbers):
    if hasattr(atoms_or_numbers, "get_atomic_numbers"):
        return np.asarray(atoms_or_numbers.get_atomic_numbers())
    return np.asarray(atoms_or_numbers)


def infer_task(atoms_or_pbc):
    """'omat' for a fully periodic cell, otherwise 'omol' (bundle_cache.py:36-43)."""
    pbc = atoms_or_pbc.get_pbc() if hasattr(atoms_or_pbc, "get_pbc") else atoms_or_pbc
    if pbc is None:
        return "omol"
    return "omat" if np.asarray(pbc, dtype=bool).all() else "omol"


def reduced_composition(numbers):
    """Sorted ((Z, count / gcd of the counts), ...): H2O and H4O2 share a key
    (bundle_cache.py:46-54)."""
    counts = Counter(int(z) for z in np.asarray(numbers).reshape(-1))
    if not counts:
        raise ValueError("a composition needs at least one atom")
    g = reduce(math.gcd, counts.values())
    return tuple(sorted((z, c // g) for z, c in counts.items()))


def composition_hash(numbers):
    """First 12 hex digits of SHA-1 over "Z:count;Z:count..." of the reduced composition
    (bundle_cache.py:64-67)."""
    key = ";".join(f"{z}:{c}" for z, c in reduced_composition(numbers))
    return hashlib.sha1(key.encode()).hexdigest()[:12]


def bundle_path(model, task, numbers, charge, spin, cache_dir=None, checkpoint=None):
    """``{model}_{task}_{hash}_c{charge}_s{spin}[_ckpt{sha1(path)[:12]}].npz`` under the cache
    directory (bundle_cache.py:69-79); an explicit checkpoint path gets its own namespace."""
    suffix = ""
    if checkpoint is not None:
        ident = str(pathlib.Path(checkpoint).expanduser().resolve())
        suffix = f"_ckpt{hashlib.sha1(ident.encode()).hexdigest()[:12]}"
    name = (f"{model}_{task}_{composition_hash(numbers)}_c{int(charge)}_s{int(spin)}"
            f"{suffix}.npz")
    return pathlib.Path(cache_dir or CACHE_DIR) / name


def get_or_build(atoms, *, model="uma-s-1", task="omol", charge=0, spin=1, refenv=None,
                 checkpoint=None, cache_dir=None, log=True):
    """Path of the cached bundle for ``atoms`` (an ASE Atoms or an array of atomic numbers)
    (bundle_cache.py:170-188).  ``refenv`` and ``log`` are accepted for signature compatibility;
    on a miss this raises ``BundleNotCached`` instead of running the reference exporter."""
    del refenv, log
    path = bundle_path(model, task, _numbers(atoms), charge, spin, cache_dir=cache_dir,
                       checkpoint=checkpoint)
    if path.exists():
        return path
    raise BundleNotCached(
        f"no merged {model} bundle for this composition (task={task}, charge={int(charge)}, "
        f"spin={int(spin)}) at {path}.  Building one merges the UMA experts with fairchem and "
        "the gated checkpoint, which this build does not do: export it with the reference's "
        "tools/export_weights.py where fairchem is installed and copy the .npz to that path "
        "(or set TT_ATOM_CACHE / cache_dir to the directory that holds it).")
