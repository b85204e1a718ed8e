"""Per-checkpoint Orb weight cache (reference orb_weight_cache.py:1-51), cache hits only.

Orb merges no routing into its weights, so one exported ``.npz`` per checkpoint name serves every
system.  The path is the reference's (``$TT_ATOM_CACHE/orb_weights/<name>.npz``, default
``~/.cache/tt_atom/orb_weights``), so weights the reference exported are found as they are.
Exporting needs orb-models and the network; a miss raises ``WeightsNotCached``.
"""
from __future__ import annotations

import os
import pathlib

CACHE_DIR = pathlib.Path(
    os.environ.get("TT_ATOM_CACHE", pathlib.Path.home() / ".cache" / "tt_atom")) / "orb_weights"

CHECKPOINTS = ("orb-v3-conservative-inf-omat", "orb-v3-direct-20-omat",
               "orb-v3-conservative-omol", "orb-v3-direct-omol")


class WeightsNotCached(RuntimeError):
    """The exported weights for this checkpoint are not in the cache directory."""


def _short_name(checkpoint):
    if checkpoint not in CHECKPOINTS:
        raise ValueError(f"unknown Orb checkpoint {checkpoint!r}; choose from {CHECKPOINTS}")
    return checkpoint[len("orb-v3-"):]


def weights_path(checkpoint, cache_dir=None):
    """``<cache>/<checkpoint without the orb-v3- prefix>.npz`` (orb_weight_cache.py:33-34)."""
    return pathlib.Path(cache_dir or CACHE_DIR) / f"{_short_name(checkpoint)}.npz"


def get_or_build(checkpoint, *, refenv=None, cache_dir=None, log=True):
    """Path of the cached weights (orb_weight_cache.py:37-51); raises ``WeightsNotCached`` on a
    miss instead of running the reference exporter."""
    del refenv, log
    path = weights_path(checkpoint, cache_dir=cache_dir)
    if path.exists():
        return path
    raise WeightsNotCached(
        f"no exported weights for {checkpoint} at {path}.  Export them with the reference's "
        "tools/export_orb_weights.py where orb-models is installed and copy the .npz to that "
        "path (or set TT_ATOM_CACHE / cache_dir to the directory that holds it).")
