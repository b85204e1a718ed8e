"""Weight bundle of the Orb-v3 path (reference orb_weights.py:15-26).

The ``.npz`` container holds a ``config`` JSON and the MoleculeGNS state dict under ``w@<key>``
(tools/export_orb_weights.py:51-82 writes it), optionally with ``a@`` activations, ``host@``
host terms, ``in@`` inputs and ``out@`` outputs of a reference run.  The container mechanics
(config parse, lazy tensor copy, ``weights``) are shared with the eSCN-MD bundle
(``tt_atom.weights.NpzBundle``); the accessors below are the Orb ones.
"""
from __future__ import annotations

from .weights import NpzBundle

__all__ = ["OrbWeights"]


class OrbWeights(NpzBundle):
    """``OrbWeights.load(path).weights`` -> {state-dict key: fp32 tensor}; ``config`` -> dict."""

    def activation(self, key):
        return self._t(f"a@{key}").float()

    def host(self, key):
        return self._t(f"host@{key}").float()

    def inp(self, key):
        return self._t(f"in@{key}")

    def out(self, key):
        return self._t(f"out@{key}")
