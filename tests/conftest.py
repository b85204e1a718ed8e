"""Shared fixtures: golden loader, marker registration and import paths."""
import json
import pathlib
import sys

import numpy as np
import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tt-atom_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the HIP kernels)")


class Golden:
    """Accessor over a golden npz in the reference's key layout (tests/util.py:20-44):
    ``w@`` weights, ``a@`` activations, ``host@`` host terms, ``in@`` inputs, ``out@`` outputs."""

    def __init__(self, name):
        self.d = np.load(GOLDEN / name)
        self.config = json.loads(bytes(self.d["config"]).decode())

    def _t(self, key):
        return torch.from_numpy(self.d[key].copy())

    def w(self):
        return {k[2:]: self._t(k).float() for k in self.d.files if k.startswith("w@")}

    def act(self, name):
        return self._t(f"a@{name}").float()

    def host(self, name):
        return self._t(f"host@{name}").float()

    def inp(self, name):
        return self._t(f"in@{name}")

    def out(self, name):
        return self._t(f"out@{name}").float()

    def has(self, key):
        return key in self.d.files


@pytest.fixture(scope="session")
def golden():
    return Golden("golden_tiny.npz")


@pytest.fixture(scope="session")
def golden_bulk():
    return Golden("golden_bulk_tiny.npz")


def golden_bufs(g, ref=None):
    """Fixed buffers of a golden bundle (the bulk fixture lacks to_m / gaussian buffers; they are
    config constants shared with the molecule fixture, same config)."""
    src = g if g.has("host@to_m") else ref
    return dict(to_m=src.host("to_m"), gauss_offset=src.host("gauss_offset"),
                gauss_coeff=src.host("gauss_coeff"), to_grid_mat=g.host("to_grid_mat"),
                from_grid_mat=g.host("from_grid_mat"))
