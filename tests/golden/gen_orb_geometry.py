"""Writes tests/golden/orb_geometry_small.npz: input/output vectors of the reference's Orb edge
geometry (tt_atom/orb_geometry.py:29-139, tt_atom/orb_model.py:69-82).

Run in the build container only (the reference is not available anywhere else):

    python tests/golden/gen_orb_geometry.py /root/reference

The closed forms of the Bessel basis and the cutoff envelope are pinned by mathematics in the
tests; what only the reference itself fixes is the component order and signs of the real
spherical harmonics (orb_geometry.py:37-62) and the flattening order of the rbf (x) sh outer
product (orb_geometry.py:95-96).  Those are what this fixture records, together with the
closed-form force VJP on the same inputs (orb_geometry.py:100-139)."""
import os
import sys

import numpy as np
import torch


def main(ref_root):
    sys.path.insert(0, ref_root)
    from tt_atom.orb_geometry import (bessel_basis, host_edge_features,  # noqa: E402
                                      host_edge_features_vjp, spherical_harmonics_l3)
    from tt_atom.orb_model import host_cutoff  # noqa: E402

    g = torch.Generator().manual_seed(23)
    n_nodes, n_edges = 12, 48
    pos = 2.0 * torch.randn(n_nodes, 3, dtype=torch.float64, generator=g)
    senders = torch.randint(n_nodes, (n_edges,), generator=g)
    receivers = (senders + torch.randint(1, n_nodes, (n_edges,), generator=g)) % n_nodes
    shift = 0.3 * torch.randn(n_edges, 3, dtype=torch.float64, generator=g)
    vec = pos[receivers] - pos[senders] + shift
    shift = shift * torch.clamp(5.5 / vec.norm(dim=-1), max=1.0)[:, None]
    edge_feat, cutoff, vectors = host_edge_features(pos, senders, receivers, shift)
    g_edge = torch.randn(edge_feat.shape, dtype=torch.float64, generator=g)
    g_cut = torch.randn(cutoff.shape, dtype=torch.float64, generator=g)
    forces = host_edge_features_vjp(vectors, senders, receivers, n_nodes, g_edge, g_cut)
    units = torch.nn.functional.normalize(torch.randn(32, 3, dtype=torch.float64, generator=g), dim=-1)
    r = torch.linspace(0.3, 6.5, 40, dtype=torch.float64)
    out = dict(pos=pos, senders=senders, receivers=receivers, shift=shift, edge_feat=edge_feat,
               cutoff=cutoff, vectors=vectors, g_edge=g_edge, g_cutoff=g_cut, forces=forces,
               units=units, sh=spherical_harmonics_l3(units), r=r,
               bessel=bessel_basis(r), envelope=host_cutoff(r))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "orb_geometry_small.npz")
    np.savez_compressed(path, **{k: v.numpy() for k, v in out.items()})
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
