"""Device radius graph (csrc/neighbors.hip) against the host neighbour list.

CPU tests pin the two pieces of arithmetic the kernel relies on: the host's fp32 norm is the
fused-multiply-add chain sqrt(fma(z, z, fma(y, y, x*x))), and "fp32 sqrt(s) < fp32(cutoff)" equals
"s < m^2" with m the midpoint below fp32(cutoff).  GPU tests require the device graph to equal
``radius_graph`` edge for edge (indices, order and shifts) on clusters, periodic crystals, capped
and uncapped, batched molecules, and pairs placed at the cutoff to the last ulp."""
import numpy as np
import pytest
import torch

from tt_atom import geometry


def _fma_chain(x, y, z):
    # single-rounding fma emulated in double (the products of fp32 values are exact in double)
    f = lambda a, b, c: (a.astype(np.float64) * b + c.astype(np.float64)).astype(np.float32)
    return f(z, z, f(y, y, (x * x).astype(np.float32)))


def test_host_norm_is_fma_chain():
    g = torch.Generator().manual_seed(5)
    pos = (torch.rand(700, 3, generator=g) * 24 - 12).float()
    diff = pos[:, None, :] - pos[None, :, :]
    d = torch.linalg.norm(diff, dim=-1).numpy()
    x, y, z = (diff[..., k].numpy() for k in range(3))
    s = _fma_chain(x, y, z)
    assert np.array_equal(np.sqrt(s.astype(np.float64)).astype(np.float32), d)


@pytest.mark.parametrize("cutoff", [5.0, 6.0, 4.7, 12.345])
def test_midpoint_predicate(cutoff):
    c32 = np.float32(cutoff)
    m = (float(np.nextafter(c32, np.float32(-np.inf))) + float(c32)) / 2.0
    mid2 = m * m
    c2 = np.float32(float(c32) ** 2)
    # every fp32 s within 4000 ulps of c32^2, plus random ones
    ulps = np.arange(-4000, 4001, dtype=np.int64)
    s = (np.array([c2], np.float32).view(np.int32).astype(np.int64) + ulps).astype(np.int32)
    s = np.concatenate([s.view(np.float32),
                        np.random.default_rng(0).uniform(0, 4 * float(c2), 20000).astype(np.float32)])
    d = np.sqrt(s.astype(np.float64)).astype(np.float32)     # correctly rounded fp32 sqrt
    assert np.array_equal(d < c32, s.astype(np.float64) < mid2)


def _cluster(n, radius, seed):
    from tt_atom import synthetic
    pos, Z = synthetic.c3_system(seed=seed, n=n, radius=radius)
    return torch.from_numpy(pos).float()


def _same(a, b):
    (ei_h, sh_h), (ei_d, sh_d) = a, b
    assert ei_h.shape == ei_d.shape, (ei_h.shape, ei_d.shape)
    assert torch.equal(ei_h.cpu().long(), ei_d.cpu())
    assert torch.equal(sh_h.cpu().float(), sh_d.cpu())


@pytest.mark.gpu
@pytest.mark.parametrize("cap", [None, 30, 7])
def test_device_graph_cluster(cap):
    pos = _cluster(2048, 17.0, 3)
    _same(geometry.radius_graph(pos, 6.0, max_neighbors=cap),
          geometry.radius_graph_device(pos, 6.0, max_neighbors=cap))


@pytest.mark.gpu
@pytest.mark.parametrize("cap", [None, 30])
def test_device_graph_periodic(cap):
    from tt_atom import synthetic
    pos, Z, cell = synthetic.c4_system(reps=4)
    pos, cell = torch.from_numpy(pos).float(), torch.from_numpy(cell).float()
    _same(geometry.radius_graph(pos, 6.0, cell, [True] * 3, max_neighbors=cap),
          geometry.radius_graph_device(pos, 6.0, cell, [True] * 3, max_neighbors=cap))
    # mixed periodicity (slab)
    _same(geometry.radius_graph(pos, 6.0, cell, [True, True, False], max_neighbors=cap),
          geometry.radius_graph_device(pos, 6.0, cell, [True, True, False], max_neighbors=cap))


@pytest.mark.gpu
def test_device_graph_at_the_cutoff():
    """Pairs whose fp32 distance lands on, one ulp inside and one ulp outside the cutoff, along
    axis and skewed directions (pairs 40 A apart from each other)."""
    c = np.float32(6.0)
    pts = []
    for dist in (c, np.nextafter(c, np.float32(0)), np.nextafter(c, np.float32(9))):
        for dirn in ([1, 0, 0], [0, 1, 0], [0.6, 0.8, 0.0], [0.48, 0.6, 0.64]):
            base = np.float32([40.0 * len(pts), 0.0, 0.0])
            v = np.asarray(dirn, np.float64)
            v = v / np.linalg.norm(v) * float(dist)
            pts.append(base)
            pts.append(base + np.float32(v))
    pos = torch.tensor(np.asarray(pts, np.float32))
    d = torch.linalg.norm(pos[0::2] - pos[1::2], dim=-1)
    assert bool((d < 6.0).any()) and bool((d >= 6.0).any())      # both sides are exercised
    for cap in (None, 1):
        _same(geometry.radius_graph(pos, 6.0, max_neighbors=cap),
              geometry.radius_graph_device(pos, 6.0, max_neighbors=cap))


@pytest.mark.gpu
def test_device_graph_batched_molecules():
    from tt_atom import synthetic
    systems = synthetic.c5_systems(K=40)
    parts, off, pos_all, lo, hi = [], 0, [], [], []
    for p, Z in systems:
        p = torch.as_tensor(np.asarray(p), dtype=torch.float32)
        ei, _ = geometry.radius_graph(p, 6.0, max_neighbors=20)
        parts.append(ei + off)
        n = p.shape[0]
        pos_all.append(p)
        lo += [off] * n
        hi += [off + n] * n
        off += n
    ref = torch.cat(parts, 1)
    ei_d, sh_d = geometry.radius_graph_device(torch.cat(pos_all), 6.0, max_neighbors=20,
                                              node_ranges=(torch.tensor(lo), torch.tensor(hi)))
    assert torch.equal(ref, ei_d.cpu()) and not sh_d.any()


@pytest.mark.gpu
def test_assemble_orb_device_equals_host():
    from tt_atom import orb, synthetic
    systems = synthetic.c5_systems(K=12)
    pos, Z, cell = synthetic.c4_system(reps=2)
    systems = systems[:5] + [dict(positions=pos, numbers=Z, cell=cell, pbc=[True] * 3)] + systems[5:]
    h = orb.assemble_orb(systems, 6.0, 20, truncate=True)
    d = orb.assemble_orb(systems, 6.0, 20, neighbor_list="device", truncate=True)
    for a, b in ((h.senders, d.senders), (h.receivers, d.receivers), (h.cell_shift, d.cell_shift),
                 (h.pos, d.pos), (h.Z, d.Z), (h.batch, d.batch)):
        assert torch.equal(a, b)
    assert h.natoms == d.natoms


@pytest.mark.gpu
@pytest.mark.parametrize("cap", [None, 12])
def test_device_graph_batched_periodic(cap):
    """Periodic systems of one batch share one device pass (per-row node and image-shift ranges):
    each system's graph equals the host's on it alone, edge for edge with the same shifts, for
    different cells, sizes, periodicities (3-D, slab, wire) and image counts, with aperiodic
    systems mixed in."""
    from tt_atom import synthetic
    g = np.random.default_rng(5)
    items = []
    for reps, pbc, scale in ((2, [True] * 3, 1.0), (3, [True, True, False], 1.03),
                             (1, [True] * 3, 0.97), (2, [False, True, False], 1.0)):
        pos, Z, cell = synthetic.c4_system(reps=reps)
        pos = (pos * scale + g.normal(0, 0.05, pos.shape)).astype(np.float32)
        items.append((torch.from_numpy(pos), torch.from_numpy((cell * scale).astype(np.float32)),
                      pbc))
    items.insert(2, (torch.from_numpy(synthetic.c5_systems(K=1)[0][0].astype(np.float32)), None,
                     None))
    host = geometry.system_graphs(items, 6.0, cap, "host")
    dev = geometry.system_graphs(items, 6.0, cap, "device")
    for (ei_h, sh_h), (ei_d, sh_d) in zip(host, dev):
        assert ei_h.shape[1] > 0
        assert torch.equal(ei_h.cpu().long(), ei_d.cpu().long())
        assert torch.equal(sh_h.cpu().float(), sh_d.cpu().float())
