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


# ----------------------------------------------------------------------------- cell list
def _bins(grid, q):
    """The kernel's bin coordinates u = fl(fl(x - origin) * inv_h) in fp32 (numpy float32
    arithmetic rounds every operation once, as __fsub_rn / __fmul_rn do)."""
    origin, inv_h, dims = grid
    u = (q.astype(np.float32) - np.asarray(origin, np.float32)) * np.float32(inv_h)
    assert u.dtype == np.float32
    return np.floor(u).astype(np.int64), np.asarray(dims)


def _pairs_fp32(p, q, cutoff):
    """Pairs (row atom a, point b) that pass the fp32 tests of either list: the aperiodic
    fma-chain norm against the midpoint, or the periodic rounded sum of squares <= fp32 cutoff^2
    (the looser of the two is taken, so the check covers both)."""
    d = p[:, None, :].astype(np.float32) - q[None, :, :].astype(np.float32)
    x, y, z = d[..., 0], d[..., 1], d[..., 2]
    s = _fma_chain(x, y, z)
    d2 = ((x * x + y * y) + z * z).astype(np.float32)
    c32 = np.float32(cutoff)
    m = (float(np.nextafter(c32, np.float32(-np.inf))) + float(c32)) / 2.0
    return (s.astype(np.float64) < m * m) | (d2 <= np.float32(cutoff * cutoff))


def _assert_covered(p, q, cutoff, grid):
    bp, dims = _bins(grid, p)
    bq, _ = _bins(grid, q)
    # every row atom is on the grid with its 27 neighbour bins
    assert (bp >= 1).all() and (bp <= dims - 2).all()
    hit = _pairs_fp32(p, q, cutoff)
    a, b = np.nonzero(hit)
    assert a.size > 0
    assert (np.abs(bp[a] - bq[b]) <= 1).all()
    # a point that is a hit never falls off the grid
    assert ((bq[b] >= 0) & (bq[b] < dims)).all()


def _at_cutoff_pairs(rng, n, cutoff, scale):
    """Pairs placed at the cutoff to the last ulp (both sides) in random directions."""
    base = rng.uniform(-scale, scale, (n, 3)).astype(np.float32)
    v = rng.normal(size=(n, 3))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    c = np.float32(cutoff)
    out = [base]
    for dist in (c, np.nextafter(c, np.float32(0)), np.nextafter(c, np.float32(99))):
        out.append((base + (v * float(dist)).astype(np.float32)).astype(np.float32))
    return np.concatenate(out)


@pytest.mark.parametrize("cutoff,scale,offset", [(6.0, 20.0, 0.0), (5.0, 30.0, 1000.0),
                                                 (12.345, 40.0, -3000.0), (6.0, 8.0, 40000.0)])
def test_cell_grid_covers_every_pair(cutoff, scale, offset):
    """Every pair that passes the fp32 distance test lies in neighbouring bins on every axis,
    with the bin coordinates computed as the kernels compute them: random clusters, pairs at
    the cutoff to the last ulp, atoms on bin boundaries, far-from-origin coordinates."""
    rng = np.random.default_rng(int(cutoff * 100) + int(scale))
    p = np.concatenate([rng.uniform(-scale, scale, (600, 3)).astype(np.float32),
                        _at_cutoff_pairs(rng, 150, cutoff, scale)]) + np.float32(offset)
    p = p.astype(np.float32)
    grid = geometry.cell_grid(p, cutoff)
    origin, inv_h, dims = grid
    assert 1.0 / inv_h >= cutoff
    # atoms moved onto bin boundaries (the value whose fp32 bin coordinate is an integer) and
    # partners at the cutoff from them along the axes
    h = 1.0 / inv_h
    k = rng.integers(2, int(dims[0]) - 2, 50)
    edge = (np.float32(origin[0]) + (k * h)).astype(np.float32)
    on = np.stack([edge, rng.uniform(-scale, scale, 50) + offset,
                   rng.uniform(-scale, scale, 50) + offset], 1).astype(np.float32)
    on2 = on.copy()
    on2[:, 0] = (on[:, 0] + np.float32(cutoff)).astype(np.float32)
    on3 = on.copy()
    on3[:, 0] = (on[:, 0] - np.nextafter(np.float32(cutoff), np.float32(0))).astype(np.float32)
    p = np.concatenate([p, on, on2, on3]).astype(np.float32)
    grid = geometry.cell_grid(p, cutoff)
    _assert_covered(p, p, cutoff, grid)


def test_cell_grid_covers_periodic_images():
    """Periodic image points q = fl(pos_j + shift_c) (rounded as the distance test rounds them)
    that pass the test against a receiver are in its neighbouring bins or on the grid's
    border-free interior; images off the grid are never hits."""
    from tt_atom import synthetic
    pos, Z, cell = synthetic.c4_system(reps=3)
    pos = (pos + np.random.default_rng(2).normal(0, 0.05, pos.shape)).astype(np.float32)
    shifts = geometry._image_shifts(torch.from_numpy(pos), 6.0, torch.from_numpy(cell),
                                    [True, True, False]).numpy().astype(np.float32)
    q = (pos[:, None, :] + shifts[None, :, :]).astype(np.float32).reshape(-1, 3)
    grid = geometry.cell_grid(pos, 6.0)
    bq, dims = _bins(grid, q)
    off = ((bq < 0) | (bq >= dims)).any(1)
    hit = _pairs_fp32(pos, q, 6.0)
    assert not hit[:, off].any()
    _assert_covered(pos, q[~off], 6.0, grid)


def test_cell_grid_ignores_non_finite_atoms():
    p = np.random.default_rng(3).uniform(-20, 20, (500, 3)).astype(np.float32)
    g = geometry.cell_grid(p, 6.0)
    q = p.copy()
    q[7] = np.nan
    q[9, 2] = np.inf
    q[11, 0] = -np.inf
    assert geometry.cell_grid(q, 6.0) == geometry.cell_grid(np.delete(q, [7, 9, 11], 0), 6.0)
    assert geometry.cell_grid(np.full((4, 3), np.nan, np.float32), 6.0)[2] == (4, 4, 4)
    assert g[2] == geometry.cell_grid(p[::-1], 6.0)[2]


def test_cell_grid_sparse_system_bounds_bins():
    """A sparse system (atoms spread far apart) gets wider bins, never more than the bin cap,
    and still covers its pairs."""
    rng = np.random.default_rng(9)
    p = np.concatenate([rng.uniform(-5000, 5000, (300, 3)),
                        rng.uniform(-5, 5, (100, 3))]).astype(np.float32)
    grid = geometry.cell_grid(p, 6.0)
    assert int(np.prod(grid[2])) <= 4096 and 1.0 / grid[1] > 6.0
    _assert_covered(p, p, 6.0, grid)
    grid = geometry.cell_grid(p, 6.0, max_bins=100)
    assert int(np.prod(grid[2])) <= 100
    _assert_covered(p, p, 6.0, grid)


def _lattice_cluster(n, spacing, seed):
    from tt_atom import synthetic
    return torch.from_numpy(synthetic.lattice_cluster(n, spacing, seed))


def _shuffled_fcc(reps, seed):
    from tt_atom import synthetic
    pos, cell = synthetic.shuffled_fcc(reps, seed)
    return torch.from_numpy(pos), torch.from_numpy(cell)


def _timed(fn):
    torch.cuda.synchronize()
    import time
    t0 = time.perf_counter()
    out = fn()
    torch.cuda.synchronize()
    return out, (time.perf_counter() - t0) * 1e3


@pytest.mark.gpu
@pytest.mark.parametrize("cap", [None, 30, 7])
def test_cell_list_cluster_equals_host(cap):
    pos = _lattice_cluster(5000, 2.2, 1)
    print(f"cell list vs host: cluster N={pos.shape[0]} cap={cap}", flush=True)
    _same(geometry.radius_graph(pos, 6.0, max_neighbors=cap),
          geometry.radius_graph_device(pos, 6.0, max_neighbors=cap, method="cells"))


@pytest.mark.gpu
@pytest.mark.parametrize("cap", [None, 30])
def test_cell_list_periodic_equals_host(cap):
    """3-D crystal, slab and wire; a 4-atom cell whose images reach two cells out (125 shifts);
    atoms in shuffled order."""
    for reps, pbc in ((4, [True] * 3), (4, [True, True, False]), (3, [False, True, False]),
                      (1, [True] * 3)):
        pos, cell = _shuffled_fcc(reps, reps)
        print(f"cell list vs host: periodic reps={reps} pbc={pbc} cap={cap}", flush=True)
        _same(geometry.radius_graph(pos, 6.0, cell, pbc, max_neighbors=cap),
              geometry.radius_graph_device(pos, 6.0, cell, pbc, max_neighbors=cap,
                                           method="cells"))


@pytest.mark.gpu
def test_cell_list_at_the_cutoff_and_degenerate():
    """Pairs at the cutoff to the last ulp (as test_device_graph_at_the_cutoff), one atom, two
    coincident atoms (no edge: d = 0), and an empty system."""
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
    for cap in (None, 1):
        _same(geometry.radius_graph(pos, 6.0, max_neighbors=cap),
              geometry.radius_graph_device(pos, 6.0, max_neighbors=cap, method="cells"))
    for p in (torch.zeros(1, 3), torch.ones(2, 3), torch.tensor([[0.0, 0, 0], [1.0, 0, 0],
                                                                [1.0, 0, 0]])):
        _same(geometry.radius_graph(p, 6.0), geometry.radius_graph_device(p, 6.0,
                                                                          method="cells"))
    ei, sh = geometry.radius_graph_device(torch.zeros(0, 3), 6.0, method="cells")
    assert ei.shape == (2, 0) and sh.shape == (0, 3)
    # non-finite atoms have no edge and do not disturb the grid of the others
    p = _lattice_cluster(600, 2.2, 5)
    p[3] = float("nan")
    p[10, 1] = float("inf")
    p[11, 2] = -float("inf")
    for cap in (None, 8):
        _same(geometry.radius_graph(p, 6.0, max_neighbors=cap),
              geometry.radius_graph_device(p, 6.0, max_neighbors=cap, method="cells"))


@pytest.mark.gpu
def test_cell_list_dense_rows_and_large_cap():
    """Rows of more than 2048 kept entries (written by the row-scan write pass), a cap of 1000
    (the one-wave threshold launch) over 2999 candidates per receiver, and caps above the
    selection's 1024 limit: a no-op one (3000) is dropped, a binding one (2100) is refused."""
    rng = np.random.default_rng(4)
    pos = torch.from_numpy(rng.uniform(0, 20.0, (3000, 3)).astype(np.float32))
    for cap in (None, 1000, 3000):
        print(f"cell list dense: cap={cap}", flush=True)
        _same(geometry.radius_graph(pos, 40.0, max_neighbors=cap),
              geometry.radius_graph_device(pos, 40.0, max_neighbors=cap, method="cells"))
    with pytest.raises(ValueError):
        geometry.radius_graph_device(pos, 40.0, max_neighbors=2100, method="cells")


@pytest.mark.gpu
@pytest.mark.parametrize("cap", [None, 30])
def test_cell_list_50k_cluster_equals_row_scan(cap):
    """A 50k-atom cluster: cell list == row scan edge for edge (the host list would need a
    50k x 50k distance matrix); times both."""
    pos = _lattice_cluster(52000, 2.2, 2)
    assert pos.shape[0] >= 50000
    print(f"cell list vs row scan: cluster N={pos.shape[0]} cap={cap}", flush=True)
    geometry.radius_graph_device(pos[:5000], 6.0, max_neighbors=cap, method="cells")  # warm-up
    rows, t_rows = _timed(lambda: geometry.radius_graph_device(pos, 6.0, max_neighbors=cap,
                                                               method="rows"))
    cells, t_cells = _timed(lambda: geometry.radius_graph_device(pos, 6.0, max_neighbors=cap,
                                                                 method="cells"))
    print(f"  E={rows[0].shape[1]} rows {t_rows:.2f} ms, cells {t_cells:.2f} ms", flush=True)
    assert rows[0].shape[1] > 20 * pos.shape[0]
    _same(rows, cells)


@pytest.mark.gpu
@pytest.mark.parametrize("cap", [None, 30])
def test_cell_list_periodic_slab_equals_row_scan(cap):
    """A 55k-atom FCC slab (periodic in x and y) in shuffled order: cell list == row scan."""
    pos, cell = _shuffled_fcc(24, 7)
    assert pos.shape[0] >= 50000
    pbc = [True, True, False]
    print(f"cell list vs row scan: slab N={pos.shape[0]} cap={cap}", flush=True)
    rows, t_rows = _timed(lambda: geometry.radius_graph_device(pos, 6.0, cell, pbc,
                                                               max_neighbors=cap, method="rows"))
    cells, t_cells = _timed(lambda: geometry.radius_graph_device(pos, 6.0, cell, pbc,
                                                                 max_neighbors=cap,
                                                                 method="cells"))
    print(f"  E={rows[0].shape[1]} rows {t_rows:.2f} ms, cells {t_cells:.2f} ms", flush=True)
    assert rows[0].shape[1] > 20 * pos.shape[0]
    _same(rows, cells)


@pytest.mark.gpu
def test_system_graphs_routes_large_systems_to_cells(monkeypatch):
    """system_graphs("device") sends systems above the size thresholds (lowered here so the host
    list stays cheap) through the cell list one at a time and batches the rest in row scans;
    every graph equals the host's."""
    from tt_atom import synthetic
    monkeypatch.setattr(geometry, "CELL_LIST_MIN_ATOMS_APERIODIC", 1000)
    monkeypatch.setattr(geometry, "CELL_LIST_MIN_ATOMS_PERIODIC", 200)
    calls = []
    orig = geometry.radius_graph_device
    monkeypatch.setattr(geometry, "radius_graph_device",
                        lambda *a, **kw: calls.append(kw.get("method")) or orig(*a, **kw))
    big = _lattice_cluster(1200, 2.2, 3)
    pos_p, cell_p = _shuffled_fcc(4, 3)
    items = [(torch.from_numpy(p), None, None) for p, _ in synthetic.c5_systems(K=3)]
    items.insert(1, (big, None, None))
    items.append((pos_p, cell_p, [True, True, False]))
    items.append((pos_p[:100].clone(), cell_p, [True] * 3))     # small periodic: row scan
    host = geometry.system_graphs(items, 6.0, 20, "host")
    dev = geometry.system_graphs(items, 6.0, 20, "device")
    assert calls.count("cells") == 2
    for (ei_h, sh_h), (ei_d, sh_d) in zip(host, dev):
        assert torch.equal(ei_h.cpu().long(), ei_d.cpu().long())
        assert torch.equal(sh_h.cpu().float(), sh_d.cpu().float())


def _sum_sq_cases(n_want, seed):
    """Periodic pairs (pj, pt), each 40 A further along z, whose squared distance, rounded product
    by product and sum by sum as the host rounds it, lies on the other side of
    fp32(cutoff^2) = 36 than either fused evaluation fma(z, z, fma(x, x, y*y)) /
    fma(z, z, fma(y, y, x*x)) would put it: the device kernels must not contract the sum of
    squares.  Returns [(pj, pt, inside)]."""
    rng = np.random.default_rng(seed)
    f32 = np.float32
    fma = lambda a, b, c: f32(np.float64(a) * np.float64(b) + np.float64(c))  # exact products
    out = []
    while len(out) < n_want:
        pj = (rng.uniform(-3, 3, 3) + [0.0, 0.0, 40.0 * len(out)]).astype(f32)
        v = rng.normal(size=3)
        v = v / np.linalg.norm(v) * 6.0
        pt0 = (pj + v.astype(f32)).astype(f32)
        for step in range(-6, 7):
            q = pt0.copy()
            for _ in range(abs(step)):
                q[0] = np.nextafter(q[0], f32(np.inf) if step > 0 else f32(-np.inf))
            x, y, z = (q - pj).astype(f32)
            sep = f32(f32(f32(x * x) + f32(y * y)) + f32(z * z))
            fa = fma(z, z, fma(x, x, f32(y * y)))
            fb = fma(z, z, fma(y, y, f32(x * x)))
            inside = bool(sep <= f32(36.0))
            if inside != bool(fa <= f32(36.0)) and inside != bool(fb <= f32(36.0)):
                out.append((pj, q, inside))
                break
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("method", ["rows", "cells"])
def test_device_graph_sum_of_squares_is_not_fused(method):
    cases = _sum_sq_cases(24, 3)
    assert any(c[2] for c in cases) and not all(c[2] for c in cases)
    pos = torch.tensor(np.asarray([p for pj, pt, _ in cases for p in (pj, pt)], np.float32))
    cell = torch.eye(3) * 2000.0
    host = geometry.radius_graph(pos, 6.0, cell, [True] * 3)
    kept = {(int(a), int(b)) for a, b in host[0].t().tolist()}
    for k, (_, _, inside) in enumerate(cases):
        assert ((2 * k, 2 * k + 1) in kept) == inside          # the host rounds term by term
    _same(host, geometry.radius_graph_device(pos, 6.0, cell, [True] * 3, method=method))
