"""Per-op entry points of the rotation and scatter modules (tt_atom.rotation, tt_atom.scatter;
reference rotation.py:188-270, scatter.py:35-89).  CPU: the table and pattern bookkeeping
against brute force.  GPU: the sparse-pattern rotation, its VJP and the table segment sum
against fp64 dense products, autograd and index_add."""
import numpy as np
import pytest
import torch

DEV = "cuda"


def _blockdiag_wigner(E, g):
    """Random [E, 9, 9] matrices with the structure of the m-primed Wigner rows: row m couples
    the columns of its degree (0 | 1..3 | 4..8)."""
    deg = [0, 1, 2, 1, 2, 1, 2, 2, 2]
    cols = {0: [0], 1: [1, 2, 3], 2: [4, 5, 6, 7, 8]}
    W = torch.zeros(E, 9, 9, dtype=torch.float64)
    for m in range(9):
        for j in cols[deg[m]]:
            W[:, m, j] = torch.randn(E, generator=g, dtype=torch.float64)
    return W


# ------------------------------------------------------------------------------- host side
def test_build_gather_table():
    """Row n lists the edges of node n in edge order, then the sentinel; Dmax is the largest
    degree floored at min_width; an empty graph has width 1 (checked against a loop per node)."""
    from tt_atom.scatter import build_gather
    rng = np.random.default_rng(3)
    N, E = 37, 400
    idx = rng.integers(0, N - 3, E)                      # the last three nodes have no edges
    idx[:60] = 7                                         # a hub
    for sentinel, min_width in ((None, 0), (E + 5, 0), (None, 90)):
        flat, D = build_gather(torch.from_numpy(idx), N, E, sentinel=sentinel, min_width=min_width)
        sv = E if sentinel is None else sentinel
        assert flat.dtype == np.int32 and flat.shape == (N * D,)
        assert D == max(int(np.bincount(idx, minlength=N).max()), min_width)
        tab = flat.reshape(N, D)
        for n in range(N):
            mine = [e for e in range(E) if idx[e] == n]
            assert tab[n, :len(mine)].tolist() == mine
            assert (tab[n, len(mine):] == sv).all()
    flat, D = build_gather(torch.zeros(0, dtype=torch.int64), 4, 0)
    assert D == 1 and (flat == 0).all() and flat.shape == (4,)


def test_pack_pattern_and_scatter_round_trip():
    """pack of block-diagonal Wigner rows yields the 35 pairs in the packed order of the fused
    kernels (row-major over (m, j)); gather_coef and scatter_coef invert each other on the
    pattern, and pack drops only entries below tol on every edge."""
    from tt_atom import rotation
    g = torch.Generator().manual_seed(5)
    W = _blockdiag_wigner(6, g)
    ij, coef = rotation.pack(W)
    deg = [0, 1, 2, 1, 2, 1, 2, 2, 2]
    cols = {0: [0], 1: [1, 2, 3], 2: [4, 5, 6, 7, 8]}
    assert ij == [(m, j) for m in range(9) for j in cols[deg[m]]]
    ii = torch.tensor([i for i, _ in ij])
    jj = torch.tensor([j for _, j in ij])
    assert torch.equal(rotation.gather_coef(W, ii, jj), coef)
    assert torch.equal(rotation.scatter_coef(coef, ij, 9), W)
    W2 = W.clone()
    W2[:, 0, 0] = 1e-8                                   # below tol on every edge: dropped
    W2[3, 4, 5] = 0.0                                    # zero on one edge only: kept
    ij2, _ = rotation.pack(W2)
    assert (0, 0) not in ij2 and (4, 5) in ij2 and len(ij2) == 34
    # rectangular
    R = torch.randn(3, 5, 7, generator=g, dtype=torch.float64)
    R[:, :, 6] = 0.0
    ijr, cr = rotation.pack(R)
    assert len(ijr) == 30 and torch.equal(rotation.scatter_coef(cr, ijr, 5, 7), R)


def test_pattern_grouping():
    """The CSR grouping the rotation kernels take: by output row for rotate, by input column for
    the input adjoint, each group in pattern order."""
    from tt_atom.rotation import _grouped
    ij = [(0, 1), (2, 0), (0, 0), (1, 2), (2, 1)]
    ptr, k, other = _grouped(ij, 3, by_out=True)
    assert ptr == [0, 2, 3, 5] and k == [0, 2, 3, 1, 4] and other == [1, 0, 2, 0, 1]
    ptr, k, other = _grouped(ij, 3, by_out=False)
    assert ptr == [0, 2, 4, 5] and k == [1, 2, 0, 4, 3] and other == [2, 0, 0, 2, 1]


# ------------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("case", ["lmax2-W128", "lmax2-W7", "rect-19x25-W16"])
def test_rotate_and_vjp(case):
    """rotation.rotate / rotate_bw against the fp64 dense product and its autograd, on the
    lmax = 2 Wigner structure (W = 128 and an odd W = 7) and on a rectangular 19 x 25 pattern
    (the shape of a reduced-m rotation) with empty output rows."""
    from tt_atom import rotation
    g = torch.Generator().manual_seed(11)
    E = 257
    if case.startswith("lmax2"):
        W = int(case.split("W")[1])
        Wd = _blockdiag_wigner(E, g)
        n_out, n_in = 9, 9
    else:
        W, n_out, n_in = 16, 19, 25
        mask = torch.rand(n_out, n_in, generator=g) < 0.3
        mask[4] = False                                  # an output row with no terms
        Wd = torch.randn(E, n_out, n_in, generator=g, dtype=torch.float64) * mask
    ij, coef = rotation.pack(Wd)
    x = torch.randn(E, n_in, W, generator=g, dtype=torch.float64)
    xr, cr = x.clone().requires_grad_(True), coef.clone().requires_grad_(True)
    dense = rotation.scatter_coef(cr, ij, n_out, n_in)
    y = torch.bmm(dense, xr)
    gy = torch.randn(E, n_out, W, generator=g, dtype=torch.float64)
    gx, gc = torch.autograd.grad((y * gy).sum(), [xr, cr])
    f = lambda t: t.float().to(DEV).contiguous()
    out = rotation.rotate(None, f(x).view(E, n_in * W), ij, f(coef), n_in, W, None, n_out=n_out)
    g_in, g_c = rotation.rotate_bw(None, f(x).view(E, n_in * W), f(gy).view(E, n_out * W), ij,
                                   f(coef), n_in, W, None, n_out=n_out)
    torch.cuda.synchronize()
    mag = torch.bmm(dense.detach().abs(), x.abs())
    assert ((out.cpu().double().view(E, n_out, W) - y.detach()).abs() / (mag + 1e-12)).max() < 1e-5
    gmag = torch.bmm(dense.detach().abs().transpose(1, 2), gy.abs())
    assert ((g_in.cpu().double().view(E, n_in, W) - gx).abs() / (gmag + 1e-12)).max() < 1e-5
    cmag = torch.stack([(gy[:, i].abs() * x[:, j].abs()).sum(1) for i, j in ij], 1)
    assert ((g_c.cpu().double() - gc).abs() / (cmag + 1e-12)).max() < 1e-5
    # deterministic
    out2 = rotation.rotate(None, f(x).view(E, n_in * W), ij, f(coef), n_in, W, None, n_out=n_out)
    assert torch.equal(out, out2)


@pytest.mark.gpu
def test_rotate_rejects_bad_pattern():
    """Pattern entries outside the blocks and coefficient arrays of the wrong width raise
    before any launch, as do patterns beyond the kernels' limits."""
    from tt_atom import rotation
    x = torch.zeros(4, 9 * 8, device=DEV)
    with pytest.raises(RuntimeError, match="outside"):
        rotation.rotate(None, x, [(0, 9)], torch.zeros(4, 1, device=DEV), 9, 8)
    with pytest.raises(RuntimeError, match="coef"):
        rotation.rotate(None, x, [(0, 0)], torch.zeros(4, 2, device=DEV), 9, 8)
    with pytest.raises(RuntimeError, match="unsupported"):
        rotation.rotate(None, torch.zeros(4, 65 * 8, device=DEV), [(0, 0)],
                        torch.zeros(4, 1, device=DEV), 65, 8)


@pytest.mark.gpu
@pytest.mark.parametrize("W", [256, 5])
def test_segment_sum_table(W):
    """scatter.segment_sum over build_gather's table (with the sentinel and a min_width pad)
    against index_add in fp64: a hub, nodes without edges, W = 256 and an odd W = 5."""
    from tt_atom.scatter import build_gather, segment_sum
    g = torch.Generator().manual_seed(W)
    N, E = 300, 5000
    idx = torch.randint(0, N - 10, (E,), generator=g)
    idx[:400] = 17
    msg = torch.randn(E, W, generator=g, dtype=torch.float64)
    ref = torch.zeros(N, W, dtype=torch.float64).index_add_(0, idx, msg)
    mag = torch.zeros(N, W, dtype=torch.float64).index_add_(0, idx, msg.abs())
    flat, D = build_gather(idx, N, E, min_width=450)
    out = segment_sum(None, msg.float().to(DEV), torch.from_numpy(flat), D, N, W)
    torch.cuda.synchronize()
    assert ((out.cpu().double() - ref).abs() / (mag + 1e-12)).max() < 2e-6
    assert (out[N - 10:] == 0).all()
