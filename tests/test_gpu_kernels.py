"""Per-kernel parity on the MI355X: every HIP kernel of the edgewise path against a torch-CPU
(fp64) restatement of the same operation, or against the oracle.  Run with ``-m gpu``."""
import math

import numpy as np
import pytest
import torch

from oracle import geometry as OG

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def nat():
    from tt_atom import _native
    _native.load()
    return _native


def _pack_ij():
    """(m-primed row, natural column) of the 35 packed coefficients, row-major (rotation.py:204-207)."""
    deg = [0, 1, 2, 1, 2, 1, 2, 2, 2]
    cols = {0: [0], 1: [1, 2, 3], 2: [4, 5, 6, 7, 8]}
    return [(m, j) for m in range(9) for j in cols[deg[m]]]


IJ = _pack_ij()


def _dense(coef):
    W = torch.zeros(coef.shape[0], 9, 9, dtype=coef.dtype)
    ii = torch.tensor([i for i, _ in IJ])
    jj = torch.tensor([j for _, j in IJ])
    W[:, ii, jj] = coef
    return W


def _jd():
    from tt_atom.synthetic import jd_matrices
    return jd_matrices()


def _rand_graph(N, E, seed):
    g = torch.Generator().manual_seed(seed)
    tgt = torch.sort(torch.randint(0, N, (E,), generator=g)).values
    src = torch.randint(0, N, (E,), generator=g)
    return src, tgt, g


def _csr(idx, N):
    ptr = torch.zeros(N + 1, dtype=torch.int64)
    ptr[1:] = torch.cumsum(torch.bincount(idx, minlength=N), 0)
    return ptr


def _i32(t):
    return t.to(torch.int32).to(DEV)


# ------------------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("M,N,K,epi", [(256, 128, 128, 0), (300, 96, 40, 0), (37, 20, 9, 0),
                                       (513, 640, 768, 0), (130, 132, 64, 1), (200, 64, 48, 2),
                                       (64, 48, 32, 3), (90, 33, 17, 4)])
def test_gemm_matches_torch(nat, M, N, K, epi):
    g = torch.Generator().manual_seed(M * 7 + N)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g)
    bias = torch.randn(N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    aux = torch.randn(M, N, generator=g)
    ref = (A.double() @ B.double()) + bias.double()
    Cd = C0.clone().to(DEV)
    C2 = torch.zeros(M, N, device=DEV)
    nat.gemm(A.to(DEV), B.to(DEV), Cd, M=M, N=N, K=K, lda=K, ldb=N, ldc=N, bias=bias.to(DEV),
             epilogue=epi, C2=C2, aux=aux.to(DEV))
    torch.cuda.synchronize()
    if epi == 1:
        ref = torch.nn.functional.silu(ref)
    elif epi == 2:
        ref = ref + C0.double()
    elif epi == 4:
        s = torch.sigmoid(aux.double())
        ref = ref * (s * (1 + aux.double() * (1 - s)))
    tol = 2e-5 * math.sqrt(K) * float(ref.abs().max())
    assert (Cd.cpu().double() - ref).abs().max() < tol
    if epi == 3:
        assert (C2.cpu().double() - torch.nn.functional.silu(ref)).abs().max() < tol


@pytest.mark.parametrize("M,N,K", [(72, 1024, 1024), (72, 1024, 256), (576, 256, 1024),
                                   (37, 100, 300), (1, 64, 512)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_gemm_splitk_matches_fp64(nat, M, N, K, epi):
    """Small-grid fp32 products run as k chunks plus an in-order reduction (the linears of small
    systems): fp64 reference at the fp32 kernel's tolerance, every epilogue, K not a multiple of
    the chunk, N and K not multiples of 4 (scalar loads), a single row."""
    g = torch.Generator().manual_seed(M + 3 * N + K)
    A, B = torch.randn(M, K, generator=g), torch.randn(K, N, generator=g)
    bias, C0, aux = torch.randn(N, generator=g), torch.randn(M, N, generator=g), \
        torch.randn(M, N, generator=g)
    probs = (nat.GemmProblem * 1)(nat.GemmProblem(None, None, None, None, None, None, M, N, K,
                                                  K, N, N, epi))
    assert nat.load().tta_gemm_f32_splitk_work(probs, 1) > 0      # this shape takes the split
    Cd, C2 = C0.clone().to(DEV), torch.zeros(M, N, device=DEV)
    nat.linear(A.to(DEV), B.to(DEV), bias.to(DEV), out=Cd, epilogue=epi, out2=C2, aux=aux.to(DEV))
    torch.cuda.synchronize()
    ref = (A.double() @ B.double()) + bias.double()
    if epi == 1:
        ref = torch.nn.functional.silu(ref)
    elif epi == 2:
        ref = ref + C0.double()
    elif epi == 4:
        s = torch.sigmoid(aux.double())
        ref = ref * (s * (1 + aux.double() * (1 - s)))
    tol = 2e-5 * math.sqrt(K) * float(ref.abs().max())
    assert (Cd.cpu().double() - ref).abs().max() < tol
    if epi == 3:
        assert (C2.cpu().double() - torch.nn.functional.silu(ref)).abs().max() < tol


def test_gemm_splitk_group_bits(nat):
    """Split-K launches: a product the rule leaves in one chunk (K = 128) gets the bits of the
    unsplit fp32 kernel, a split product matches its unsplit value to fp32 rounding, and repeated
    launches are bit-identical.  (70 + 50 tiles of 32 x 64: below the 160-tile limit.)"""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(300, 1024, generator=g).to(DEV)
    w1, w2 = torch.randn(1024, 448, generator=g).to(DEV), torch.randn(128, 320, generator=g).to(DEV)
    b2 = torch.randn(320, generator=g).to(DEV)
    o1, o2 = torch.empty(300, 448, device=DEV), torch.empty(300, 320, device=DEV)
    items = [(x, w1, None, o1, nat.EPI_SILU), (x[:, :128], w2, b2, o2, nat.EPI_STORE)]
    probs = (nat.GemmProblem * 2)(*[nat.GemmProblem(None, None, None, None, None, None, 300, w.shape[1],
                                                    a.shape[1], 1024, w.shape[1], w.shape[1], 0)
                                    for a, w, *_ in items])
    assert nat.load().tta_gemm_f32_splitk_work(probs, 2) > 0
    nat.linear_group(items)
    r1, r2 = torch.empty_like(o1), torch.empty_like(o2)
    nat.gemm(x, w1, r1, M=300, N=448, K=1024, lda=1024, ldb=448, ldc=448, epilogue=nat.EPI_SILU)
    nat.gemm(x, w2, r2, M=300, N=320, K=128, lda=1024, ldb=320, ldc=320, bias=b2)
    a1, a2 = torch.empty_like(o1), torch.empty_like(o2)
    nat.linear_group([(x, w1, None, a1, nat.EPI_SILU), (x[:, :128], w2, b2, a2, nat.EPI_STORE)])
    torch.cuda.synchronize()
    assert torch.equal(o2, r2) and torch.equal(o2, a2) and torch.equal(o1, a1)
    assert (o1 - r1).abs().max() < 1e-4 * float(r1.abs().max())


@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_split_gemm_small_splitk(nat, epi):
    """Small-M products of packed (mode 16) weights that would run unsplit on the fp32 kernel at
    its matrix rate take the split kernel's split-K form: 576 x 1024 x 1024 (8 chunks of 128)
    against fp64 at the split kernel's fp32-level accuracy, every epilogue, with rows scaled far
    outside the unscaled window and a row whose values only start in the second chunk, and
    bit-identical on a second call."""
    g = torch.Generator().manual_seed(40 + epi)
    M, N, K = 576, 1024, 1024
    A = torch.randn(M, K, generator=g)
    A[3] *= 2.0 ** 20
    A[4] *= 2.0 ** -30
    A[5, :200] = 0.0
    A[6, 700:] *= 2.0 ** 17
    B = torch.randn(K, N, generator=g) / math.sqrt(K)
    bias, C0, aux = torch.randn(N, generator=g), torch.randn(M, N, generator=g), \
        torch.randn(M, N, generator=g)
    pw = nat.PackedWeight(B.to(DEV), nat.SPLIT_F16X3)
    probs = (nat.GemmProblem * 1)(nat.GemmProblem(None, None, None, None, None, None, M, N, K,
                                                  K, 0, N, epi))
    assert nat.load().tta_gemm_bf16x_splitk_work(probs, 1) > 0
    outs = []
    for _ in range(2):
        Cd, C2 = C0.clone().to(DEV), torch.zeros(M, N, device=DEV)
        nat.linear(A.to(DEV), pw, bias.to(DEV), out=Cd, epilogue=epi, out2=C2, aux=aux.to(DEV))
        torch.cuda.synchronize()
        outs.append((Cd.cpu(), C2.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    ref = (A.double() @ B.double()) + bias.double()
    mag = A.double().abs() @ B.double().abs() + bias.double().abs()
    if epi == 1:
        ref = torch.nn.functional.silu(ref)
    elif epi == 2:
        ref = ref + C0.double()
        mag = mag + C0.double().abs()
    elif epi == 4:
        # the fp32 SiLU derivative itself is good to ~1e-7 absolute, which dominates where
        # silu'(aux) nears its zero
        s = torch.sigmoid(aux.double())
        d = s * (1 + aux.double() * (1 - s))
        ref, mag = ref * d, mag * (d.abs() + 0.05)
    out = outs[0][0].double()
    assert torch.isfinite(out).all()
    assert ((out - ref).abs() / mag).max().item() < 2e-6
    if epi == 3:
        pre = (A.double() @ B.double()) + bias.double()
        assert ((outs[0][1].double() - torch.nn.functional.silu(pre)).abs() / mag).max() < 2e-6


def test_split_gemm_small_splitk_group(nat):
    """An SO(2)-shaped group at 576 edges (the three m-block products, K = 768 / 1024 / 512)
    through linear_group on the split kernel's split-K form, each product against fp64."""
    g = torch.Generator().manual_seed(77)
    M = 576
    shapes = [(768, 640), (1024, 512), (512, 256)]
    xs = [torch.randn(M, K, generator=g) for K, _ in shapes]
    ws = [torch.randn(K, N, generator=g) / math.sqrt(K) for K, N in shapes]
    pws = [nat.PackedWeight(w.to(DEV), nat.SPLIT_F16X3) for w in ws]
    outs = [torch.full((M, N), float("nan"), device=DEV) for _, N in shapes]
    probs = (nat.GemmProblem * 3)(*[nat.GemmProblem(None, None, None, None, None, None, M, N, K,
                                                    K, 0, N, 0) for K, N in shapes])
    assert nat.load().tta_gemm_bf16x_splitk_work(probs, 3) > 0
    nat.linear_group([(x.to(DEV), pw, None, o) for x, pw, o in zip(xs, pws, outs)])
    torch.cuda.synchronize()
    for x, w, o in zip(xs, ws, outs):
        ref = x.double() @ w.double()
        mag = x.double().abs() @ w.double().abs()
        assert ((o.cpu().double() - ref).abs() / mag).max().item() < 2e-6


def test_gemm_batched_strided(nat):
    g = torch.Generator().manual_seed(5)
    N_, C, H = 50, 32, 24
    x = torch.randn(N_, 9, C, generator=g)
    W = torch.randn(9, C, H, generator=g)
    b = torch.randn(9, H, generator=g)
    out = torch.empty(N_, 9, H, device=DEV)
    nat.gemm(x.to(DEV), W.to(DEV), out, bias=b.to(DEV), M=N_, N=H, K=C, lda=9 * C, ldb=H,
             ldc=9 * H, batch=9, sA=C, sB=C * H, sC=H, sBias=H)
    ref = torch.einsum("nic,ich->nih", x.double(), W.double()) + b.double()[None]
    assert (out.cpu().double() - ref).abs().max() < 1e-4


@pytest.mark.parametrize("M,N,K", [(4100, 200, 196), (8192, 640, 768), (5000, 16, 1000),
                                   (40001, 1100, 128), (9000, 300, 36)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("mode", [6, 16])
def test_split_bf16_gemm_fp32_accuracy(nat, M, N, K, epi, mode):
    """Mode 6 (three bf16 planes, six products) and mode 16 (two scaled fp16 planes, three
    products) have the accuracy of an fp32 GEMM: the error relative to |A| |B| stays within the
    fp32 kernel's, on ragged M / N / K tails too, and with thousands of tiles (40001 x 1100:
    313 x 9 tiles of 128 x 128)."""
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g) / math.sqrt(K)
    bias = torch.randn(N, generator=g)
    C0 = torch.randn(M, N, generator=g)
    aux = torch.randn(M, N, generator=g)
    ref = (A.double() @ B.double()) + bias.double()
    scale = A.double().abs() @ B.double().abs() + 1.0
    if epi == 1:
        ref = torch.nn.functional.silu(ref)
    elif epi == 2:
        ref = ref + C0.double()
    elif epi == 4:
        s = torch.sigmoid(aux.double())
        ref = ref * (s * (1 + aux.double() * (1 - s)))
        scale = scale * 1.2
    pw = nat.PackedWeight(B.to(DEV), mode)
    outs = {}
    for name, w in (("split", pw), ("f32", B.to(DEV))):
        Cd = C0.clone().to(DEV)
        C2 = torch.zeros(M, N, device=DEV)
        nat.linear(A.to(DEV), w, bias.to(DEV), out=Cd, epilogue=epi, out2=C2, aux=aux.to(DEV))
        outs[name] = ((Cd.cpu().double() - ref).abs() / scale).max().item(), C2.cpu().double()
    assert outs["split"][0] < max(2.0 * outs["f32"][0], 1e-6), outs
    if epi == 3:
        assert (outs["split"][1] - torch.nn.functional.silu(ref)).abs().max() < 1e-5 * float(
            scale.max())


@pytest.mark.parametrize("mode,tol", [(1, 2e-2), (3, 2e-4), (6, 1e-6), (16, 1e-6)])
def test_split_gemm_persistent_tiles(nat, mode, tol):
    """More tiles than resident blocks: every block of the split kernel walks several tiles
    (70001 x 700 -> 547 x 6 tiles of 128 x 128 over at most two blocks per compute unit), with a
    ragged last row tile and column tile and a K (164) that ends inside a 32-wide slab; plus a
    grouped launch whose two products have different tile counts.  Error relative to |A| |B| as
    the mode's planes allow (bf16: 2^-8; two bf16 planes: 2^-16; fp32-accurate modes 6 / 16)."""
    g = torch.Generator().manual_seed(70 + mode)
    M, N, K = 70001, 700, 164
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g) / math.sqrt(K)
    bias = torch.randn(N, generator=g)
    ref = A.double() @ B.double() + bias.double()
    scale = A.double().abs() @ B.double().abs() + 1.0
    pw = nat.PackedWeight(B.to(DEV), mode)
    out = torch.full((M, N), float("nan"), device=DEV)
    nat.linear(A.to(DEV), pw, bias.to(DEV), out=out)
    err = ((out.cpu().double() - ref).abs() / scale).max().item()
    assert err < tol, err
    # grouped: the same product next to a small one (5000 rows: 40 x 6 tiles)
    out_g = torch.full((M, N), float("nan"), device=DEV)
    small = torch.full((5000, N), float("nan"), device=DEV)
    nat.linear_group([(A.to(DEV), pw, bias.to(DEV), out_g),
                      (A[:5000].to(DEV), pw, None, small)])
    assert torch.equal(out_g, out)
    assert torch.equal(small.cpu(), (out - bias.to(DEV))[:5000].cpu()) or \
        ((small.cpu().double() - (ref - bias.double())[:5000]).abs() / scale[:5000]).max() < tol


@pytest.mark.parametrize("K", [128, 100, 36])
@pytest.mark.parametrize("epi", [0, 1])
def test_split_gemm_short_k_panel(nat, K, epi):
    """Short-K mode-16 products (K <= 128, at least 128 columns, plain or SiLU
    epilogue) run on the panel kernel: a workgroup splits a 128-row panel of A once and sweeps a
    run of column tiles.  K = 128 goes through linear_group as the radial output layer does (two
    products of different widths: 1536 = two runs of twelve 64-column tiles, 1100 = eighteen
    tiles, in runs of twelve and six, with a ragged last one); the K that end inside a 32-wide
    slab through the C entry point.  Ragged rows (20001 = 156 panels of 128 rows + 33 rows), and
    rows whose scale leaves the unscaled window (max 2^20, 2^-12 and 2^-30 times the rest, an
    all-zero row).  Error at fp32 level, each row's against
    its own |A| |B|."""
    g = torch.Generator().manual_seed(K + 7 * epi)
    M1, M2 = 20001, 6000
    A1 = torch.randn(M1, K, generator=g)
    B1 = torch.randn(K, 1536, generator=g) / math.sqrt(K)
    bias1 = torch.randn(1536, generator=g)
    A2 = torch.randn(M2, K, generator=g)
    A2[5] *= 2.0 ** 20
    A2[300] *= 2.0 ** -12
    A2[301] *= 2.0 ** -30
    A2[302] = 0.0
    A2[M2 - 1, : K // 2] *= 1e3
    B2 = torch.randn(K, 1100, generator=g) / math.sqrt(K)
    pw1, pw2 = nat.PackedWeight(B1.to(DEV), 16), nat.PackedWeight(B2.to(DEV), 16)
    o1 = torch.full((M1, 1536), float("nan"), device=DEV)
    o2 = torch.full((M2, 1100), float("nan"), device=DEV)
    if K == 128:
        nat.linear_group([(A1.to(DEV), pw1, bias1.to(DEV), o1, epi),
                          (A2.to(DEV), pw2, None, o2, epi)])
    else:
        nat._gemm_bf16x(A1.to(DEV), pw1, o1, bias1.to(DEV), epi, None, None)
        nat._gemm_bf16x(A2.to(DEV), pw2, o2, None, epi, None, None)
    for A, B, bias, o in ((A1, B1, bias1, o1), (A2, B2, None, o2)):
        ref = A.double() @ B.double()
        mag = A.double().abs() @ B.double().abs()
        if bias is not None:
            ref = ref + bias.double()
            mag = mag + bias.double().abs()
        if epi == 1:
            ref = torch.nn.functional.silu(ref)
        out = o.cpu().double()
        assert torch.isfinite(out).all()
        err = (out - ref).abs() / mag.clamp_min(1e-300)
        err[mag == 0] = (out - ref).abs()[mag == 0]
        assert err.max().item() < 2e-6, (err.max(dim=1).values.argmax().item(), err.max().item())


def test_split_bf16_gemm_modes_and_gather(nat):
    g = torch.Generator().manual_seed(3)
    M, N, K, Nn = 6000, 256, 512, 300
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g) / math.sqrt(K)
    P = torch.randn(Nn, 2 * N, generator=g)
    i0 = torch.randint(Nn, (M,), generator=g)
    i1 = torch.randint(Nn, (M,), generator=g)
    ref = A.double() @ B.double() + P.double()[i0, :N] + P.double()[i1, N:]
    scale = (A.double().abs() @ B.double().abs()).max().item()
    errs = {}
    for mode in (nat.SPLIT_F32, nat.SPLIT_F16X3, nat.SPLIT_3, nat.SPLIT_BF16):
        pw = nat.PackedWeight(B.to(DEV), mode)
        out = torch.empty(M, N, device=DEV)
        nat.linear_gather(A.to(DEV), pw, None, out, P.to(DEV), _i32(i0), _i32(i1), N)
        errs[mode] = (out.cpu().double() - ref).abs().max().item() / scale
    # bf16 operands: ~2^-8 relative; two planes: ~2^-16; three planes: fp32 level
    assert errs[nat.SPLIT_BF16] < 2e-2 and errs[nat.SPLIT_3] < 2e-5 and errs[nat.SPLIT_F32] < 2e-6, errs
    assert errs[nat.SPLIT_F16X3] < 2e-6, errs
    assert max(errs[nat.SPLIT_F32], errs[nat.SPLIT_F16X3]) < errs[nat.SPLIT_3] < errs[nat.SPLIT_BF16]


def _scaling_cases():
    g = torch.Generator().manual_seed(11)
    M, K, N = 3000, 520, 300
    rn = lambda *s: torch.randn(*s, generator=g)
    ru = lambda *s: torch.rand(*s, generator=g)
    grow = 2.0 ** (torch.arange(K) / 16.0)
    spikes = rn(M, K)
    spikes[::7] = 0                      # all-zero rows
    spikes[1::7, :300] = 0               # rows whose first nonzero values come late
    spikes[2::7, 17] = 1e6               # one huge value per row
    colsc = rn(K, N) * 10.0 ** (ru(1, N) * 40 - 20)
    colsc[:, 5] = 0                      # an all-zero column
    return {
        "row scales 1e-30..1e30": (rn(M, K) * 10.0 ** (ru(M, 1) * 60 - 30), rn(K, N)),
        "element scales 1e-4..1e2": (rn(M, K) * 10.0 ** (ru(M, K) * 6 - 4), rn(K, N)),
        "growing along K": (rn(M, K) * grow, rn(K, N)),
        "shrinking along K": (rn(M, K) / grow, rn(K, N)),
        "zero rows and columns, spikes, column scales": (spikes, colsc),
        "fp32 subnormal rows": (rn(M, K) * 1e-40, rn(K, N)),
        "rows near 1e35": (rn(M, K) * 1e35, rn(K, N) / math.sqrt(K)),
    }


@pytest.mark.parametrize("case", list(_scaling_cases()))
def test_split_f16_scaling(nat, case):
    """Mode 16's power-of-two scales (per B column at packing, per A row tracked along K with
    accumulator rescaling) keep fp32 accuracy over fp32's whole range: rows and columns of very
    different magnitude, values that grow or shrink along K (rescales), all-zero rows and
    columns, rows whose first nonzero value comes late, isolated huge values, fp32 subnormals."""
    A, B = _scaling_cases()[case]
    M, N = A.shape[0], B.shape[1]
    ref = A.double() @ B.double()
    scale = A.double().abs() @ B.double().abs()
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    errs = {}
    for name, w in (("f16x3", nat.PackedWeight(B.to(DEV), nat.SPLIT_F16X3)), ("f32", B.to(DEV))):
        out = torch.empty(M, N, device=DEV)
        nat.linear(A.to(DEV), w, out=out)
        o = out.cpu().double()
        assert bool(torch.isfinite(o).all()), (case, name)
        errs[name] = ((o - ref).abs() / scale).max().item()
    assert errs["f16x3"] <= max(2.0 * errs["f32"], 1e-6), (case, errs)


@pytest.mark.parametrize("case", ["grows past 2^15", "late first values", "tiny late values"])
def test_split_f16_fast_loop_retry(nat, case):
    """K a multiple of 32: waves whose rows are all unscaled run the fast loop, whose slab check
    only branches out for a scale event (a row passing 2^15, or a row's first nonzero slab).  A
    row planted into one tile of a normal matrix -- values that pass 2^15 from k = 256 on, a row
    that is zero for its first slab, or one whose late values are tiny -- must leave every other
    row bit-identical to the run without it (the event rescales only its own row), and be
    accurate itself."""
    g = torch.Generator().manual_seed(5)
    M, K, N = 1000, 512, 384                 # the split kernel through its C entry point
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g) / math.sqrt(K)
    pw = nat.PackedWeight(B.to(DEV), nat.SPLIT_F16X3)
    r = 300                                  # a row inside the third 128-row tile
    A2 = A.clone()
    if case == "grows past 2^15":
        A2[r, 256:] *= 2.0 ** 17
    elif case == "late first values":
        A2[r, :32] = 0.0
    else:
        A2[r, :64] = 0.0
        A2[r, 64:] *= 2.0 ** -20
    outs = []
    for a in (A, A2):
        out = torch.empty(M, N, device=DEV)
        nat._gemm_bf16x(a.to(DEV), pw, out, None, nat.EPI_STORE, None, None)
        outs.append(out.cpu())
    others = torch.ones(M, dtype=torch.bool)
    others[r] = False
    assert torch.equal(outs[0][others], outs[1][others])
    ref = A2[r].double() @ B.double()
    mag = A2[r].double().abs() @ B.double().abs()
    assert ((outs[1][r].double() - ref).abs() / mag).max().item() < 2e-6


# ------------------------------------------------------------------------------ geometry
def _oracle_wig(ev, jd):
    eul = OG.euler_angles(ev)
    wig = OG.eulers_to_wigner(eul, 2, [j.to(ev.dtype) for j in jd])
    perm = torch.tensor([0, 2, 6, 3, 7, 1, 5, 8, 4])
    return wig.index_select(1, perm)


def _test_vectors(n, seed):
    g = torch.Generator().manual_seed(seed)
    ev = torch.randn(n, 3, generator=g) * 2.0
    # directions at and near the poles of the edge frame (the +-y axis) and along x / z
    special = torch.tensor([[0.0, 1.0, 0.0], [0.0, -2.0, 0.0], [1e-4, 1.0, 0.0], [0.0, 1.0, 1e-5],
                            [3.0, 0.0, 0.0], [0.0, 0.0, -1.5], [1.0, 1.0, 1.0], [-1e-3, -3.0, 2e-3]])
    return torch.cat([ev, special], 0)


def test_edge_wigner_matches_oracle(nat):
    jd = _jd()
    ev = _test_vectors(500, 0)
    E = ev.shape[0]
    pos = torch.cat([ev, torch.zeros(1, 3)], 0)                    # ev = pos[e] - pos[E]
    src = torch.arange(E)
    tgt = torch.full((E,), E)
    jdf = torch.cat([j.reshape(-1) for j in jd]).to(DEV)
    evd, dist, coef = (torch.empty(E, 3, device=DEV), torch.empty(E, device=DEV),
                       torch.empty(E, 35, device=DEV))
    nat.edge_wigner(pos.to(DEV), _i32(src), _i32(tgt), None, jdf, 0.0, evd, dist, coef)
    torch.cuda.synchronize()
    ref = _oracle_wig(ev.double(), jd)
    ref_c = torch.stack([ref[:, i, j] for i, j in IJ], 1)
    # fp64 for the generic directions; near the pole fp32 acos itself limits the accuracy
    assert (coef.cpu().double() - ref_c)[:-8].abs().max() < 2e-6
    assert (dist.cpu().double() - ev.double().norm(dim=1)).abs().max() < 1e-5
    # the same through the fp32 oracle (what the parity tests compare against)
    g32 = _oracle_wig(ev, [j.float() for j in jd])
    assert (coef.cpu() - torch.stack([g32[:, i, j] for i, j in IJ], 1)).abs().max() < 2e-6


@pytest.mark.parametrize("nb,ec", [(32, 8), (30, 6)])
def test_edge_features_matches_oracle(nat, nb, ec):
    """Gaussian basis, species embeddings and envelope; (32, 8) runs the float4 wavefront-per-edge
    kernel, (30, 6) the element-per-thread one."""
    g = torch.Generator().manual_seed(3)
    E = 400
    dist = torch.rand(E, generator=g) * 6.5 + 0.2
    zs, zt = torch.randint(0, 10, (E,), generator=g), torch.randint(0, 10, (E,), generator=g)
    semb, temb = torch.randn(10, ec, generator=g), torch.randn(10, ec, generator=g)
    off = torch.linspace(0, 6.0, nb)
    coeff = -0.5 / float(2 * (off[1] - off[0])) ** 2
    xe, env = torch.empty(E, nb + 2 * ec, device=DEV), torch.empty(E, device=DEV)
    nat.edge_features(dist.to(DEV), _i32(zs), _i32(zt), semb.to(DEV), temb.to(DEV), off.to(DEV),
                      coeff, 6.0, nb, ec, xe, env)
    torch.cuda.synchronize()
    gauss = torch.exp(coeff * (dist.view(-1, 1) - off.view(1, -1)) ** 2)
    ref = torch.cat([gauss, semb[zs], temb[zt]], 1)
    assert (xe.cpu() - ref).abs().max() < 1e-5
    ds = dist / 6.0
    ev_ = 1 + ds ** 5 * (-21 + ds * (35 - 15 * ds))
    ref_env = torch.where(ds < 1, ev_, torch.zeros_like(ev_))
    assert (env.cpu() - ref_env).abs().max() < 1e-5


@pytest.mark.parametrize("E,nb,ec,periodic", [(1000, 32, 8, False), (130, 512, 128, True),
                                              (64, 16, 0, False), (77, 30, 6, True)])
def test_edge_geometry_fwd_equals_two_passes(nat, E, nb, ec, periodic):
    """The one-launch forward geometry equals tta_edge_wigner + tta_edge_features bit for bit:
    blocks of 64 edges with a partial last block (1000, 130, 77), the C3 row width (512 + 2 x 128),
    no species embedding (ec = 0), and rows that take the two-kernel route (30, 6)."""
    g = torch.Generator().manual_seed(11)
    N = 50
    pos = (torch.rand(N, 3, generator=g) * 8.0).to(DEV)
    src, tgt = torch.randint(0, N, (E,), generator=g), torch.randint(0, N, (E,), generator=g)
    tgt = torch.where(tgt == src, (tgt + 1) % N, tgt)
    shift = (torch.randint(-1, 2, (E, 3), generator=g).float() * 8.0).to(DEV) if periodic else None
    zs, zt = torch.randint(0, 10, (E,), generator=g), torch.randint(0, 10, (E,), generator=g)
    semb = torch.randn(10, ec, generator=g).to(DEV) if ec else None
    temb = torch.randn(10, ec, generator=g).to(DEV) if ec else None
    off = torch.linspace(0, 6.0, nb).to(DEV)
    coeff = -0.5 / float(2 * (off[1] - off[0])) ** 2
    jdf = torch.cat([j.reshape(-1) for j in _jd()]).to(DEV)

    def outs():
        return (torch.full((E, 3), 7.0, device=DEV), torch.full((E,), 7.0, device=DEV),
                torch.full((E, 35), 7.0, device=DEV), torch.full((E, nb + 2 * ec), 7.0, device=DEV),
                torch.full((E,), 7.0, device=DEV))

    a, b = outs(), outs()
    args = (_i32(src), _i32(tgt), shift, jdf, 0.3)
    nat.edge_wigner(pos, *args, a[0], a[1], a[2])
    nat.edge_features(a[1], _i32(zs), _i32(zt), semb, temb, off, coeff, 6.0, nb, ec, a[3], a[4])
    nat.edge_geometry_fwd(pos, *args, _i32(zs), _i32(zt), semb, temb, off, coeff, 6.0, nb, ec,
                          *b)
    torch.cuda.synchronize()
    for name, x, y in zip(("ev", "dist", "coef", "x_edge", "env"), a, b):
        assert torch.equal(x, y), name


def test_geometry_vjp_matches_autograd(nat):
    jd = _jd()
    ev = _test_vectors(400, 1)
    E = ev.shape[0]
    nb, cutoff = 16, 6.0
    off = torch.linspace(0, cutoff, nb, dtype=torch.float64)
    coeff = -0.5 / float(2 * (off[1] - off[0])) ** 2
    g = torch.Generator().manual_seed(11)
    g_coef = torch.randn(E, 35, generator=g)
    g_env = torch.randn(E, generator=g)
    g_gauss = torch.randn(E, nb, generator=g)
    # autograd reference in fp64 through the oracle's functions
    e64 = ev.double().clone().requires_grad_(True)
    wig = _oracle_wig(e64, jd)
    coef = torch.stack([wig[:, i, j] for i, j in IJ], 1)
    d = torch.linalg.norm(e64, dim=1)
    gauss = torch.exp(coeff * (d.view(-1, 1) - off.view(1, -1)) ** 2)
    ds = d / cutoff
    envv = torch.where(ds < 1, 1 + ds ** 5 * (-21 + ds * (35 - 15 * ds)), torch.zeros_like(ds))
    loss = (coef * g_coef.double()).sum() + (envv * g_env.double()).sum() + \
           (gauss * g_gauss.double()).sum()
    (ref,) = torch.autograd.grad(loss, e64)
    out = torch.empty(E, 3, device=DEV)
    jdf = torch.cat([j.reshape(-1) for j in jd]).to(DEV)
    nat.edge_geometry_bwd(ev.to(DEV), ev.norm(dim=1).to(DEV), g_coef.to(DEV), g_env.to(DEV),
                          g_gauss.to(DEV), nb, off.float().to(DEV), coeff, cutoff, nb, jdf, 0.0, out)
    torch.cuda.synchronize()
    err = (out.cpu().double() - ref).abs()
    scale = ref.abs().clamp(min=1.0)
    # exactly-on-pole vectors hit the EPS regularisation: compare those with a looser bound
    assert (err[:-8] / scale[:-8]).max() < 5e-4
    assert torch.isfinite(out).all()


# ------------------------------------------------------------------------------ rotation
@pytest.mark.parametrize("C", [16, 32, 128])
def test_gather_rotate_fwd_bwd(nat, C):
    N, E = 40, 300
    src, tgt, g = _rand_graph(N, E, C)
    x = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    coef = torch.randn(E, 35, generator=g, dtype=torch.float64)
    rad = torch.randn(E, 6, 2 * C, generator=g, dtype=torch.float64)
    rb = [0, 1, 2, 3, 4, 3, 4, 5, 5]
    xr, cr, rr = (t.clone().requires_grad_(True) for t in (x, coef, rad))
    m = torch.bmm(_dense(cr), torch.cat([xr[src], xr[tgt]], 2)) * rr[:, rb, :]
    gout = torch.randn(E, 9, 2 * C, generator=g, dtype=torch.float64)
    gx, gc, grd = torch.autograd.grad((m * gout).sum(), [xr, cr, rr])
    out = torch.empty(E, 9, 2 * C, device=DEV)
    f = lambda t: t.float().to(DEV).contiguous()
    nat.gather_rotate(f(x), _i32(src), _i32(tgt), f(coef), f(rad), out)
    g_rad, g_mcat = torch.empty(E, 6, 2 * C, device=DEV), torch.empty(E, 9, 2 * C, device=DEV)
    g_coef = torch.zeros(E, 35, device=DEV)
    nat.gather_rotate_bw(f(gout), f(rad), f(x), _i32(src), _i32(tgt), f(coef), g_rad, g_mcat, g_coef)
    # node adjoint via the src / tgt CSR sum
    sptr, perm = _csr(src, N), torch.argsort(src, stable=True)
    tptr = _csr(tgt, N)
    gn = torch.empty(N, 9, C, device=DEV)
    nat.node_gather_sum(g_mcat, _i32(sptr), _i32(perm), _i32(tptr), None, gn)
    torch.cuda.synchronize()
    assert (out.cpu().double() - m.detach()).abs().max() < 1e-4
    assert (g_rad.cpu().double() - grd).abs().max() < 1e-4
    assert (g_coef.cpu().double() - gc).abs().max() < 1e-3
    assert (gn.cpu().double() - gx).abs().max() < 1e-3


@pytest.mark.parametrize("C", [16, 32, 64, 128, 256])
def test_gather_rotate_bw_dst_bit_equal(nat, C):
    """The destination-walked backward (a block per node, the destination half of the adjoint
    summed in registers) gives the same bits as the edge-walked kernel followed by the CSR node
    sum for g_rad, the source half of g_mcat and the node adjoint (with a residual), and the
    accumulated g_coef to fp32 rounding (its channel sum runs per half, then adds the halves);
    the walk from both ends of every edge (source walk, then destination walk, no g_mcat) gives
    the destination walk's bits for g_rad and the node adjoint and its g_coef to fp32 rounding.
    A graph with a destination hub, nodes without incoming edges and isolated nodes."""
    N, E = 60, 700
    g = torch.Generator().manual_seed(C + 7)
    tgt = torch.randint(0, N - 6, (E,), generator=g)
    tgt[:200] = 5                                           # destination hub
    tgt = torch.sort(tgt).values                            # edges sorted by destination
    src = torch.randint(0, N - 3, (E,), generator=g)        # nodes N-3.. isolated
    x = torch.randn(N, 9, C, generator=g)
    coef = torch.randn(E, 35, generator=g)
    rad = torch.randn(E, 6, 2 * C, generator=g)
    gout = torch.randn(E, 9, 2 * C, generator=g)
    gc0 = torch.randn(E, 35, generator=g)                   # g_coef is accumulated into
    f = lambda t: t.to(DEV).contiguous()
    sptr, perm, tptr = _csr(src, N), torch.argsort(src, stable=True), _csr(tgt, N)
    outs = {}
    res = torch.randn(N, 9, C, generator=g)
    for walk in ("edge", "dst", "nodes"):
        g_rad = torch.full((E, 6, 2 * C), float("nan"), device=DEV)
        g_mcat = torch.zeros(E, 9, 2 * C, device=DEV)
        g_coef = f(gc0.clone())
        gn = torch.full((N, 9, C), float("nan"), device=DEV)
        if walk == "edge":
            nat.gather_rotate_bw(f(gout), f(rad), f(x), _i32(src), _i32(tgt), f(coef), g_rad,
                                 g_mcat, g_coef)
            nat.node_gather_sum(g_mcat, _i32(sptr), _i32(perm), _i32(tptr), f(res), gn)
        elif walk == "dst":
            tsum = torch.full((N, 9, C), float("nan"), device=DEV)
            nat.gather_rotate_bw_dst(f(gout), f(rad), f(x), _i32(src), _i32(tptr), f(coef), g_rad,
                                     g_mcat, g_coef, tsum)
            nat.node_gather_sum_dst(g_mcat, _i32(sptr), _i32(perm), tsum, f(res), gn)
        else:
            ssum = torch.full((N, 9, C), float("nan"), device=DEV)
            half = torch.full((E, 35), float("nan"), device=DEV)
            nat.gather_rotate_bw_nodes(f(gout), f(rad), f(x), _i32(sptr), _i32(perm), _i32(tptr),
                                       f(coef), g_rad, g_coef, half, ssum, f(res), gn)
        torch.cuda.synchronize()
        outs[walk] = (g_rad.cpu(), gn.cpu(), g_coef.cpu(), g_mcat.cpu()[:, :, :C])
    for a, b in zip(outs["edge"][:2], outs["dst"][:2]):
        assert torch.equal(a, b)
    assert torch.equal(outs["edge"][3], outs["dst"][3])        # the source half of g_mcat
    ga, gb = outs["edge"][2].double(), outs["dst"][2].double()
    assert ((ga - gb).abs() / (ga.abs() + 1.0)).max() < 1e-5
    # the walk from both ends: the bits of the destination walk for g_rad and the node adjoint;
    # g_coef to fp32 rounding (its channel sums reduce across lanes in another order)
    for a, b in zip(outs["dst"][:2], outs["nodes"][:2]):
        assert torch.equal(a, b)
    gn_ = outs["nodes"][2].double()
    assert ((gb - gn_).abs() / (gb.abs() + 1.0)).max() < 1e-5


@pytest.mark.parametrize("C", [16, 128, 256, 1024])
def test_node_gather_sum_order_and_hubs(nat, C):
    """Every node's sum is bit-equal to a plain fp32 loop in edge order (src edges in the
    src-sorted order, then tgt edges, then src + tgt + res): hubs with more than 64 src and tgt
    edges, isolated nodes and degrees that are not multiples of the unroll."""
    N = 24
    g = torch.Generator().manual_seed(C)
    src = torch.randint(0, N, (400,), generator=g)
    src[:150] = 3                                                  # src hub
    tgt = torch.randint(0, N, (400,), generator=g)
    tgt[150:230] = 5                                               # tgt hub
    tgt[(src == 7) | (tgt == 7)] = 8
    src[src == 7] = 9                                              # node 7 has no edges
    tgt = torch.sort(tgt).values
    E = src.numel()
    gm = torch.randn(E, 9, 2 * C, generator=g).float()
    res = torch.randn(N, 9, C, generator=g).float()
    perm = torch.argsort(src, stable=True)
    sptr, tptr = _csr(src, N), _csr(tgt, N)
    gmn = gm.numpy()
    want = np.empty((N, 9, C), np.float32)
    for n in range(N):
        a = np.zeros((9, C), np.float32)
        for k in range(int(sptr[n]), int(sptr[n + 1])):
            a = a + gmn[int(perm[k]), :, :C]
        b = np.zeros((9, C), np.float32)
        for e in range(int(tptr[n]), int(tptr[n + 1])):
            b = b + gmn[e, :, C:]
        want[n] = (a + b) + res[n].numpy()
    out = torch.empty(N, 9, C, device=DEV)
    nat.node_gather_sum(gm.to(DEV), _i32(sptr), _i32(perm), _i32(tptr), res.to(DEV), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)
    assert int(sptr[8] - sptr[7]) == 0 and int(tptr[8] - tptr[7]) == 0


@pytest.mark.parametrize("n_in,env_first", [(9, True), (3, False)])
def test_rotate_env_segsum_fwd_bwd(nat, n_in, env_first):
    N, E, C = 30, 250, 32
    src, tgt, g = _rand_graph(N, E, 7 + n_in)
    m = torch.randn(E, n_in, C, generator=g, dtype=torch.float64)
    coef = torch.randn(E, 35, generator=g, dtype=torch.float64)
    env = torch.rand(E, generator=g, dtype=torch.float64)
    res = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    div = 1.0 if env_first else 5.0
    mr, cr, er = (t.clone().requires_grad_(True) for t in (m, coef, env))
    mp = torch.nn.functional.pad(mr, (0, 0, 0, 9 - n_in))
    Wt = _dense(cr).transpose(1, 2)
    if env_first:
        v = torch.bmm(Wt, mp * er.view(-1, 1, 1))
    else:
        v = torch.bmm(Wt, mp) * er.view(-1, 1, 1) / div
    out_ref = torch.zeros(N, 9, C, dtype=torch.float64).index_add(0, tgt, v) + res
    gnode = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    gm, gc, ge = torch.autograd.grad((out_ref * gnode).sum(), [mr, cr, er])
    f = lambda t: t.float().to(DEV).contiguous()
    out = torch.empty(N, 9, C, device=DEV)
    nat.rotate_env_segsum(f(m), f(coef), f(env), _i32(_csr(tgt, N)), f(res), out, n_in=n_in,
                          env_first=env_first, div=div)
    g_m = torch.empty(E, n_in, C, device=DEV)
    g_coef, g_env = torch.zeros(E, 35, device=DEV), torch.zeros(E, device=DEV)
    nat.rotate_env_segsum_bw(f(gnode), _i32(tgt), f(m), f(coef), f(env), g_m, g_coef, g_env,
                             n_in=n_in, env_first=env_first, div=div)
    torch.cuda.synchronize()
    assert (out.cpu().double() - out_ref.detach()).abs().max() < 1e-4
    assert (g_m.cpu().double() - gm).abs().max() < 1e-4
    assert (g_env.cpu().double() - ge).abs().max() < 1e-3
    if n_in == 3:   # only coefficients with m-primed row < 3 receive an adjoint
        rows = torch.tensor([i for i, _ in IJ])
        gc = gc * (rows < 3).double()
    assert (g_coef.cpu().double() - gc).abs().max() < 1e-3


# ------------------------------------------------------------------------------ row-wise
@pytest.mark.parametrize("natural", [False, True])
def test_gate_fwd_bwd(nat, natural):
    R, H = 200, 48
    idx = (0, 0, 0, 1, 1, 1, 1, 1) if natural else (0, 1, 0, 1, 0, 1, 1, 1)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(R, 9, H, generator=g, dtype=torch.float64)
    gat = torch.randn(R, 2 * H, generator=g, dtype=torch.float64)
    xr, gr = x.clone().requires_grad_(True), gat.clone().requires_grad_(True)
    sg = torch.sigmoid(gr).view(R, 2, H)[:, list(idx), :]
    y = torch.cat([torch.nn.functional.silu(xr[:, :1]), xr[:, 1:] * sg], 1)
    gy = torch.randn(R, 9, H, generator=g, dtype=torch.float64)
    gx, gg = torch.autograd.grad((y * gy).sum(), [xr, gr])
    f = lambda t: t.float().to(DEV).contiguous()
    idx_t = torch.tensor(idx, dtype=torch.int32, device=DEV)
    yo = torch.empty(R, 9, H, device=DEV)
    nat.gate_fwd(f(x), f(gat), yo, idx_t, R=R, H=H, L=2)
    gxo, ggo = torch.empty(R, 9, H, device=DEV), torch.empty(R, 2 * H, device=DEV)
    nat.gate_bwd(f(gy), f(x), f(gat), gxo, ggo, idx_t, R=R, H=H, L=2)
    torch.cuda.synchronize()
    assert (yo.cpu().double() - y.detach()).abs().max() < 1e-5
    assert (gxo.cpu().double() - gx).abs().max() < 1e-5
    assert (ggo.cpu().double() - gg).abs().max() < 1e-5
    # the combined row layout [gating | x] of the conv-1 GEMM output (row stride 11 H)
    comb = torch.cat([gat, x.reshape(R, 9 * H)], 1).float().to(DEV).contiguous()
    yo2 = torch.empty(R, 9, H, device=DEV)
    nat.gate_fwd(comb[:, 2 * H:], comb, yo2, idx_t, R=R, H=H, L=2, ldx=11 * H, ldg=11 * H)
    gcomb = torch.zeros(R, 11 * H, device=DEV)
    nat.gate_bwd(f(gy), comb[:, 2 * H:], comb, gcomb[:, 2 * H:], gcomb, idx_t, R=R, H=H, L=2,
                 ldx=11 * H, ldg=11 * H)
    torch.cuda.synchronize()
    assert torch.equal(yo2, yo)
    assert torch.equal(gcomb[:, 2 * H:].reshape(R, 9, H), gxo) and torch.equal(gcomb[:, :2 * H], ggo)


def _conv1_case(M, H, cin, seed):
    """Operands of an SO(2) conv-1 at channel width cin: x rows of the three m-blocks (3, 4 and 2
    coefficients of 2 cin), the m = 0 weight [3 cin, 2 H + 3 H] with its gating columns first,
    the m = 1 and m = 2 weights, the m = 0 bias."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, 9 * 2 * cin, generator=g)
    x[5] *= 2.0 ** 18                      # a row far outside the unscaled window
    wm0 = torch.randn(3 * 2 * cin, 5 * H, generator=g) / math.sqrt(6 * cin)
    w1 = torch.randn(4 * 2 * cin, 4 * H, generator=g) / math.sqrt(8 * cin)
    w2 = torch.randn(2 * 2 * cin, 2 * H, generator=g) / math.sqrt(4 * cin)
    bm0 = torch.randn(5 * H, generator=g)
    return x, wm0, w1, w2, bm0


@pytest.mark.parametrize("mode,M", [(16, 5000), (1, 5000), (16, 700)])
def test_gemm_gate_epilogue(nat, mode, M):
    """The gate applied in the SO(2) conv-1 products' epilogue (tta_gemm_bf16x_group_gate, m-primed
    gate table, H = 48 so that 128-column tiles straddle coefficients) after the gating columns'
    sigmoid epilogue: at M = 5000 (direct launches, ragged last row tile) the gated rows and
    coefficient 0's pre-activation equal the ungated launch followed by tta_gate_fwd bit for bit,
    the sigmoids match; at M = 700 (split-K, the gate applied in the reduction) all of them match
    fp64 at fp32-GEMM accuracy."""
    H, cin, L = 48, 32, 2
    x, wm0, w1, w2, bm0 = _conv1_case(M, H, cin, 60 + mode + M)
    idx = (0, 1, 0, 1, 0, 1, 1, 1)
    P = lambda w: nat.PackedWeight(w.to(DEV).contiguous(), mode)
    xd = x.to(DEV)
    k0, k1 = 3 * 2 * cin, 7 * 2 * cin
    # fused: the gating sigmoids, then the gated coefficient products
    sig = torch.empty(M, L * H, device=DEV)
    y = torch.full((M, 9 * H), float("nan"), device=DEV)
    x0 = torch.full((M, H), float("nan"), device=DEV)
    nat.linear(xd[:, :k0], P(wm0[:, :L * H]), bm0[:L * H].to(DEV), out=sig,
               epilogue=nat.EPI_SIGMOID)
    nat.linear_group_gate([(xd[:, :k0], P(wm0[:, L * H:]), bm0[L * H:].to(DEV), y[:, :3 * H]),
                           (xd[:, k0:k1], P(w1), None, y[:, 3 * H:7 * H]),
                           (xd[:, k1:], P(w2), None, y[:, 7 * H:])], (0, 3, 7), sig, x0, idx, H)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(x0).all()
    if M >= 4096:
        o1 = torch.empty(M, L * H + 9 * H, device=DEV)
        nat.linear_group([(xd[:, :k0], P(wm0), bm0.to(DEV), o1[:, :L * H + 3 * H]),
                          (xd[:, k0:k1], P(w1), None, o1[:, L * H + 3 * H:L * H + 7 * H]),
                          (xd[:, k1:], P(w2), None, o1[:, L * H + 7 * H:])])
        yr = torch.empty(M, 9, H, device=DEV)
        nat.gate_fwd(o1[:, L * H:], o1, yr, idx, R=M, H=H, L=L, ldx=L * H + 9 * H,
                     ldg=L * H + 9 * H)
        torch.cuda.synchronize()
        assert (sig.cpu().double() - torch.sigmoid(o1[:, :L * H].cpu().double())).abs().max() < 3e-7
        assert torch.equal(x0, o1[:, L * H:L * H + H])
        assert torch.equal(y, yr.view(M, 9 * H))
        return
    xd64 = x.double()
    pre = torch.cat([xd64[:, :k0] @ wm0.double() + bm0.double(), xd64[:, k0:k1] @ w1.double(),
                     xd64[:, k1:] @ w2.double()], 1)
    mag = torch.cat([xd64[:, :k0].abs() @ wm0.double().abs() + bm0.double().abs(),
                     xd64[:, k0:k1].abs() @ w1.double().abs(),
                     xd64[:, k1:].abs() @ w2.double().abs()], 1)
    gpre, cpre = pre[:, :L * H], pre[:, L * H:].view(M, 9, H)
    sg = torch.sigmoid(gpre).view(M, L, H)[:, list(idx), :]
    yref = torch.cat([torch.nn.functional.silu(cpre[:, :1]), cpre[:, 1:] * sg], 1)
    cmag = mag[:, L * H:].view(M, 9, H)
    # sigmoid' <= 1/4: the sigmoid's error is at most a quarter of its argument's
    assert ((sig.cpu().double() - torch.sigmoid(gpre)).abs() / mag[:, :L * H]).max() < 2e-6
    assert ((x0.cpu().double() - cpre[:, 0]).abs() / cmag[:, 0]).max() < 2e-6
    assert ((y.cpu().double().view(M, 9, H) - yref).abs() / cmag).max() < 4e-6


@pytest.mark.parametrize("M", [5000, 700])
def test_gemm_gate_bwd_epilogue(nat, M):
    """The SO(2) conv-2 adjoint products with the gate's input adjoint applied in their epilogue
    (tta_gemm_bf16x_group_gate_bwd) and the gating adjoint from them (tta_gate_gating_bwd), on
    strided views of one [gating | coefficients] adjoint row: at M = 5000 the coefficient
    adjoints equal the plain products followed by tta_gate_bwd bit for bit (the sigmoids come
    from the GEMM's sigmoid epilogue on the same gating pre-activations) and the gating adjoint
    matches it to fp32 rounding; at M = 700 (split-K) both match fp64."""
    H, C, L = 48, 64, 2                                # K = 192, 256, 128: all on the split kernel
    idx = (0, 1, 0, 1, 0, 1, 1, 1)
    g = torch.Generator().manual_seed(90 + M)
    gm = torch.randn(M, 9 * C, generator=g)
    gm[7] *= 2.0 ** -20
    W0 = torch.randn(3 * C, 3 * H, generator=g) / math.sqrt(3 * C)
    W1 = torch.randn(4 * C, 4 * H, generator=g) / math.sqrt(4 * C)
    W2 = torch.randn(2 * C, 2 * H, generator=g) / math.sqrt(2 * C)
    x = torch.randn(M, 9, H, generator=g)
    gx_in = torch.randn(M, 64, generator=g)            # gating pre-activations = gx_in @ Wg + bg
    Wg = torch.randn(64, L * H, generator=g) / 4.0
    bg = torch.randn(L * H, generator=g)
    P = lambda w: nat.PackedWeight(w.to(DEV).contiguous(), nat.SPLIT_F16X3)
    Pg = P(Wg)
    gat = torch.empty(M, L * H, device=DEV)
    sig = torch.empty(M, L * H, device=DEV)
    nat.linear(gx_in.to(DEV), Pg, bg.to(DEV), out=gat)
    nat.linear(gx_in.to(DEV), Pg, bg.to(DEV), out=sig, epilogue=nat.EPI_SIGMOID)
    xd = x.to(DEV)
    y = torch.empty(M, 9, H, device=DEV)
    nat.gate_fwd(xd, gat, y, idx, R=M, H=H, L=L)
    x0 = xd[:, 0].contiguous()
    gmd = gm.to(DEV)
    LHc = L * H + 9 * H
    g1 = torch.full((M, LHc), float("nan"), device=DEV)
    nat.linear_group_gate([(gmd[:, :3 * C], P(W0), None, g1[:, L * H:L * H + 3 * H]),
                           (gmd[:, 3 * C:7 * C], P(W1), None, g1[:, L * H + 3 * H:L * H + 7 * H]),
                           (gmd[:, 7 * C:], P(W2), None, g1[:, L * H + 7 * H:])],
                          (0, 3, 7), sig, x0, idx, H, backward=True)
    nat.gate_gating_bwd(g1[:, L * H:], y, sig, g1[:, :L * H], idx, R=M, H=H, L=L)
    torch.cuda.synchronize()
    assert torch.isfinite(g1).all()
    if M >= 4096:
        gy = torch.empty(M, 9 * H, device=DEV)
        nat.linear_group([(gmd[:, :3 * C], P(W0), None, gy[:, :3 * H]),
                          (gmd[:, 3 * C:7 * C], P(W1), None, gy[:, 3 * H:7 * H]),
                          (gmd[:, 7 * C:], P(W2), None, gy[:, 7 * H:])])
        gxo, ggo = torch.empty(M, 9, H, device=DEV), torch.empty(M, L * H, device=DEV)
        nat.gate_bwd(gy, xd, gat, gxo, ggo, idx, R=M, H=H, L=L)
        torch.cuda.synchronize()
        assert torch.equal(g1[:, L * H:].reshape(M, 9, H), gxo)
        scale = ggo.abs().max().item()
        assert (g1[:, :L * H] - ggo).abs().max().item() <= 2e-6 * scale
        return
    gy_ref = torch.cat([gm.double()[:, :3 * C] @ W0.double(), gm.double()[:, 3 * C:7 * C] @ W1.double(),
                        gm.double()[:, 7 * C:] @ W2.double()], 1).view(M, 9, H)
    gy_mag = torch.cat([gm.double()[:, :3 * C].abs() @ W0.double().abs(),
                        gm.double()[:, 3 * C:7 * C].abs() @ W1.double().abs(),
                        gm.double()[:, 7 * C:].abs() @ W2.double().abs()], 1).view(M, 9, H)
    s64 = sig.cpu().double().view(M, L, H)
    sc = s64[:, list(idx), :]
    x64 = x.double()
    sgrad0 = torch.sigmoid(x64[:, 0]) * (1 + x64[:, 0] * (1 - torch.sigmoid(x64[:, 0])))
    gx_ref = torch.cat([gy_ref[:, :1] * sgrad0[:, None], gy_ref[:, 1:] * sc], 1)
    gx_mag = torch.cat([gy_mag[:, :1] * (sgrad0.abs()[:, None] + 0.05), gy_mag[:, 1:] * sc], 1)
    out = g1[:, L * H:].cpu().double().view(M, 9, H)
    assert ((out - gx_ref).abs() / gx_mag).max() < 4e-6
    gg_ref = torch.zeros(M, L, H, dtype=torch.float64)
    gg_mag = torch.zeros(M, L, H, dtype=torch.float64)
    for c in range(1, 9):
        t = idx[c - 1]
        gg_ref[:, t] += gy_ref[:, c] * x64[:, c]
        gg_mag[:, t] += gy_mag[:, c] * x64[:, c].abs()
    d = s64 * (1 - s64)
    gg_ref, gg_mag = gg_ref * d, gg_mag * d
    gg = g1[:, :L * H].cpu().double().view(M, L, H)
    assert ((gg - gg_ref).abs() / (gg_mag + 1e-30)).max() < 1e-5


@pytest.mark.parametrize("n", [16, 64, 100, 128, 200, 256, 512])
def test_ln_silu_fwd_bwd(nat, n):
    R = 301                     # odd: the last two-row wavefront of short rows has one row
    g = torch.Generator().manual_seed(n)
    a = torch.randn(R, n, generator=g, dtype=torch.float64) * 2 + 0.5
    gam = 1 + 0.1 * torch.randn(n, generator=g, dtype=torch.float64)
    bet = 0.1 * torch.randn(n, generator=g, dtype=torch.float64)
    ar = a.clone().requires_grad_(True)
    nrm = torch.nn.functional.layer_norm(ar, (n,), gam, bet, 1e-5)
    s = torch.nn.functional.silu(nrm)
    gs = torch.randn(R, n, generator=g, dtype=torch.float64)
    (ga,) = torch.autograd.grad((s * gs).sum(), [ar])
    f = lambda t: t.float().to(DEV).contiguous()
    no, so, gao = (torch.empty(R, n, device=DEV) for _ in range(3))
    nat.ln_silu_fwd(f(a), f(gam), f(bet), no, so, R=R, n=n)
    nat.ln_silu_bwd(f(gs), f(a), no, f(gam), gao, R=R, n=n)
    torch.cuda.synchronize()
    assert (no.cpu().double() - nrm.detach()).abs().max() < 1e-5
    assert (so.cpu().double() - s.detach()).abs().max() < 1e-5
    assert (gao.cpu().double() - ga).abs().max() < 1e-4
    # strided rows: a / nrm / g_a as a column block of a wider buffer
    wide = torch.zeros(R, 3 * n, device=DEV)
    wide[:, n:2 * n] = f(a)
    nw, gw = torch.zeros(R, 3 * n, device=DEV), torch.zeros(R, 3 * n, device=DEV)
    so2 = torch.empty(R, n, device=DEV)
    nat.ln_silu_fwd(wide[:, n:2 * n], f(gam), f(bet), nw[:, n:2 * n], so2, R=R, n=n, lda=3 * n,
                    lds=n)
    nat.ln_silu_bwd(f(gs), wide[:, n:2 * n], nw[:, n:2 * n], f(gam), gw[:, n:2 * n], R=R, n=n,
                    ldg=n, lda=3 * n, ldo=3 * n)
    torch.cuda.synchronize()
    assert torch.equal(so2, so) and torch.equal(gw[:, n:2 * n], gao)
    assert gw[:, :n].abs().max() == 0 and gw[:, 2 * n:].abs().max() == 0
    # nothing is written past row R - 1
    nb, sb, gb = (torch.full((R + 1, n), float("nan"), device=DEV) for _ in range(3))
    nat.ln_silu_fwd(f(a), f(gam), f(bet), nb[:R], sb[:R], R=R, n=n)
    nat.ln_silu_bwd(f(gs), f(a), no, f(gam), gb[:R], R=R, n=n)
    torch.cuda.synchronize()
    assert torch.equal(nb[:R], no) and torch.equal(sb[:R], so) and torch.equal(gb[:R], gao)
    assert all(bool(t[R].isnan().all()) for t in (nb, sb, gb))
    # without the saved LayerNorm output: the forward does not write it, the backward recomputes
    # it from a, gamma and beta -- the same values, so the same adjoint bit for bit
    s3, g3 = torch.empty(R, n, device=DEV), torch.full((R + 1, n), float("nan"), device=DEV)
    nat.ln_silu_fwd(f(a), f(gam), f(bet), None, s3, R=R, n=n)
    nat.ln_silu_bwd(f(gs), f(a), None, f(gam), g3[:R], R=R, n=n, beta=f(bet))
    torch.cuda.synchronize()
    assert torch.equal(s3, so) and torch.equal(g3[:R], gao) and bool(g3[R].isnan().all())
    with pytest.raises(RuntimeError):
        nat.ln_silu_bwd(f(gs), f(a), None, f(gam), g3[:R], R=R, n=n)
    # g 4 bytes off a 16-byte boundary sends the backward down the element-wise path while the
    # forward (aligned rows) took the float4 one: the row statistics are summed in the same order
    # on both paths, so the recomputed LayerNorm output and the adjoint equal the float4 ones
    gbuf = torch.empty(R * n + 1, device=DEV)
    gmis = gbuf[1:].view(R, n)
    gmis.copy_(f(gs))
    g4, g5 = torch.empty(R, n, device=DEV), torch.empty(R, n, device=DEV)
    nat.ln_silu_bwd(gmis, f(a), None, f(gam), g4, R=R, n=n, beta=f(bet))
    nat.ln_silu_bwd(gmis, f(a), no, f(gam), g5, R=R, n=n)
    # and the forward on the element-wise path (misaligned LayerNorm output)
    nbuf = torch.empty(R * n + 1, device=DEV)
    nmis = nbuf[1:].view(R, n)
    s6 = torch.empty(R, n, device=DEV)
    nat.ln_silu_fwd(f(a), f(gam), f(bet), nmis, s6, R=R, n=n)
    torch.cuda.synchronize()
    for t, what in ((g4, "recomputed, element-wise"), (g5, "saved, element-wise")):
        assert torch.equal(t, gao), f"{what} adjoint differs in {int((t != gao).sum())} elements"
    assert torch.equal(nmis, no) and torch.equal(s6, so), "element-wise forward differs"


@pytest.mark.parametrize("C", [16, 128, 96, 256, 300])
def test_rmsnorm_sh_fwd_bwd(nat, C):
    from oracle.uma import rms_norm_sh
    N = 60
    g = torch.Generator().manual_seed(C)
    x = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    w = {"p.affine_weight": 1 + 0.1 * torch.randn(3, C, generator=g, dtype=torch.float64),
         "p.affine_bias": 0.1 * torch.randn(C, generator=g, dtype=torch.float64)}
    add0 = torch.randn(N, C, generator=g, dtype=torch.float64)
    res = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    y = rms_norm_sh(xr, w, "p", 2, C)
    y = torch.cat([y[:, :1] + add0[:, None], y[:, 1:]], 1)
    gy = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    (gx,) = torch.autograd.grad((y * gy).sum(), [xr])
    f = lambda t: t.float().to(DEV).contiguous()
    yo, inv, gxo = torch.empty(N, 9, C, device=DEV), torch.empty(N, device=DEV), torch.empty(N, 9, C, device=DEV)
    nat.rmsnorm_sh_fwd(f(x), f(w["p.affine_weight"]), f(w["p.affine_bias"]), f(add0), yo, inv)
    nat.rmsnorm_sh_bwd(f(gy), f(x), f(w["p.affine_weight"]), inv, f(res), gxo)
    torch.cuda.synchronize()
    assert (yo.cpu().double() - y.detach()).abs().max() < 1e-5
    assert (gxo.cpu().double() - (gx + res)).abs().max() < 1e-4


def test_forces_virial_and_sum(nat):
    N, E = 50, 600
    src, tgt, g = _rand_graph(N, E, 9)
    g_ev = torch.randn(E, 3, generator=g)
    ev = torch.randn(E, 3, generator=g)
    ref_F = -(torch.zeros(N, 3).index_add(0, src, g_ev) - torch.zeros(N, 3).index_add(0, tgt, g_ev))
    ref_V = 0.5 * (ev.T @ g_ev + g_ev.T @ ev)
    Fo, Vo, work = torch.empty(N, 3, device=DEV), torch.empty(9, device=DEV), torch.empty(256 * 9, device=DEV)
    nat.node_forces(g_ev.to(DEV), _i32(_csr(src, N)), _i32(torch.argsort(src, stable=True)),
                    _i32(_csr(tgt, N)), Fo)
    nat.virial(ev.to(DEV), g_ev.to(DEV), work, Vo)
    x = torch.randn(5000, generator=g)
    so = torch.empty(1, device=DEV)
    nat.reduce_sum(x.to(DEV), 5000, 1, so)
    torch.cuda.synchronize()
    assert (Fo.cpu() - ref_F).abs().max() < 1e-5
    assert (Vo.cpu().reshape(3, 3) - ref_V).abs().max() < 1e-3
    assert abs(float(so) - float(x.double().sum())) < 1e-3
    # a hub node (300 source and 200 destination edges: many passes of the 16 lanes of a node),
    # isolated nodes, and the same bits on a second call
    N2, E2 = 40, 900
    src2 = torch.randint(0, 30, (E2,), generator=g)
    tgt2 = torch.randint(0, 30, (E2,), generator=g)
    src2[:300], tgt2[300:500] = 7, 7
    o = torch.argsort(tgt2, stable=True)
    src2, tgt2 = src2[o], tgt2[o]
    g2 = torch.randn(E2, 3, generator=g)
    ref2 = -(torch.zeros(N2, 3).index_add(0, src2, g2) - torch.zeros(N2, 3).index_add(0, tgt2, g2))
    F2 = [torch.empty(N2, 3, device=DEV) for _ in range(2)]
    for Fi in F2:
        nat.node_forces(g2.to(DEV), _i32(_csr(src2, N2)), _i32(torch.argsort(src2, stable=True)),
                        _i32(_csr(tgt2, N2)), Fi)
    torch.cuda.synchronize()
    assert (F2[0].cpu() - ref2).abs().max() < 1e-4 and torch.equal(F2[0], F2[1])
    assert F2[0][30:].abs().max() == 0


@pytest.mark.parametrize("mode,M", [(16, 5000), (6, 5000), (16, 700)])
def test_linear_group_equals_separate_calls(nat, mode, M):
    """Grouped launches (one launch for up to four products: column blocks of one input and one
    output, as the SO(2) m-blocks use them, with bias / accumulate / two-output / silu-grad
    epilogues) give the same bits as one call per product on the split kernel in modes 16 and 6
    (M = 5000).  On the fp32 kernel (M = 700 < 4096 routes there) a product that alone is too
    small to fill the GPU (700 x 256, 88 tiles) runs split-K alone but not in the group, so the
    two agree to fp32 rounding there and bit for bit elsewhere."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, 9 * 128, generator=g).to(DEV)
    outs = {}
    for grouped in (False, True):
        out = torch.zeros(M, 640 + 512 + 256, device=DEV)
        out2 = torch.zeros(M, 640 + 512 + 256, device=DEV)  # second output: out's row layout
        aux = torch.randn(M, 256, generator=torch.Generator().manual_seed(2)).to(DEV)
        out[:, 640 + 512:] = 0.5
        ws = [torch.randn(384, 640, generator=torch.Generator().manual_seed(3)) / 20,
              torch.randn(512, 512, generator=torch.Generator().manual_seed(4)) / 20,
              torch.randn(256, 256, generator=torch.Generator().manual_seed(5)) / 20]
        ws = [nat.PackedWeight(w.to(DEV), mode) for w in ws]
        bias = torch.randn(640, generator=torch.Generator().manual_seed(6)).to(DEV)
        items = [(x[:, :384], ws[0], bias, out[:, :640], nat.EPI_STORE),
                 (x[:, 384:896], ws[1], None, out[:, 640:640 + 512], nat.EPI_PRE_SILU,
                  out2[:, 640:640 + 512]),
                 (x[:, 896:1152], ws[2], None, out[:, 640 + 512:], nat.EPI_ACCUM)]
        if grouped:
            nat.linear_group(items)
        else:
            for it in items:
                nat.linear(it[0], it[1], it[2], out=it[3], epilogue=it[4],
                           out2=it[5] if len(it) > 5 else None)
        # a fourth product type: silu-grad epilogue on its own group of one
        o4 = torch.empty(M, 256, device=DEV)
        item4 = (x[:, :256], ws[2], None, o4, nat.EPI_SILU_GRAD, None, aux)
        if grouped:
            nat.linear_group([item4])
        else:
            nat.linear(x[:, :256], ws[2], out=o4, epilogue=nat.EPI_SILU_GRAD, aux=aux)
        torch.cuda.synchronize()
        outs[grouped] = (out.clone(), out2.clone(), o4.clone())
    for a, b in zip(outs[False], outs[True]):
        if M >= 4096:
            assert torch.equal(a, b)
        else:
            assert torch.equal(a[:, :640 + 512], b[:, :640 + 512])
            assert (a - b).abs().max() <= 1e-5 * max(1.0, float(a.abs().max()))
    assert outs[True][1][:, :640].abs().max() == 0 and outs[True][1][:, 1152:].abs().max() == 0
    ref = x[:, :384].double().cpu() @ ws[0].w_t.double().cpu() + bias.double().cpu()
    assert (outs[True][0][:, :640].cpu().double() - ref).abs().max() < 1e-3


@pytest.mark.parametrize("n", [64, 128, 200])
def test_ln_silu_groups_equal_per_group(nat, n):
    """Grouped LayerNorm-SiLU (five radial MLPs side by side, odd row count) gives the same bits
    as one call per column block."""
    R, G = 1001, 5
    g = torch.Generator().manual_seed(n + 1)
    a = (torch.randn(R, G * n, generator=g) * 2 + 0.3).to(DEV)
    gam = (1 + 0.1 * torch.randn(G * n, generator=g)).to(DEV)
    bet = (0.1 * torch.randn(G * n, generator=g)).to(DEV)
    gy = torch.randn(R, G * n, generator=g).to(DEV)
    outs = []
    for grouped in (True, False):
        nrm, s, ga = (torch.full((R, G * n), float("nan"), device=DEV) for _ in range(3))
        if grouped:
            nat.ln_silu_fwd(a, gam, bet, nrm, s, R=R, n=n, groups=G)
            nat.ln_silu_bwd(gy, a, nrm, gam, ga, R=R, n=n, groups=G)
        else:
            for k in range(G):
                c = slice(k * n, (k + 1) * n)
                nat.ln_silu_fwd(a[:, c], gam[c], bet[c], nrm[:, c], s[:, c], R=R, n=n,
                                lda=G * n, lds=G * n)
                nat.ln_silu_bwd(gy[:, c], a[:, c], nrm[:, c], gam[c], ga[:, c], R=R, n=n,
                                ldg=G * n, lda=G * n, ldo=G * n)
        torch.cuda.synchronize()
        outs.append((nrm.clone(), s.clone(), ga.clone()))
    for x, y in zip(*outs):
        assert not bool(x.isnan().any()) and torch.equal(x, y)
