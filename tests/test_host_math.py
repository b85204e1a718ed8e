"""CPU tests of the device arithmetic the gfx950 kernels share with a host build
(csrc/geometry_math.h, csrc/nl_math.h): compiled here with g++ under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/host_math/host_math.cpp) and compared with the oracle.

* Wigner coefficients (geometry.py:112-155, packed as rotation.py:196-208) against the oracle's
  euler_angles / eulers_to_wigner in fp64 and fp32, pole directions included;
* their closed-form VJP against torch autograd through the oracle's SafeAcos / SafeAtan2
  (geometry.py:87-109), the regularised derivatives the reference defines;
* the p = 5 envelope and its derivative (geometry.py:243-251) against the closed form and autograd;
* the neighbour-list predicates: torch's fp32 vector norm, the per-operation rounded sums of
  squares of the periodic mask and the cap key (numpy fp32), and the cap-key order (tuples).
"""
import os
import pathlib
import shutil
import subprocess

import numpy as np
import pytest
import torch

from oracle import geometry as OG

ROOT = pathlib.Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "host_math" / "host_math.cpp"
CSRC = ROOT / "tt-atom_amd" / "csrc"

DEG = [0, 1, 2, 1, 2, 1, 2, 2, 2]
IJ = [(m, j) for m in range(9) for j in {0: [0], 1: [1, 2, 3], 2: [4, 5, 6, 7, 8]}[DEG[m]]]
PERM = torch.tensor([0, 2, 6, 3, 7, 1, 5, 8, 4])


@pytest.fixture(scope="module")
def host_math(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ is not available")
    exe = tmp_path_factory.mktemp("host_math") / "host_math"
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-Wall", "-Werror", "-Wno-unknown-pragmas",
           "-ffp-contract=off", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", f"-I{CSRC}", str(SRC), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    work = exe.parent

    def run(mode, n, param, *arrays, out_dtype=np.float32):
        inp, outp = work / f"{mode}.in", work / f"{mode}.out"
        with open(inp, "wb") as f:
            for a in arrays:
                f.write(np.ascontiguousarray(a).tobytes())
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
                   UBSAN_OPTIONS="print_stacktrace=1")
        r = subprocess.run([str(exe), mode, str(n), repr(float(param)), str(inp), str(outp)],
                           capture_output=True, text=True, env=env)
        assert r.returncode == 0, f"host_math {mode} failed ({r.returncode}):\n{r.stderr}"
        assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr
        return np.fromfile(outp, dtype=out_dtype)
    return run


def _jd():
    from tt_atom.synthetic import jd_matrices
    return jd_matrices()


def _vectors(n, seed):
    g = torch.Generator().manual_seed(seed)
    ev = torch.randn(n, 3, generator=g) * 2.0
    # at and near the poles of the edge frame (+-y), along x / z, a long and a short vector
    special = torch.tensor([[0.0, 1.0, 0.0], [0.0, -2.0, 0.0], [1e-4, 1.0, 0.0], [0.0, 1.0, 1e-5],
                            [3.0, 0.0, 0.0], [0.0, 0.0, -1.5], [1.0, 1.0, 1.0], [-1e-3, -3.0, 2e-3],
                            [40.0, -25.0, 7.0], [2e-3, 1e-3, -3e-3]])
    return torch.cat([ev, special], 0)


def _oracle_coef(ev, jd):
    wig = OG.eulers_to_wigner(OG.euler_angles(ev), 2, [j.to(ev.dtype) for j in jd])
    wig = wig.index_select(1, PERM)
    return torch.stack([wig[:, i, j] for i, j in IJ], 1)


def _jd_flat(jd):
    return torch.cat([j.reshape(-1) for j in jd]).float().numpy()


def test_wigner_coefficients(host_math):
    jd = _jd()
    ev = _vectors(600, 0)
    n = ev.shape[0]
    coef = host_math("wigner", n, 0.0, _jd_flat(jd), ev.numpy()).reshape(n, 35)
    ref64 = _oracle_coef(ev.double(), jd).numpy()
    ref32 = _oracle_coef(ev, [j.float() for j in jd]).numpy()
    # fp64 oracle on generic directions; exactly on a pole fp32 acos limits the accuracy
    assert np.abs(coef - ref64)[:-10].max() < 2e-6
    # the fp32 oracle (what the parity tests compare against) everywhere
    assert np.abs(coef - ref32).max() < 2e-6
    # orthogonality of each rebuilt block: W W^T = I
    W = np.zeros((n, 9, 9))
    for k, (i, j) in enumerate(IJ):
        W[:, i, j] = coef[:, k]
    assert np.abs(W @ W.transpose(0, 2, 1) - np.eye(9)).max() < 1e-5


def test_wigner_vjp(host_math):
    jd = _jd()
    ev = _vectors(500, 1)
    n = ev.shape[0]
    g = torch.Generator().manual_seed(11)
    g_coef = torch.randn(n, 35, generator=g)
    out = host_math("vjp", n, 0.0, _jd_flat(jd), ev.numpy(), g_coef.numpy()).reshape(n, 3)
    assert np.isfinite(out).all()
    for dt, rows, tol in ((torch.float64, slice(0, -10), 5e-4), (torch.float32, slice(None), 5e-3)):
        e = ev.to(dt).clone().requires_grad_(True)
        (ref,) = torch.autograd.grad((_oracle_coef(e, jd) * g_coef.to(dt)).sum(), e)
        ref = ref.double().numpy()
        err = np.abs(out - ref) / np.maximum(np.abs(ref), 1.0)
        assert err[rows].max() < tol, (dt, float(err[rows].max()))


def test_envelope(host_math):
    cutoff = 6.0
    d = torch.cat([torch.linspace(0.0, 7.0, 701), torch.tensor([cutoff, cutoff - 1e-6, 1e-8])])
    out = host_math("envelope", d.numel(), cutoff, d.numpy()).reshape(2, -1)
    x = d.double().clone().requires_grad_(True)
    ds = x / cutoff
    env = torch.where(ds < 1, 1 + ds ** 5 * (-21 + ds * (35 - 15 * ds)), torch.zeros_like(ds))
    (denv,) = torch.autograd.grad(env.sum(), x)
    # fp32 evaluation of polynomials whose terms reach 21 + 35 + 15 = 71 (value) and about 70
    # (derivative): near the cutoff they cancel, leaving ~71 * 2^-24 = 4.2e-6 of rounding
    assert np.abs(out[0] - env.detach().numpy()).max() < 5e-6
    assert np.abs(out[1] - denv.numpy()).max() < 1e-5
    assert out[0][d.numpy() >= cutoff].max() == 0 and out[1][d.numpy() >= cutoff].max() == 0


def test_neighbor_predicates(host_math):
    rng = np.random.default_rng(5)
    n = 4000
    a = (rng.standard_normal((n, 3)) * rng.choice([1e-3, 1.0, 30.0, 1e4], (n, 1))).astype(np.float32)
    b = (a + rng.standard_normal((n, 3)).astype(np.float32) * 3).astype(np.float32)
    sh = (rng.integers(-2, 3, (n, 3)) * 3.61).astype(np.float32)
    out = host_math("nl", n, 0.0, a, b, sh).reshape(4, n)
    f = np.float32
    # torch's fp32 norm of a - b is the square root of norm2_fma (the device lists' distance test)
    dn = torch.linalg.norm(torch.from_numpy(a) - torch.from_numpy(b), dim=1).numpy()
    assert np.array_equal(np.sqrt(out[0]), dn)

    def sum_sq(v):   # (x^2 + y^2) + z^2, every operation rounded to fp32
        return ((v[:, 0] * v[:, 0]).astype(f) + (v[:, 1] * v[:, 1]).astype(f)).astype(f) + \
               (v[:, 2] * v[:, 2]).astype(f)
    assert np.array_equal(out[1], sum_sq((a - b).astype(f)))
    assert np.array_equal(out[2], sum_sq((a - (b + sh).astype(f)).astype(f)))
    assert np.array_equal(out[3], sum_sq(((a - b).astype(f) + sh).astype(f)))


def test_cap_key_order(host_math):
    rng = np.random.default_rng(6)
    n = 3000
    d1 = rng.choice([0.5, 1.0, 2.0], n).astype(np.float32)
    d2 = rng.choice([0.5, 1.0, 2.0], n).astype(np.float32)
    a1, a2, c1, c2 = (rng.integers(0, 3, n).astype(np.int32) for _ in range(4))
    out = host_math("key", n, 0.0, d1, a1, c1, d2, a2, c2, out_dtype=np.int32).reshape(2, n)
    k1 = list(zip(d1.tolist(), a1.tolist(), c1.tolist()))
    k2 = list(zip(d2.tolist(), a2.tolist(), c2.tolist()))
    assert out[0].tolist() == [int(x <= y) for x, y in zip(k1, k2)]
    assert out[1].tolist() == [int(x < y) for x, y in zip(k1, k2)]
