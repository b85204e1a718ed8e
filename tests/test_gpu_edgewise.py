"""GPU parity of the isolated edgewise step (the C2 workload) against the CPU oracle."""
import pytest
import torch

from oracle import uma as U
from tt_atom import synthetic as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat():
    from tt_atom import _native
    _native.load()
    return _native


def _ref(ei, vec, x, g, w, N):
    ev = torch.from_numpy(vec).double().requires_grad_(True)
    out = U.isolated_edgewise(torch.from_numpy(x).double(), ev, torch.from_numpy(ei[0]),
                              torch.from_numpy(ei[1]), {k: v.double() for k, v in w.items()}, "c2",
                              S.jd_matrices(), N)
    g_ev = torch.autograd.grad((out * torch.from_numpy(g).double()).sum(), ev)[0]
    return out.detach(), g_ev


# The edge-vector VJP is ill-conditioned for edges close to the frame's pole (the +-y axis): the
# fp32 CPU oracle itself is 7.3e-5 (relative to max |g_ev|) off the fp64 one on this input, at an
# edge along -y, so the fp32 bound is 2e-4.
@pytest.mark.parametrize("precision,tol_out,tol_gev", [("f32", 2e-6, 2e-4),
                                                       ("f32-bf16x6", 2e-6, 2e-4),
                                                       ("f32-mfma", 2e-6, 2e-4),
                                                       ("bf16", 2e-2, 5e-2)])
def test_edgewise_step_matches_oracle(nat, precision, tol_out, tol_gev):
    """C2 pipeline at N = 512 (in-degree 25, E = 12,800): output and edge-vector VJP against the
    fp64 oracle; errors relative to the largest magnitude.  bf16 operands: ~2^-8 relative."""
    from tt_atom.edgewise import EdgewiseStep
    N = 512
    ei, vec, x, g = S.c2_tensors(N=N)
    w = S.c2_weights()
    step = EdgewiseStep(w, "c2", S.jd_matrices(), ei[0], ei[1], N, precision=precision)
    out, g_ev = step(x, vec, g)
    r_out, r_gev = _ref(ei, vec, x, g, w, N)
    e_out = (out.cpu().double() - r_out).abs().max().item() / r_out.abs().max().item()
    e_gev = (g_ev.cpu().double() - r_gev).abs().max().item() / r_gev.abs().max().item()
    assert e_out < tol_out and e_gev < tol_gev, (precision, e_out, e_gev)


def test_edgewise_step_full_size_vjp_is_linear(nat):
    """At the full C2 size (N = 8192, E = 204,800) the VJP is linear in the upstream adjoint:
    vjp(g1 + 2 g2) = vjp(g1) + 2 vjp(g2) up to rounding, and the forward does not depend on it.
    The residual is rounding noise: the default arithmetic's stays within 3x the fp32 MFMA
    kernel's on the same inputs (both measured ~1e-5 of max |vjp|)."""
    from tt_atom.edgewise import EdgewiseStep
    ei, vec, x, g1 = S.c2_tensors()
    g2 = torch.randn(g1.shape, generator=torch.Generator().manual_seed(9)).numpy()
    errs = {}
    for precision in ("f32", "f32-mfma"):
        step = EdgewiseStep(S.c2_weights(), "c2", S.jd_matrices(), ei[0], ei[1], 8192,
                            precision=precision)
        o1, v1 = (t.clone() for t in step(x, vec, g1))
        o2, v2 = (t.clone() for t in step(x, vec, g2))
        o3, v3 = step(x, vec, g1 + 2 * g2)
        assert torch.equal(o1, o2) and torch.equal(o1, o3)
        errs[precision] = (v3 - (v1 + 2 * v2)).abs().max().item() / v3.abs().max().item()
    assert errs["f32-mfma"] < 2e-5 and errs["f32"] < 3.0 * max(errs["f32-mfma"], 1e-6), errs


def _ref32(ei, vec, x, g, w, N):
    ev = torch.from_numpy(vec).float().requires_grad_(True)
    out = U.isolated_edgewise(torch.from_numpy(x).float(), ev, torch.from_numpy(ei[0]),
                              torch.from_numpy(ei[1]), {k: v.float() for k, v in w.items()}, "c2",
                              S.jd_matrices(), N)
    g_ev = torch.autograd.grad((out * torch.from_numpy(g).float()).sum(), ev)[0]
    return out.detach(), g_ev


_FULL_REF = {}


def _full_refs():
    """C2 full-size inputs and the fp64 / fp32 oracle results, computed once per module."""
    if not _FULL_REF:
        ei, vec, x, g = S.c2_tensors()
        w = S.c2_weights()
        _FULL_REF.update(inputs=(ei, vec, x, g), w=w, ref64=_ref(ei, vec, x, g, w, 8192),
                         ref32=_ref32(ei, vec, x, g, w, 8192))
    return _FULL_REF


# f32: errors relative to the largest magnitude within twice the fp32 CPU oracle's on the same
# inputs, or within the reduced test's bounds (2e-6 / 2e-4).
# bf16 operands (~2^-9 relative rounding per operand): output within 2e-2 of its largest
# magnitude.  The edge-vector VJP of an edge at polar angle beta from the frame's pole (the +-y
# axis) carries the Euler-angle derivative d(alpha)/d(ev) ~ 1 / (|ev| sin(beta)), which
# amplifies any rounding of that edge's coefficient adjoint by 1 / sin(beta): among 204,800
# random directions the nearest edge sits at sin(beta) ~ 3e-3, and even the fp32 oracle is
# 1.4e-4 off there.  The bf16 bounds are therefore stated on the conditioning-weighted error
# max_e |dg_e| sin(beta_e) / max |g| < 5e-2 and on the normwise error ||dg|| / ||g|| < 2e-2.
@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_edgewise_full_size_matches_oracle(nat, precision):
    """The full C2 workload (N = 8192, E = 204,800, C = 128) against the fp64 oracle."""
    from tt_atom.edgewise import EdgewiseStep
    ref = _full_refs()
    ei, vec, x, g = ref["inputs"]
    step = EdgewiseStep(ref["w"], "c2", S.jd_matrices(), ei[0], ei[1], 8192, precision=precision)
    out, g_ev = step(x, vec, g)
    r_out, r_gev = ref["ref64"]
    f_out, f_gev = ref["ref32"]
    rel = lambda a, b: (a.cpu().double() - b).abs().max().item() / b.abs().max().item()
    e_out, e_gev = rel(out, r_out), rel(g_ev, r_gev)
    b_out, b_gev = rel(f_out, r_out), rel(f_gev, r_gev)
    print(f"C2 full ({precision}): GPU out {e_out:.2e}, g_ev {e_gev:.2e}; fp32 oracle out "
          f"{b_out:.2e}, g_ev {b_gev:.2e}", flush=True)
    if precision == "bf16":
        v = torch.from_numpy(vec).double()
        sinb = torch.sqrt(v[:, 0] ** 2 + v[:, 2] ** 2) / torch.linalg.norm(v, dim=1)
        dg = (g_ev.cpu().double() - r_gev).abs().max(dim=1).values
        w_gev = (dg * sinb).max().item() / r_gev.abs().max().item()
        n_gev = (torch.linalg.norm(g_ev.cpu().double() - r_gev) / torch.linalg.norm(r_gev)).item()
        print(f"C2 full (bf16): conditioning-weighted g_ev {w_gev:.2e}, normwise {n_gev:.2e}, "
              f"min sin(beta) {sinb.min().item():.1e}", flush=True)
        assert e_out < 2e-2 and w_gev < 5e-2 and n_gev < 2e-2, (e_out, w_gev, n_gev)
    else:
        assert e_out < max(2e-6, 2 * b_out) and e_gev < max(2e-4, 2 * b_gev), (e_out, e_gev)
