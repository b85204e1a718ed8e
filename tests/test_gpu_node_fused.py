"""The fused node-level kernels (csrc/node.hip) against the oracle's restatement of the same
modules (fp64, CPU): one block's tail -- RMSNormSH_2, the spectral FF, the residual and the next
RMSNormSH -- forward and its VJP by autograd, and the per-node energy head forward and adjoint.
Node counts that are not multiples of the 16-node workgroup tile exercise the partial tiles."""
import math

import pytest
import torch

from oracle import uma as U

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def nat():
    from tt_atom import _native
    _native.load()
    return _native


def _block_weights(C, H, g):
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    w = {"n2.affine_weight": 1 + 0.1 * r(3, C), "n2.affine_bias": 0.1 * r(C),
         "nn.affine_weight": 1 + 0.1 * r(3, C), "nn.affine_bias": 0.1 * r(C),
         "ff.scalar_mlp.0.weight": r(2 * H, C) / math.sqrt(C), "ff.scalar_mlp.0.bias": 0.1 * r(2 * H),
         "ff.so3_linear_1.weight": r(3, H, C) / math.sqrt(C), "ff.so3_linear_1.bias": 0.1 * r(H),
         "ff.so3_linear_2.weight": r(3, C, H) / math.sqrt(H), "ff.so3_linear_2.bias": 0.1 * r(C)}
    return w


def _ref_block(x1, w, add0, C, H):
    n2 = U.rms_norm_sh(x1, w, "n2", 2, C)
    x2 = x1 + U.spectral_atomwise(n2, w, "ff", 2, H)
    yn = U.rms_norm_sh(x2, w, "nn", 2, C)
    if add0 is not None:
        yn = torch.cat([yn[:, :1] + add0[:, None], yn[:, 1:]], 1)
    return n2, x2, yn


@pytest.mark.parametrize("N,C,H,with_add0,with_res", [(37, 128, 128, True, True),
                                                      (16, 32, 64, False, False),
                                                      (5, 16, 16, True, False),
                                                      (70, 64, 32, False, True)])
def test_spectral_block_fwd_bwd(nat, N, C, H, with_add0, with_res):
    g = torch.Generator().manual_seed(N + C + H)
    w = _block_weights(C, H, g)
    x1 = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    add0 = torch.randn(N, C, generator=g, dtype=torch.float64) if with_add0 else None
    g_n = torch.randn(N, 9, C, generator=g, dtype=torch.float64)
    res = torch.randn(N, 9, C, generator=g, dtype=torch.float64) if with_res else None
    xr = x1.clone().requires_grad_(True)
    n2, x2, yn = _ref_block(xr, w, add0, C, H)
    loss = (yn * g_n).sum() + ((x2 * res).sum() if res is not None else 0.0)
    (g_x1,) = torch.autograd.grad(loss, [xr])
    a_s = n2[:, 0, :] @ w["ff.scalar_mlp.0.weight"].T + w["ff.scalar_mlp.0.bias"]
    W1 = w["ff.so3_linear_1.weight"]
    h = torch.cat([n2[:, :1] @ W1[0].T + w["ff.so3_linear_1.bias"], n2[:, 1:4] @ W1[1].T,
                   n2[:, 4:] @ W1[2].T], 1)

    f = lambda t: None if t is None else t.float().to(DEV).contiguous()
    W2 = w["ff.so3_linear_2.weight"]
    ff = (f(w["ff.scalar_mlp.0.weight"].T), f(w["ff.scalar_mlp.0.bias"]), f(W1.transpose(1, 2)),
          f(w["ff.so3_linear_1.bias"]), f(W2.transpose(1, 2)), f(w["ff.so3_linear_2.bias"]))
    ffb = (f(W1), f(W2), f(w["ff.scalar_mlp.0.weight"]))
    e = lambda *s: torch.full(s, float("nan"), device=DEV)
    inv2, a_so, ho, x2o, yno, invn = e(N), e(N, 2 * H), e(N, 9, H), e(N, 9, C), e(N, 9, C), e(N)
    nat.spectral_block_fwd(f(x1), (f(w["n2.affine_weight"]), f(w["n2.affine_bias"])), ff, inv2,
                           a_so, ho, x2o, next_norm=(f(w["nn.affine_weight"]),
                                                     f(w["nn.affine_bias"])),
                           add0=f(add0), yn=yno, invn=invn)
    gx1o = e(N, 9, C)
    nat.spectral_block_bwd(f(g_n), x2o, f(w["nn.affine_weight"]), invn, f(res), f(x1),
                           f(w["n2.affine_weight"]), inv2, a_so, ho, ffb, gx1o)
    torch.cuda.synchronize()
    err = lambda a, b: ((a.cpu().double() - b.detach()).abs().max() /
                        max(1.0, b.detach().abs().max().item())).item()
    errs = dict(a_s=err(a_so, a_s), h=err(ho, h), x2=err(x2o, x2), yn=err(yno, yn),
                g_x1=err(gx1o, g_x1))
    print(f"fused block N={N} C={C} H={H}: {errs}", flush=True)
    assert max(errs[k] for k in ("a_s", "h", "x2", "yn")) < 2e-5, errs
    assert errs["g_x1"] < 5e-5, errs
    # the x2-only form (no next norm) writes the same x2
    x2b = e(N, 9, C)
    nat.spectral_block_fwd(f(x1), (f(w["n2.affine_weight"]), f(w["n2.affine_bias"])), ff, inv2,
                           a_so, ho, x2b)
    torch.cuda.synchronize()
    assert torch.equal(x2b, x2o)


@pytest.mark.parametrize("N,C,H", [(41, 128, 128), (9, 16, 32)])
def test_energy_head_fwd_bwd(nat, N, C, H):
    g = torch.Generator().manual_seed(7 * N + C)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    w = {"energy_block.0.weight": r(H, C) / math.sqrt(C), "energy_block.0.bias": 0.1 * r(H),
         "energy_block.2.weight": r(H, H) / math.sqrt(H), "energy_block.2.bias": 0.1 * r(H),
         "energy_block.4.weight": r(1, H) / math.sqrt(H), "energy_block.4.bias": 0.1 * r(1)}
    ne = r(N, 9, C)
    nr = ne.clone().requires_grad_(True)
    node_e = U.node_energy(nr, w)[:, 0]
    (g_ne,) = torch.autograd.grad(node_e.sum(), [nr])
    f = lambda t: t.float().to(DEV).contiguous()
    Wt = (f(w["energy_block.0.weight"].T), f(w["energy_block.2.weight"].T),
          f(w["energy_block.4.weight"]))
    b = (f(w["energy_block.0.bias"]), f(w["energy_block.2.bias"]), f(w["energy_block.4.bias"]))
    a1, a2, eo = (torch.full(s, float("nan"), device=DEV) for s in ((N, H), (N, H), (N,)))
    nat.energy_head_fwd(f(ne), Wt, b, a1, a2, eo)
    go = torch.full((N, 9, C), float("nan"), device=DEV)
    nat.energy_head_bwd(a1, a2, f(w["energy_block.0.weight"]), f(w["energy_block.2.weight"]),
                        f(w["energy_block.4.weight"]), go)
    torch.cuda.synchronize()
    assert (eo.cpu().double() - node_e.detach()).abs().max() < 2e-5 * max(1.0, node_e.abs().max())
    assert (go.cpu().double() - g_ne).abs().max() < 2e-5 * max(1.0, g_ne.abs().max())
    assert torch.count_nonzero(go[:, 1:]).item() == 0


def test_fused_step_equals_unfused(nat):
    """uma-s-1-shaped model (spectral FF, C = H = 32) on a small cluster: the fused node path and
    the kernel-by-kernel path give the same energy and forces to fp32 rounding."""
    from tt_atom import geometry, model, synthetic, trace
    cfg = dict(synthetic.CFG_UMA_S, sphere_channels=32, hidden_channels=32, edge_channels=32,
               num_distance_basis=32, num_layers=3)
    w, host = synthetic.random_uma_bundle(cfg, seed=17)
    pos, Z = synthetic.c3_system(seed=5, n=96, radius=17.0 * (96 / 2048) ** (1 / 3))
    pos, Z = torch.from_numpy(pos), torch.from_numpy(Z)
    ei, _ = geometry.radius_graph(pos, cfg["cutoff"], max_neighbors=cfg["max_neighbors"])
    se = geometry.csd_embedding(w, torch.tensor([0.0]), torch.tensor([1.0]),
                                dataset=cfg["task"]).expand(len(Z), -1).contiguous()
    bb = model.Backbone(w, DEV, cfg)
    geo = geometry.HostGeometry(w, cfg, host["to_m"], host["gauss_offset"], host["gauss_coeff"],
                                device=DEV)
    eng = trace.TracedEngine(bb, geo, Z, ei, se, use_graph=False)
    assert eng.fused
    E1, F1 = eng(pos.to(DEV))
    ref = trace.TracedEngine(bb, geo, Z, ei, se, use_graph=False)
    ref.fused = False
    E0, F0 = ref(pos.to(DEV))
    print(f"fused vs unfused: E {E1:.8f} / {E0:.8f}, max|dF| "
          f"{(F1 - F0).abs().max().item():.2e}", flush=True)
    assert abs(E1 - E0) <= 2e-6 * max(1.0, abs(E0))
    assert (F1 - F0).abs().max().item() <= 2e-5 * max(1.0, F0.abs().max().item())
