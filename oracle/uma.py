"""Oracle: the eSCN-MD (UMA) backbone forward and energy head, torch-CPU.

Test infrastructure only (see ``oracle/__init__.py``).  Restates ``tests/mirror.py`` of the
reference (a bit-exact torch transcription of its device forward) and adds the two modules the
mirror lacks: the spectral feed-forward (``tt_atom/spectral.py:146-188``) used by uma-s-1, and
the per-node energy head (``tt_atom/model.py:223-235``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .geometry import radial_mlp


def l_of_coeff(lmax):
    """mirror.py:17-18."""
    return [l for l in range(lmax + 1) for _ in range(2 * l + 1)]


def expand_index_m_prime(lmax, mmax):
    """Gate index per vector coefficient in m-primed order; activation.py:19-26."""
    idx = list(range(lmax))
    for mval in range(1, mmax + 1):
        r = list(range(mval - 1, lmax))
        idx += r + r
    return idx


def so2(x, x_edge, w, p, lmax, mmax, Cin, H, extra):
    """SO(2) convolution; mirror.py:31-61 (radial multiply, m=0 linear, per-m complex GEMM)."""
    E, nsph = x.shape[0], (lmax + 1) ** 2
    xf = x.reshape(E, nsph * Cin)
    num_coef = [lmax - m + 1 for m in range(mmax + 1)]
    off = [0, (lmax + 1) * Cin]
    for m in range(1, mmax + 1):
        off.append(off[-1] + 2 * num_coef[m] * Cin)
    if f"{p}.rad_func.net.0.weight" in w:
        rad = radial_mlp(x_edge, w, f"{p}.rad_func")
        sizes = [num_coef[m] * Cin for m in range(mmax + 1)]
        o, rms = 0, []
        for m in range(mmax + 1):
            rms.append(rad[:, o:o + sizes[m]])
            o += sizes[m]
        mult = torch.cat([rms[0]] + sum(([rms[m], rms[m]] for m in range(1, mmax + 1)), []), 1)
        xf = xf * mult
    blocks = []
    x0 = F.linear(xf[:, off[0]:off[1]], w[f"{p}.fc_m0.weight"], w[f"{p}.fc_m0.bias"])
    extra_t = None
    if extra:
        extra_t, x0 = x0[:, :extra], x0[:, extra:]
    blocks.append(x0)
    for m in range(1, mmax + 1):
        nc = num_coef[m]
        blk = xf[:, off[m]:off[m + 1]].reshape(E, 2, nc * Cin)
        blk = blk @ w[f"{p}.so2_m_conv.{m-1}.fc.weight"].T
        Hh = blk.shape[-1] // 2
        blk = blk.reshape(E, 4 * Hh)
        a, b, c, d = blk[:, :Hh], blk[:, Hh:2 * Hh], blk[:, 2 * Hh:3 * Hh], blk[:, 3 * Hh:]
        blocks.append(a - d)
        blocks.append(c + b)
    out = torch.cat(blocks, 1).reshape(E, nsph, H)
    return (out, extra_t) if extra else out


def rms_norm_sh(x, w, p, lmax, C, eps=1e-5):
    """Equivariant RMS norm over SH coefficients; mirror.py:64-75."""
    nsph = (lmax + 1) ** 2
    lc = l_of_coeff(lmax)
    bdw = torch.tensor([1.0 / (2 * l + 1) / (lmax + 1) for l in lc], dtype=x.dtype).view(1, nsph, 1)
    l0 = x[:, 0:1, :]
    x = torch.cat([l0 - l0.mean(2, keepdim=True), x[:, 1:, :]], 1)
    fn = (x * x * bdw).sum(1, keepdim=True).mean(2, keepdim=True)
    fn = torch.rsqrt(fn + eps)
    aw = w[f"{p}.affine_weight"][torch.tensor(lc)].view(1, nsph, C)
    out = x * (fn * aw)
    ab = w[f"{p}.affine_bias"].view(1, 1, C)
    return torch.cat([out[:, 0:1, :] + ab, out[:, 1:, :]], 1)


def gate(gating, x, lmax, mmax, H):
    """m-primed GateActivation; mirror.py:78-82."""
    N = x.shape[0]
    ei = expand_index_m_prime(lmax, mmax)
    g = torch.sigmoid(gating).view(N, lmax, H)[:, ei, :]
    return torch.cat([F.silu(x[:, 0:1, :]), x[:, 1:, :] * g], 1)


def grid_atomwise(x, w, p, to_grid, from_grid):
    """Grid feed-forward; mirror.py:85-92."""
    b, a, nsph = to_grid.shape
    tg, fg = to_grid.reshape(b * a, nsph), from_grid.reshape(b * a, nsph)
    g = torch.einsum("pi,nic->npc", tg, x)
    g = F.silu(g @ w[f"{p}.grid_mlp.0.weight"].T)
    g = F.silu(g @ w[f"{p}.grid_mlp.2.weight"].T)
    g = g @ w[f"{p}.grid_mlp.4.weight"].T
    return torch.einsum("pi,npc->nic", fg, g)


def spectral_atomwise(x, w, p, lmax, H):
    """Spectral feed-forward (uma-s-1's FF); spectral.py:146-166 semantics.

    gating = SiLU(x[:,0] @ Ws^T + b); h = SO3_Linear_1(x) (per-degree shared weight, bias on
    l=0); h0 -> SiLU, degree-l rows * sigmoid(gating[:, (l-1)H:lH]); out = SO3_Linear_2."""
    def so3_linear(v, Wt, bias):
        outs, start = [], 0
        for l in range(lmax + 1):
            n = 2 * l + 1
            ob = v[:, start:start + n, :] @ Wt[l].T
            if l == 0:
                ob = ob + bias.view(1, 1, -1)
            outs.append(ob)
            start += n
        return torch.cat(outs, 1)

    gating = F.silu(F.linear(x[:, 0, :], w[f"{p}.scalar_mlp.0.weight"], w[f"{p}.scalar_mlp.0.bias"]))
    h = so3_linear(x, w[f"{p}.so3_linear_1.weight"], w[f"{p}.so3_linear_1.bias"])
    sg = torch.sigmoid(gating)
    parts, start = [F.silu(h[:, 0:1, :])], 1
    for l in range(1, lmax + 1):
        n = 2 * l + 1
        parts.append(h[:, start:start + n, :] * sg[:, (l - 1) * H:l * H].unsqueeze(1))
        start += n
    g = torch.cat(parts, 1)
    return so3_linear(g, w[f"{p}.so3_linear_2.weight"], w[f"{p}.so3_linear_2.bias"])


def edgewise(x, w, p, cfg, wigner, winv, x_edge, envelope, edge_index, N):
    """eSCN-MD message block; mirror.py:95-109."""
    C, H = cfg["sphere_channels"], cfg["hidden_channels"]
    lmax, mmax = cfg["lmax"], cfg["mmax"]
    nsph = (lmax + 1) ** 2
    src, tgt = edge_index[0], edge_index[1]
    m = torch.cat([x[src], x[tgt]], dim=2)
    m = torch.bmm(wigner, m)
    m, gating = so2(m, x_edge, w, f"{p}.so2_conv_1", lmax, mmax, 2 * C, H, lmax * H)
    m = gate(gating, m, lmax, mmax, H)
    m = so2(m, x_edge, w, f"{p}.so2_conv_2", lmax, mmax, H, C, 0)
    m = m * envelope
    m = torch.bmm(winv, m)
    out = torch.zeros(N, nsph, C, dtype=m.dtype)
    out.index_add_(0, tgt, m)
    return out


def backbone(w, cfg, x_init, wigner, winv, x_edge, envelope, sys_emb, edge_index,
             to_grid=None, from_grid=None):
    """Backbone; mirror.py:112-126 with the ff_type switch of model.py:148-156."""
    C, lmax, H = cfg["sphere_channels"], cfg["lmax"], cfg["hidden_channels"]
    N = x_init.shape[0]
    ff = cfg.get("ff_type", "grid")
    x = x_init
    for i in range(cfg["num_layers"]):
        p = f"blocks.{i}"
        x_res = x
        n = rms_norm_sh(x, w, f"{p}.norm_1", lmax, C)
        n = torch.cat([n[:, 0:1, :] + sys_emb.view(N, 1, C), n[:, 1:, :]], 1)
        x = edgewise(n, w, f"{p}.edge_wise", cfg, wigner, winv, x_edge, envelope, edge_index, N) + x_res
        x_res = x
        n = rms_norm_sh(x, w, f"{p}.norm_2", lmax, C)
        if ff == "spectral":
            x = spectral_atomwise(n, w, f"{p}.atom_wise", lmax, H) + x_res
        else:
            x = grid_atomwise(n, w, f"{p}.atom_wise", to_grid, from_grid) + x_res
    return rms_norm_sh(x, w, "norm", lmax, C)


def node_energy(node_emb, w):
    """Per-node energy MLP on coefficient 0; mirror.py:129-134, model.py:223-231."""
    h = node_emb[:, 0, :]
    h = F.silu(F.linear(h, w["energy_block.0.weight"], w["energy_block.0.bias"]))
    h = F.silu(F.linear(h, w["energy_block.2.weight"], w["energy_block.2.bias"]))
    return F.linear(h, w["energy_block.4.weight"], w["energy_block.4.bias"])


def energy(node_emb, w):
    return node_energy(node_emb, w).sum()


def isolated_edgewise(x, ev, src, tgt, w, p, Jd, N):
    """The isolated edgewise map (gather source features, rotate into the edge frame, SO(2)
    convolution, rotate back, segment-sum to destinations; edgewise.py:52-86 without radial, gate
    and envelope) as a differentiable function of the edge vectors ``ev``."""
    from .geometry import euler_angles, eulers_to_wigner
    C = x.shape[2]
    perm = torch.tensor([0, 2, 6, 3, 7, 1, 5, 8, 4])
    W = eulers_to_wigner(euler_angles(ev, 0.0), 2, [j.to(ev.dtype) for j in Jd]).index_select(1, perm)
    xe = torch.bmm(W, x[src])
    m = so2(xe, None, w, p, 2, 2, C, C, 0)
    back = torch.bmm(W.transpose(1, 2), m)
    return torch.zeros(N, 9, C, dtype=x.dtype).index_add_(0, tgt, back)
