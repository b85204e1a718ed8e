"""eSCN-MD backbone weights and per-topology graph context, laid out for the gfx950 kernels.

``Backbone`` (reference model.py:175-247) uploads the bundle's torch-``Linear``-layout weights
once, in the forms the HIP GEMMs consume: ``[in, out]`` for the forward and ``[out, in]`` for
the input-adjoint (no weight gradients are needed for forces), the SO(2) m>0 blocks fused into
``[[Wa, Wb], [-Wb, Wa]]`` (so2.py:230-253), the SO3_Linear per-degree weights expanded to one
matrix per coefficient so a batched GEMM covers all nine (spectral.py:90-103).

``GraphContext`` (reference model.py:42-135) holds the fixed-topology device buffers: the
destination-sorted edge order, the destination CSR, the source CSR permutation and the
per-edge element indices.  The per-step geometric terms live in the step engine.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _native as nat

NSPH = 9
# m-primed gate row per vector coefficient (activation.py:19-26 for lmax = mmax = 2) and the
# natural-order one of the spectral feed-forward (spectral.py:77-88)
GATE_IDX_MPRIME = (0, 1, 0, 1, 0, 1, 1, 1)
GATE_IDX_NATURAL = (0, 0, 0, 1, 1, 1, 1, 1)
TO_M_PERM = (0, 2, 6, 3, 7, 1, 5, 8, 4)

_UNSUPPORTED = ("this MI355X build runs the uma-s shape (lmax = mmax = 2, permutation to_m); "
                "got {what}")


def _dev(t, device):
    """Device copy with standard row-major strides (also for size-1 dimensions, whose stride
    torch otherwise keeps from a transposed source)."""
    t = t.detach()
    out = torch.empty(tuple(t.shape), device=device, dtype=torch.float32)
    out.copy_(t)
    return out


# GEMM arithmetic per precision setting, all with fp32 accumulation: "f32" = two power-of-two-
# scaled fp16 planes per operand, three MFMA products (fp32 GEMM accuracy), "f32-bf16x6" = three
# bf16 planes, six products (fp32 GEMM accuracy), "f32-mfma" = the fp32 MFMA kernel only,
# "bf16" = bf16 operands.
PRECISIONS = {"f32": nat.SPLIT_F16X3, "f32-bf16x6": nat.SPLIT_F32, "f32-mfma": None,
              "bf16": nat.SPLIT_BF16}


def _gw(t, device, mode):
    """A GEMM weight operand [K, N]: packed for the split kernel unless mode is None."""
    d = t if (isinstance(t, torch.Tensor) and t.is_cuda) else _dev(t, device)
    return nat.PackedWeight(d, mode) if mode is not None else d


class RadialWeights:
    """Linear -> LN -> SiLU -> Linear -> LN -> SiLU -> Linear (so2.py:54-163)."""

    def __init__(self, w, prefix, device, n_gauss, mode=None):
        g = lambda k: w[f"{prefix}.{k}"]
        self.k_in = g("net.0.weight").shape[1]
        self.hidden = g("net.0.weight").shape[0]
        self.n_out = g("net.6.weight").shape[0]
        self.w0t = _dev(g("net.0.weight").T, device)
        self.b0 = _dev(g("net.0.bias"), device)
        self.ln1w, self.ln1b = _dev(g("net.1.weight"), device), _dev(g("net.1.bias"), device)
        self.w3t = _gw(g("net.3.weight").T, device, mode)
        self.b3 = _dev(g("net.3.bias"), device)
        self.ln4w, self.ln4b = _dev(g("net.4.weight"), device), _dev(g("net.4.bias"), device)
        self.w6t = _gw(g("net.6.weight").T, device, mode)
        self.b6 = _dev(g("net.6.bias"), device)
        # adjoint operands: g @ W for each Linear; only the gaussian columns of net.0 matter for
        # the force (the element-embedding columns of x_edge do not depend on positions)
        self.w6 = _gw(g("net.6.weight"), device, mode)
        self.w3 = _gw(g("net.3.weight"), device, mode)
        self.w0g = _dev(g("net.0.weight")[:, :n_gauss], device)


def _so2_block(wm):
    """torch weight [2*Hh, K] of one m>0 SO(2) linear -> fused [[Wa, Wb], [-Wb, Wa]] [2K, 2Hh]."""
    wt = wm.T.float()                 # [K, 2Hh]
    K, twoHh = wt.shape
    Hh = twoHh // 2
    Wa, Wb = wt[:, :Hh], wt[:, Hh:]
    blk = torch.zeros(2 * K, 2 * Hh)
    blk[:K, :Hh], blk[:K, Hh:] = Wa, Wb
    blk[K:, :Hh], blk[K:, Hh:] = -Wb, Wa
    return blk


class SO2Weights:
    """SO2Convolution (so2.py:166-330) for lmax = mmax = 2."""

    def __init__(self, w, prefix, device, cin, hout, extra, n_gauss, mode=None):
        self.cin, self.hout, self.extra = cin, hout, extra
        wm0 = w[f"{prefix}.fc_m0.weight"]            # [extra + 3 hout, 3 cin]
        bm0 = w[f"{prefix}.fc_m0.bias"]
        if wm0.shape != (extra + 3 * hout, 3 * cin):
            raise RuntimeError(_UNSUPPORTED.format(what=f"fc_m0 {tuple(wm0.shape)}"))
        # one m = 0 GEMM yields [gating (extra) | coefficients 0..2 (3 hout)], the column order of
        # the torch weight; its adjoint is one GEMM with the weight as stored
        self.wm0_t = _gw(wm0.T, device, mode)                           # [3 cin, extra + 3 hout]
        self.bm0 = _dev(bm0, device)
        self.wm0 = _gw(wm0, device, mode)                               # [extra + 3 hout, 3 cin]
        # packed weights: the gating columns and the coefficient columns as separate products,
        # so that the gate can be applied in the coefficient products' epilogue
        # (the split kernel's float4 epilogue and 16-byte aligned m-block column offsets)
        self.gate_split = mode is not None and extra > 0 and hout % 4 == 0 and cin % 4 == 0
        if self.gate_split:
            self.wm0g_t = _gw(wm0[:extra].T.contiguous(), device, mode)    # [3 cin, extra]
            self.wm0c_t = _gw(wm0[extra:].T.contiguous(), device, mode)    # [3 cin, 3 hout]
            self.bm0g = _dev(bm0[:extra].contiguous(), device)
            self.bm0c = _dev(bm0[extra:].contiguous(), device)
        b1 = _so2_block(w[f"{prefix}.so2_m_conv.0.fc.weight"])          # [4 cin, 4 hout]
        b2 = _so2_block(w[f"{prefix}.so2_m_conv.1.fc.weight"])          # [2 cin, 2 hout]
        if b1.shape != (4 * cin, 4 * hout) or b2.shape != (2 * cin, 2 * hout):
            raise RuntimeError(_UNSUPPORTED.format(what="SO(2) m>0 weight shapes"))
        self.w1, self.w1_t = _gw(b1, device, mode), _gw(b1.T, device, mode)
        self.w2, self.w2_t = _gw(b2, device, mode), _gw(b2.T, device, mode)
        self.rad = (RadialWeights(w, f"{prefix}.rad_func", device, n_gauss, mode)
                    if f"{prefix}.rad_func.net.0.weight" in w else None)


class NormWeights:
    def __init__(self, w, prefix, device):
        self.aw = _dev(w[f"{prefix}.affine_weight"], device)   # [lmax+1, C]
        self.ab = _dev(w[f"{prefix}.affine_bias"], device)     # [C]


def _expand_so3(W, device):
    """SO3_Linear weight [lmax+1, out, in] -> per-coefficient [9, in, out] and [9, out, in]."""
    deg = [0, 1, 1, 1, 2, 2, 2, 2, 2]
    fwd = torch.stack([W[l].T for l in deg])
    bwd = torch.stack([W[l] for l in deg])
    return _dev(fwd, device), _dev(bwd, device)


class SpectralWeights:
    """SpectralAtomwise (spectral.py:41-188)."""

    def __init__(self, w, prefix, device, C, H):
        self.ws_t = _dev(w[f"{prefix}.scalar_mlp.0.weight"].T, device)   # [C, L*H]
        self.bs = _dev(w[f"{prefix}.scalar_mlp.0.bias"], device)
        self.ws = _dev(w[f"{prefix}.scalar_mlp.0.weight"], device)       # [L*H, C]
        self.w1_t, self.w1 = _expand_so3(w[f"{prefix}.so3_linear_1.weight"], device)
        self.w2_t, self.w2 = _expand_so3(w[f"{prefix}.so3_linear_2.weight"], device)
        b1 = torch.zeros(NSPH, H)
        b1[0] = w[f"{prefix}.so3_linear_1.bias"]
        b2 = torch.zeros(NSPH, C)
        b2[0] = w[f"{prefix}.so3_linear_2.bias"]
        self.b1, self.b2 = _dev(b1, device), _dev(b2, device)
        # per-degree forms for the fused node kernels: [in, out] forward, [out, in] backward
        W1, W2 = w[f"{prefix}.so3_linear_1.weight"], w[f"{prefix}.so3_linear_2.weight"]
        self.w1t_deg = _dev(W1.transpose(1, 2).contiguous(), device)     # [3, C, H]
        self.w2t_deg = _dev(W2.transpose(1, 2).contiguous(), device)     # [3, H, C]
        self.w1_deg = _dev(W1.contiguous(), device)                      # [3, H, C]
        self.w2_deg = _dev(W2.contiguous(), device)                      # [3, C, H]
        self.b1_l0 = _dev(w[f"{prefix}.so3_linear_1.bias"], device)
        self.b2_l0 = _dev(w[f"{prefix}.so3_linear_2.bias"], device)

    @property
    def fused_fwd(self):
        return (self.ws_t, self.bs, self.w1t_deg, self.b1_l0, self.w2t_deg, self.b2_l0)

    @property
    def fused_bwd(self):
        return (self.w1_deg, self.w2_deg, self.ws)


class GridWeights:
    """GridAtomwise (grid.py:25-76): to_grid / from_grid projections around a channel MLP."""

    def __init__(self, w, prefix, device, to_grid_mat, from_grid_mat):
        b, a, nsph = to_grid_mat.shape
        self.npts = b * a
        tg = to_grid_mat.reshape(self.npts, nsph).float()
        fg = from_grid_mat.reshape(self.npts, nsph).float()
        self.tg, self.tg_t = _dev(tg, device), _dev(tg.T, device)      # [P, 9], [9, P]
        self.fg, self.fg_t = _dev(fg, device), _dev(fg.T, device)
        self.w0_t = _dev(w[f"{prefix}.grid_mlp.0.weight"].T, device)
        self.w2_t = _dev(w[f"{prefix}.grid_mlp.2.weight"].T, device)
        self.w4_t = _dev(w[f"{prefix}.grid_mlp.4.weight"].T, device)
        self.w0 = _dev(w[f"{prefix}.grid_mlp.0.weight"], device)
        self.w2 = _dev(w[f"{prefix}.grid_mlp.2.weight"], device)
        self.w4 = _dev(w[f"{prefix}.grid_mlp.4.weight"], device)


class BlockWeights:
    def __init__(self, w, prefix, device, cfg, to_grid, from_grid, n_gauss, mode=None):
        C, H, L = cfg["sphere_channels"], cfg["hidden_channels"], cfg["lmax"]
        self.norm_1 = NormWeights(w, f"{prefix}.norm_1", device)
        self.norm_2 = NormWeights(w, f"{prefix}.norm_2", device)
        self.so2_1 = SO2Weights(w, f"{prefix}.edge_wise.so2_conv_1", device, 2 * C, H, L * H,
                                n_gauss, mode)
        self.so2_2 = SO2Weights(w, f"{prefix}.edge_wise.so2_conv_2", device, H, C, 0, n_gauss,
                                mode)
        if self.so2_1.rad is None:
            raise RuntimeError(_UNSUPPORTED.format(what="so2_conv_1 without a radial MLP"))
        self.ff_type = cfg.get("ff_type", "grid")
        if self.ff_type == "spectral":
            self.atom_wise = SpectralWeights(w, f"{prefix}.atom_wise", device, C, H)
        else:
            self.atom_wise = GridWeights(w, f"{prefix}.atom_wise", device, to_grid, from_grid)


class Backbone:
    """eSCN-MD backbone + energy head weights on the device (reference model.py:175-247)."""

    def __init__(self, weights, device, cfg, to_grid_mat=None, from_grid_mat=None, *, fast=False,
                 n_gauss=None, precision="f32"):
        # fast=True is the reference's reduced-precision device path (bf16 / bf8 weights and
        # edge tensors, device.py:146-155, calculator.py:22-66): here bf16 GEMM operands with
        # fp32 accumulation, the same rule as the Orb modules (orb_model._precision)
        if fast:
            precision = "bf16"
        if precision not in PRECISIONS:
            raise RuntimeError(f"precision must be one of {sorted(PRECISIONS)}")
        self.precision = precision
        mode = PRECISIONS[precision]
        lmax, mmax = cfg["lmax"], cfg.get("mmax", cfg["lmax"])
        if lmax != 2 or mmax != 2:
            raise RuntimeError(_UNSUPPORTED.format(what=f"lmax={lmax}, mmax={mmax}"))
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.cfg = dict(cfg)
        self.C, self.H, self.L = cfg["sphere_channels"], cfg["hidden_channels"], lmax
        if self.C % 4 or self.H % 4:
            raise RuntimeError(_UNSUPPORTED.format(what="channel counts not a multiple of 4"))
        nb = n_gauss if n_gauss is not None else cfg["num_distance_basis"]
        self.n_gauss = nb
        w = weights
        dev = self.device
        self.blocks = [BlockWeights(w, f"blocks.{i}", dev, cfg, to_grid_mat, from_grid_mat, nb, mode)
                       for i in range(cfg["num_layers"])]
        self.final_norm = NormWeights(w, "norm", dev)
        self.edge_degree = RadialWeights(w, "edge_degree_embedding.rad_func", dev, nb, mode)
        self.sphere_emb = _dev(w["sphere_embedding.weight"], dev)
        self.src_emb = _dev(w["source_embedding.weight"], dev)
        self.tgt_emb = _dev(w["target_embedding.weight"], dev)
        self.edge_channels = w["source_embedding.weight"].shape[1]
        eb = [w[f"energy_block.{i}.weight"] for i in (0, 2, 4)]
        self.eh_w_t = [_dev(x.T, dev) for x in eb]
        self.eh_w = [_dev(x, dev) for x in eb]
        self.eh_b = [_dev(w[f"energy_block.{i}.bias"], dev) for i in (0, 2, 4)]
        # the first layers of all radial MLPs read the same x_edge: one GEMM for all of them, and one
        # for the gaussian part of their input adjoints (order: edge-degree, then block 0..L-1)
        self.radials = [self.edge_degree] + [b.so2_1.rad for b in self.blocks]
        self.rad_w0t_all = _gw(torch.cat([r.w0t for r in self.radials], 1).contiguous(), dev, mode)
        self.rad_b0_all = torch.cat([r.b0 for r in self.radials]).contiguous()
        self.rad_w0g_all = _gw(torch.cat([r.w0g for r in self.radials], 0).contiguous(), dev, mode)
        if len({r.hidden for r in self.radials}) != 1 or len({r.k_in for r in self.radials}) != 1:
            raise RuntimeError(_UNSUPPORTED.format(what="radial MLPs of different widths"))
        # the LayerNorm parameters of all radial MLPs side by side (grouped LayerNorm-SiLU)
        cat = lambda name: torch.cat([getattr(r, name) for r in self.radials]).contiguous()
        self.rad_ln1w_all, self.rad_ln1b_all = cat("ln1w"), cat("ln1b")
        self.rad_ln4w_all, self.rad_ln4b_all = cat("ln4w"), cat("ln4b")
        # host tables: the entry points read them while building a launch
        self.gate_idx_mprime = GATE_IDX_MPRIME
        self.gate_idx_natural = GATE_IDX_NATURAL


class GraphContext:
    """Fixed-topology device buffers (reference model.py:42-135).

    The reference's edge order is kept at the API; internally edges are stably sorted by their
    destination (tgt) so every destination segment is contiguous, which makes the message scatter
    a deterministic segmented sum in the same per-node order as ``index_add_``."""

    def __init__(self, device, *, edge_index, num_nodes, atomic_numbers, edge_cell_shift=None):
        # The sort and the CSR offsets are built where the engine runs (an edge list from the
        # device neighbour search never leaves the device); two host synchronisations remain,
        # for the range check and the maximum in-degree.
        dev = torch.device(device)
        ei = torch.as_tensor(edge_index)
        if ei.dim() != 2 or ei.shape[0] != 2:
            raise ValueError("edge_index must be [2, E]")
        ei = ei.to(dev, torch.int64)
        N = int(num_nodes)
        E = int(ei.shape[1])
        if N >= 2 ** 31 or E >= 2 ** 31:
            raise ValueError("graph too large for int32 indices")
        if E and (N == 0 or not bool(((ei >= 0) & (ei < N)).all())):
            raise ValueError("edge_index out of range")
        self.N, self.E = N, E
        order = torch.argsort(ei[1], stable=True)                 # reference order -> dst-sorted
        self.order = order
        src_s, tgt_s = ei[0][order], ei[1][order]
        t_cnt = torch.bincount(tgt_s, minlength=N)
        tgt_ptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        tgt_ptr[1:] = torch.cumsum(t_cnt, 0)
        src_perm = torch.argsort(src_s, stable=True)              # dst-order edge ids by src
        src_ptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        src_ptr[1:] = torch.cumsum(torch.bincount(src_s, minlength=N), 0)
        i32 = lambda a: a.to(torch.int32).contiguous()
        self.src, self.tgt = i32(src_s), i32(tgt_s)
        self.tgt_ptr, self.src_ptr, self.src_perm = i32(tgt_ptr), i32(src_ptr), i32(src_perm)
        self.Z = torch.as_tensor(atomic_numbers).to(dev, torch.int64)
        self.zsrc, self.ztgt = i32(self.Z[src_s]), i32(self.Z[tgt_s])
        self.shift = None
        if edge_cell_shift is not None:
            sh = torch.as_tensor(edge_cell_shift, dtype=torch.float32).to(dev)[order]
            self.shift = sh.contiguous()
        self.max_in_degree = int(t_cnt.max()) if N else 0
