"""Fixed-topology energy + forces (+ virial) step on the GPU: the eSCN-MD forward and its
hand-written reverse pass, every E-sized operation a gfx950 HIP kernel.

Reference: the device forward (model.py:158-235, edgewise.py:39-87, so2.py:255-330,
edge_degree.py:43-66), the device VJP (forces.py:104-495), the host geometry and its autograd
finish (geometry.py:226-280, forces.py:545-589) and the trace engine interface
(trace.py:83-215: build once per topology, then ``engine(pos)`` per step).  Here the geometric
terms and their VJP are kernels too, so a step is positions in, (E, F[, virial]) out, with no
host round trip in between.  All buffers are allocated once per topology.

Batching across the layer structure (same math, fewer and larger launches):
* the first linear of every radial MLP (edge-degree + one per block) reads the same x_edge, so
  it is one GEMM with the stacked weights; the gaussian part of their input adjoints is likewise
  one GEMM over the stacked first-layer adjoints (no read-modify-write accumulation);
* conv-1's m = 0 block produces [gating | coefficients 0..2] with one GEMM into a combined row
  ``[gating (L*H) | out (9*H)]``; its adjoint is one GEMM on the same combined layout.
"""
from __future__ import annotations

import torch

from . import _native as nat
from .graphs import StepGraphs
from .model import GraphContext, NSPH


class _Buf:
    pass


class TracedEngine:
    """``engine = TracedEngine(bb, geo, Z, edge_index, sys_emb, edge_cell_shift=None)``;
    ``E, F = engine(pos)`` or ``E, F, virial = engine(pos, compute_stress=True)``.

    ``pos`` may be a host or device tensor; returned forces live on the device of ``pos``.
    With ``use_graph`` (default) the step is a HIP graph captured on the second call of each
    variant (with / without stress) and replayed afterwards, as the reference replays its trace."""

    def __init__(self, bb, geo, atomic_numbers, edge_index, sys_emb, edge_cell_shift=None,
                 use_graph=True):
        nat.load()
        self.use_graph = use_graph
        self._graphs = StepGraphs(self._step)
        self.bb, self.geo = bb, geo
        dev = bb.device
        self.device = dev
        N = int(torch.as_tensor(atomic_numbers).numel())
        self.g = GraphContext(dev, edge_index=edge_index, num_nodes=N,
                              atomic_numbers=atomic_numbers, edge_cell_shift=edge_cell_shift)
        g = self.g
        E = g.E
        if E == 0:
            raise ValueError("no edges within cutoff -- system too sparse for this model")
        zmax = min(bb.sphere_emb.shape[0], bb.src_emb.shape[0], bb.tgt_emb.shape[0])
        if N and (int(g.Z.min()) < 0 or int(g.Z.max()) >= zmax):
            raise ValueError(f"atomic numbers must lie in [0, {zmax})")
        C, H, L = bb.C, bb.H, bb.L
        ec = bb.edge_channels
        nb = geo.n_gauss
        if nb != bb.n_gauss:
            raise RuntimeError("gaussian basis size differs between geometry and backbone")
        self.N, self.E, self.C, self.H, self.L, self.ec, self.nb = N, E, C, H, L, ec, nb
        self.k_in = nb + 2 * ec
        f32 = dict(device=dev, dtype=torch.float32)
        z = lambda *s: torch.zeros(*s, **f32)
        emp = lambda *s: torch.empty(*s, **f32)
        hid = bb.edge_degree.hidden
        self.hid = hid
        nrad = len(bb.radials)
        self.nrad = nrad
        # pos-independent node init: sphere_emb[Z] + sys_emb on coefficient 0 (geometry.py:257-258)
        se = torch.as_tensor(sys_emb, dtype=torch.float32).reshape(N, C).to(dev)
        self.sys_emb = se.contiguous()
        self.l0 = z(N, NSPH, C)
        self.l0[:, 0, :] = bb.sphere_emb[g.Z] + se
        # per-step geometry
        self.pos = emp(N, 3)
        self.ev, self.dist, self.coef, self.env = emp(E, 3), emp(E), emp(E, 35), emp(E)
        self.x_edge = emp(E, self.k_in)
        # accumulated geometric adjoints
        self.g_coef, self.g_env, self.g_gauss = emp(E, 35), emp(E), emp(E, nb)
        self.g_ev, self.forces = emp(E, 3), emp(N, 3)
        self.energy_buf, self.virial_buf, self.virial_work = emp(1), emp(9), emp(256 * 9)
        # radial MLPs side by side (edge-degree, then block 0..L-1): pre-LN and SiLU outputs of
        # both hidden layers (the LayerNorm outputs are recomputed in the backward), and the
        # adjoints
        self.a0_all, self.g_a0_all = (emp(E, nrad * hid) for _ in range(2))
        self.s1_all, self.a3_all, self.s2_all = (emp(E, nrad * hid) for _ in range(3))
        self.t1_all, self.t2_all = emp(E, nrad * hid), emp(E, nrad * hid)
        # shared edge temporaries
        self.LHc = L * H + NSPH * H                      # combined conv-1 row [gating | out]
        self.xf, self.g_xf = emp(E, NSPH, 2 * C), emp(E, NSPH, 2 * C)
        # the rotation backward walks each node's edges from both ends (C <= 64, 128 or 256), so
        # the [E, 9, 2C] adjoint of the gather exists only for other widths; coef_half: the
        # source walk's coefficient sums
        self.bw_walk = nat.bw_walk_width_ok(C)
        self.g_mcat = None if self.bw_walk else emp(E, NSPH, 2 * C)
        self.coef_half = emp(E, 35) if self.bw_walk else None
        # the gate in the SO(2) GEMM epilogues for edge-level launches on the split kernel; below
        # 4096 edges (launch-latency bound) the separate gating product would add launches, so
        # the gate keeps its own passes there
        self.gate_fused = E >= 4096 and all(b.so2_1.gate_split for b in bb.blocks)
        if not self.gate_fused:
            # the gated conv-1 rows and their adjoint on the path with the gate as its own pass
            self.y, self.g_y = emp(E, NSPH, H), emp(E, NSPH, H)
        self.g_tsum = emp(N, NSPH, C)                    # per-node source-half adjoint sums
        self.g1c = emp(E, self.LHc)
        self.g_mso2 = emp(E, NSPH, C)
        # per-radial output caches and their adjoints (kept per block: the radial backward of all
        # blocks runs once, after the blocks)
        self.ed = self._radial_cache(E, 3 * C, dev, 0)
        # per-block caches
        self.blk = []
        for i, b in enumerate(bb.blocks):
            c = _Buf()
            c.x_in, c.n1, c.x1, c.n2 = (emp(N, NSPH, C) for _ in range(4))
            c.inv1, c.inv2 = emp(N), emp(N)
            c.rad = self._radial_cache(E, 6 * 2 * C, dev, 1 + i)
            c.mso2 = emp(E, NSPH, C)
            if self.gate_fused:
                # the gate runs in the conv-1 epilogue: gating sigmoids, the gated rows (conv-2's
                # input, kept for the backward) and coefficient 0's pre-activation
                c.sig1, c.y1, c.x01 = emp(E, L * H), emp(E, NSPH, H), emp(E, H)
            else:
                c.o1c = emp(E, self.LHc)         # [gating | ungated coefficients]
            if b.ff_type == "spectral":
                c.a_s, c.gat, c.h, c.gout = emp(N, L * H), emp(N, L * H), emp(N, NSPH, H), emp(N, NSPH, H)
            else:
                P = b.atom_wise.npts
                c.xg, c.a1, c.sg1, c.a2, c.sg2, c.gg = (emp(N, P, C) for _ in range(6))
            self.blk.append(c)
        self.x_final, self.ne, self.inv_f = emp(N, NSPH, C), emp(N, NSPH, C), emp(N)
        self.eh_a1, self.eh_s1 = emp(N, H), emp(N, H)
        self.eh_a2, self.eh_s2 = emp(N, H), emp(N, H)
        self.node_e = emp(N, 1)
        self.ones = torch.ones(N, 1, **f32)
        # node adjoint temporaries
        self.gn_a, self.gn_b, self.gn_c = emp(N, NSPH, C), emp(N, NSPH, C), emp(N, NSPH, C)
        self.g_eh1, self.g_eh2 = emp(N, H), emp(N, H)
        self.gs_h, self.gs_h2, self.gs_g = emp(N, NSPH, H), emp(N, NSPH, H), emp(N, L * H)
        self.gs_a = emp(N, L * H)
        P = max([b.atom_wise.npts for b in bb.blocks if b.ff_type != "spectral"], default=0)
        self.gt1, self.gt2 = emp(N * P, C), emp(N * P, C)
        # uma-s-1 form (spectral FF in every block): each block's node-level tail -- RMSNormSH_2,
        # the spectral FF, the residual add and the next RMSNormSH -- and the energy head run as
        # single fused kernels, forward and backward
        self.fused = (len(bb.blocks) > 0 and all(b.ff_type == "spectral" for b in bb.blocks)
                      and nat.node_fusable(C, H))

    def _radial_cache(self, E, n_out, dev, r):
        c = _Buf()
        f32 = dict(device=dev, dtype=torch.float32)
        c.r = r
        c.out = torch.empty(E, n_out, **f32)
        c.g_out = torch.empty(E, n_out, **f32)
        return c

    # ------------------------------------------------------------------ radial MLPs
    # The radial MLPs of the edge-degree embedding and of every block (so2.py:54-163) depend only
    # on the edge features, so they run side by side: one grouped LayerNorm-SiLU per hidden layer
    # and one grouped GEMM launch per linear, forward before the blocks and backward after them.
    def _radials_fwd(self):
        bb, E, hid, R = self.bb, self.E, self.hid, self.nrad
        col = lambda t, r: t[:, r * hid:(r + 1) * hid]
        caches = [self.ed] + [c.rad for c in self.blk]
        nat.ln_silu_fwd(self.a0_all, bb.rad_ln1w_all, bb.rad_ln1b_all, None, self.s1_all,
                        R=E, n=hid, groups=R)
        nat.linear_group([(col(self.s1_all, r), rw.w3t, rw.b3, col(self.a3_all, r))
                          for r, rw in enumerate(bb.radials)])
        nat.ln_silu_fwd(self.a3_all, bb.rad_ln4w_all, bb.rad_ln4b_all, None, self.s2_all,
                        R=E, n=hid, groups=R)
        nat.linear_group([(col(self.s2_all, r), rw.w6t, rw.b6, c.out)
                          for r, (rw, c) in enumerate(zip(bb.radials, caches))])

    def _radials_bwd(self):
        bb, E, hid, R = self.bb, self.E, self.hid, self.nrad
        col = lambda t, r: t[:, r * hid:(r + 1) * hid]
        caches = [self.ed] + [c.rad for c in self.blk]
        nat.linear_group([(c.g_out, rw.w6, None, col(self.t1_all, r))
                          for r, (rw, c) in enumerate(zip(bb.radials, caches))])
        nat.ln_silu_bwd(self.t1_all, self.a3_all, None, bb.rad_ln4w_all, self.t2_all,
                        R=E, n=hid, groups=R, beta=bb.rad_ln4b_all)
        nat.linear_group([(col(self.t2_all, r), rw.w3, None, col(self.t1_all, r))
                          for r, rw in enumerate(bb.radials)])
        nat.ln_silu_bwd(self.t1_all, self.a0_all, None, bb.rad_ln1w_all, self.g_a0_all,
                        R=E, n=hid, groups=R, beta=bb.rad_ln1b_all)

    # ------------------------------------------------------------------ feed-forward
    def _spectral_fwd(self, aw, c, x, res, out):
        N, C, H, L = self.N, self.C, self.H, self.L
        x2d = x.view(N, NSPH * C)
        nat.linear(x2d[:, :C], aw.ws_t, aw.bs, out=c.a_s, epilogue=nat.EPI_PRE_SILU, out2=c.gat)
        nat.gemm(x, aw.w1_t, c.h, bias=aw.b1, M=N, N=H, K=C, lda=NSPH * C, ldb=H, ldc=NSPH * H,
                 batch=NSPH, sA=C, sB=C * H, sC=H, sBias=H)
        nat.gate_fwd(c.h, c.gat, c.gout, self.bb.gate_idx_natural, R=N, H=H, L=L)
        out.copy_(res)
        nat.gemm(c.gout, aw.w2_t, out, bias=aw.b2, M=N, N=C, K=H, lda=NSPH * H, ldb=C,
                 ldc=NSPH * C, batch=NSPH, sA=H, sB=H * C, sC=C, sBias=C, epilogue=nat.EPI_ACCUM)

    def _spectral_bwd(self, aw, c, g, out):
        N, C, H, L = self.N, self.C, self.H, self.L
        nat.gemm(g, aw.w2, self.gs_h, M=N, N=H, K=C, lda=NSPH * C, ldb=H, ldc=NSPH * H,
                 batch=NSPH, sA=C, sB=C * H, sC=H)
        nat.gate_bwd(self.gs_h, c.h, c.gat, self.gs_h2, self.gs_g, self.bb.gate_idx_natural,
                     R=N, H=H, L=L)
        nat.gemm(self.gs_h2, aw.w1, out, M=N, N=C, K=H, lda=NSPH * H, ldb=C, ldc=NSPH * C,
                 batch=NSPH, sA=H, sB=H * C, sC=C)
        nat.silu_bwd(self.gs_g, c.a_s, self.gs_a)
        nat.linear(self.gs_a, aw.ws, out=out.view(N, NSPH * C)[:, :C], epilogue=nat.EPI_ACCUM)

    def _grid_fwd(self, aw, c, x, res, out):
        N, C, P = self.N, self.C, aw.npts
        nat.gemm(aw.tg, x, c.xg, M=P, N=C, K=NSPH, lda=NSPH, ldb=C, ldc=C, batch=N, sA=0,
                 sB=NSPH * C, sC=P * C)
        xg, a1, s1, a2, s2, gg = (t.view(N * P, C) for t in (c.xg, c.a1, c.sg1, c.a2, c.sg2, c.gg))
        nat.linear(xg, aw.w0_t, out=a1, epilogue=nat.EPI_PRE_SILU, out2=s1)
        nat.linear(s1, aw.w2_t, out=a2, epilogue=nat.EPI_PRE_SILU, out2=s2)
        nat.linear(s2, aw.w4_t, out=gg)
        out.copy_(res)
        nat.gemm(aw.fg_t, c.gg, out, M=NSPH, N=C, K=P, lda=P, ldb=C, ldc=C, batch=N, sA=0,
                 sB=P * C, sC=NSPH * C, epilogue=nat.EPI_ACCUM)

    def _grid_bwd(self, aw, c, g, out):
        N, C, P = self.N, self.C, aw.npts
        t1, t2 = self.gt1[:N * P], self.gt2[:N * P]
        nat.gemm(aw.fg, g, t1, M=P, N=C, K=NSPH, lda=NSPH, ldb=C, ldc=C, batch=N, sA=0,
                 sB=NSPH * C, sC=P * C)                                   # g wrt grid output
        nat.linear(t1, aw.w4, out=t2, epilogue=nat.EPI_SILU_GRAD, aux=c.a2.view(N * P, C))
        nat.linear(t2, aw.w2, out=t1, epilogue=nat.EPI_SILU_GRAD, aux=c.a1.view(N * P, C))
        nat.linear(t1, aw.w0, out=t2)                                     # g wrt x_grid
        nat.gemm(aw.tg_t, t2, out, M=NSPH, N=C, K=P, lda=P, ldb=C, ldc=C, batch=N, sA=0,
                 sB=P * C, sC=NSPH * C)

    # ------------------------------------------------------------------ forward
    def _forward(self):
        bb, geo, g = self.bb, self.geo, self.g
        E, N, C, H, L = self.E, self.N, self.C, self.H, self.L
        LH, LHc = L * H, self.LHc
        nat.edge_geometry_fwd(self.pos, g.src, g.tgt, g.shift, geo.jd, geo.gamma, g.zsrc,
                              g.ztgt, bb.src_emb, bb.tgt_emb, geo.offset, geo.coeff, geo.cutoff,
                              self.nb, self.ec, self.ev, self.dist, self.coef, self.x_edge,
                              self.env)
        nat.linear(self.x_edge, bb.rad_w0t_all, bb.rad_b0_all, out=self.a0_all)
        self._radials_fwd()
        # edge-degree node init (geometry.py:268-276)
        x = self.blk[0].x_in if self.blk else self.x_final
        nat.rotate_env_segsum(self.ed.out, self.coef, self.env, g.tgt_ptr, self.l0, x, n_in=3,
                              env_first=False, div=geo.rescale)
        Cin = 2 * C
        for i, (bw, c) in enumerate(zip(bb.blocks, self.blk)):
            s1w, s2w = bw.so2_1, bw.so2_2
            if not self.fused or i == 0:       # fused: produced by the previous block's tail
                nat.rmsnorm_sh_fwd(c.x_in, bw.norm_1.aw, bw.norm_1.ab, self.sys_emb, c.n1, c.inv1)
            nat.gather_rotate(c.n1, g.src, g.tgt, self.coef, c.rad.out, self.xf)
            xf = self.xf.view(E, NSPH * Cin)
            if self.gate_fused:
                # the gating columns' sigmoids first, then the three m-block contractions (m = 0,
                # 1, 2: one launch) with the gate applied as their rows are written
                nat.linear(xf[:, :3 * Cin], s1w.wm0g_t, s1w.bm0g, out=c.sig1,
                           epilogue=nat.EPI_SIGMOID)
                yv = c.y1.view(E, NSPH * H)
                nat.linear_group_gate([(xf[:, :3 * Cin], s1w.wm0c_t, s1w.bm0c, yv[:, :3 * H]),
                                       (xf[:, 3 * Cin:7 * Cin], s1w.w1, None, yv[:, 3 * H:7 * H]),
                                       (xf[:, 7 * Cin:], s1w.w2, None, yv[:, 7 * H:])],
                                      (0, 3, 7), c.sig1, c.x01, bb.gate_idx_mprime, H)
                y = yv
            else:
                o1 = c.o1c
                # the three m-block contractions (m = 0 with the gating columns, 1, 2): one launch
                nat.linear_group([(xf[:, :3 * Cin], s1w.wm0_t, s1w.bm0, o1[:, :LH + 3 * H]),
                                  (xf[:, 3 * Cin:7 * Cin], s1w.w1, None, o1[:, LH + 3 * H:LH + 7 * H]),
                                  (xf[:, 7 * Cin:], s1w.w2, None, o1[:, LH + 7 * H:])])
                nat.gate_fwd(o1[:, LH:], o1, self.y, bb.gate_idx_mprime, R=E, H=H, L=L, ldx=LHc,
                             ldg=LHc)
                y = self.y.view(E, NSPH * H)
            ms = c.mso2.view(E, NSPH * C)
            nat.linear_group([(y[:, :3 * H], s2w.wm0_t, s2w.bm0, ms[:, :3 * C]),
                              (y[:, 3 * H:7 * H], s2w.w1, None, ms[:, 3 * C:7 * C]),
                              (y[:, 7 * H:], s2w.w2, None, ms[:, 7 * C:])])
            nat.rotate_env_segsum(c.mso2, self.coef, self.env, g.tgt_ptr, c.x_in, c.x1, n_in=9,
                                  env_first=True)
            x_out = self.blk[i + 1].x_in if i + 1 < len(self.blk) else self.x_final
            if self.fused:
                if i + 1 < len(self.blk):
                    nb, nc = bb.blocks[i + 1], self.blk[i + 1]
                    nxt = dict(next_norm=(nb.norm_1.aw, nb.norm_1.ab), add0=self.sys_emb,
                               yn=nc.n1, invn=nc.inv1)
                else:
                    nxt = dict(next_norm=(bb.final_norm.aw, bb.final_norm.ab), yn=self.ne,
                               invn=self.inv_f)
                nat.spectral_block_fwd(c.x1, (bw.norm_2.aw, bw.norm_2.ab),
                                       bw.atom_wise.fused_fwd, c.inv2, c.a_s, c.h, x_out, **nxt)
                continue
            nat.rmsnorm_sh_fwd(c.x1, bw.norm_2.aw, bw.norm_2.ab, None, c.n2, c.inv2)
            if bw.ff_type == "spectral":
                self._spectral_fwd(bw.atom_wise, c, c.n2, c.x1, x_out)
            else:
                self._grid_fwd(bw.atom_wise, c, c.n2, c.x1, x_out)
        if self.fused:
            nat.energy_head_fwd(self.ne, (bb.eh_w_t[0], bb.eh_w_t[1], bb.eh_w[2]), bb.eh_b,
                                self.eh_a1, self.eh_a2, self.node_e.view(N))
            nat.reduce_sum(self.node_e, N, 1, self.energy_buf)
            return
        nat.rmsnorm_sh_fwd(self.x_final, bb.final_norm.aw, bb.final_norm.ab, None, self.ne,
                           self.inv_f)
        ne2 = self.ne.view(N, NSPH * C)
        nat.linear(ne2[:, :C], bb.eh_w_t[0], bb.eh_b[0], out=self.eh_a1,
                   epilogue=nat.EPI_PRE_SILU, out2=self.eh_s1)
        nat.linear(self.eh_s1, bb.eh_w_t[1], bb.eh_b[1], out=self.eh_a2,
                   epilogue=nat.EPI_PRE_SILU, out2=self.eh_s2)
        nat.linear(self.eh_s2, bb.eh_w_t[2], bb.eh_b[2], out=self.node_e)
        nat.reduce_sum(self.node_e, N, 1, self.energy_buf)

    # ------------------------------------------------------------------ reverse
    def _backward(self):
        bb, N, C = self.bb, self.N, self.C
        nat.fill(self.g_coef, 0.0)
        nat.fill(self.g_env, 0.0)
        if self.fused:
            self._backward_fused()
            return
        # energy head (forces.py:438-461): dE/dnode_e = 1
        nat.linear(self.ones, bb.eh_w[2], out=self.g_eh2, epilogue=nat.EPI_SILU_GRAD, aux=self.eh_a2)
        nat.linear(self.g_eh2, bb.eh_w[1], out=self.g_eh1, epilogue=nat.EPI_SILU_GRAD, aux=self.eh_a1)
        nat.fill(self.gn_a, 0.0)
        nat.linear(self.g_eh1, bb.eh_w[0], out=self.gn_a.view(N, NSPH * C)[:, :C])
        gcur = self.gn_b
        nat.rmsnorm_sh_bwd(self.gn_a, self.x_final, bb.final_norm.aw, self.inv_f, None, gcur)
        for bw, c in zip(reversed(bb.blocks), reversed(self.blk)):
            # x2 = ff(norm2(x1)) + x1
            g_n2 = self.gn_a
            if bw.ff_type == "spectral":
                self._spectral_bwd(bw.atom_wise, c, gcur, g_n2)
            else:
                self._grid_bwd(bw.atom_wise, c, gcur, g_n2)
            g_x1 = self.gn_c
            nat.rmsnorm_sh_bwd(g_n2, c.x1, bw.norm_2.aw, c.inv2, gcur, g_x1)
            # x1 = edgewise(norm1(x_in)) + x_in
            g_n1 = self.gn_a
            self._edgewise_bwd(bw, c, g_x1, g_n1)
            g_in = self.gn_b
            nat.rmsnorm_sh_bwd(g_n1, c.x_in, bw.norm_1.aw, c.inv1, g_x1, g_in)
            gcur = g_in
        self._backward_tail(gcur)

    def _edgewise_bwd(self, bw, c, g_x1, g_n1):
        """The edgewise block's reverse from the adjoint g_x1 of its output (the residual's
        share excluded) to the adjoint g_n1 of its normalised input (forces.py:352-418)."""
        g = self.g
        E, C, H, L = self.E, self.C, self.H, self.L
        LH, LHc, Cin = L * H, self.LHc, 2 * C
        s1w, s2w = bw.so2_1, bw.so2_2
        nat.rotate_env_segsum_bw(g_x1, g.tgt, c.mso2, self.coef, self.env, self.g_mso2,
                                 self.g_coef, self.g_env, n_in=9, env_first=True)
        gm = self.g_mso2.view(E, NSPH * C)
        g1 = self.g1c
        if self.gate_fused:
            # conv-2's adjoint products with the gate's input adjoint applied as they are written
            # (straight into the coefficient part of conv-1's adjoint operand), then the gating
            # adjoint from them and the kept gated rows
            nat.linear_group_gate([(gm[:, :3 * C], s2w.wm0, None, g1[:, LH:LH + 3 * H]),
                                   (gm[:, 3 * C:7 * C], s2w.w1_t, None, g1[:, LH + 3 * H:LH + 7 * H]),
                                   (gm[:, 7 * C:], s2w.w2_t, None, g1[:, LH + 7 * H:])],
                                  (0, 3, 7), c.sig1, c.x01, self.bb.gate_idx_mprime, H,
                                  backward=True)
            nat.gate_gating_bwd(g1[:, LH:], c.y1, c.sig1, g1[:, :LH], self.bb.gate_idx_mprime,
                                R=E, H=H, L=L)
        else:
            gy = self.g_y.view(E, NSPH * H)
            nat.linear_group([(gm[:, :3 * C], s2w.wm0, None, gy[:, :3 * H]),
                              (gm[:, 3 * C:7 * C], s2w.w1_t, None, gy[:, 3 * H:7 * H]),
                              (gm[:, 7 * C:], s2w.w2_t, None, gy[:, 7 * H:])])
            o1 = c.o1c
            nat.gate_bwd(self.g_y, o1[:, LH:], o1, g1[:, LH:], g1, self.bb.gate_idx_mprime, R=E,
                         H=H, L=L, ldx=LHc, ldg=LHc)
        gx = self.g_xf.view(E, NSPH * Cin)
        nat.linear_group([(g1[:, :LH + 3 * H], s1w.wm0, None, gx[:, :3 * Cin]),
                          (g1[:, LH + 3 * H:LH + 7 * H], s1w.w1_t, None, gx[:, 3 * Cin:7 * Cin]),
                          (g1[:, LH + 7 * H:], s1w.w2_t, None, gx[:, 7 * Cin:])])
        if self.bw_walk:
            # walked from both ends of every edge: each half of the gather adjoint is summed per
            # node in registers instead of crossing HBM as [E, 9, C] (source half) and being
            # gathered back
            nat.gather_rotate_bw_nodes(self.g_xf, c.rad.out, c.n1, g.src_ptr, g.src_perm,
                                       g.tgt_ptr, self.coef, c.rad.g_out, self.g_coef,
                                       self.coef_half, self.g_tsum, None, g_n1)
        else:
            nat.gather_rotate_bw(self.g_xf, c.rad.out, c.n1, g.src, g.tgt, self.coef,
                                 c.rad.g_out, self.g_mcat, self.g_coef)
            nat.node_gather_sum(self.g_mcat, g.src_ptr, g.src_perm, g.tgt_ptr, None, g_n1)

    def _backward_fused(self):
        """Reverse of the fused forward: the energy head's adjoint, then per block (last first) the
        fused node-level tail (the next norm's backward + the residual adjoint, the spectral FF
        and norm_2 backward) and the edgewise reverse; block 0's norm_1 last."""
        bb, N = self.bb, self.N
        g_n = self.gn_a
        nat.energy_head_bwd(self.eh_a1, self.eh_a2, bb.eh_w[0], bb.eh_w[1], bb.eh_w[2], g_n)
        res = None
        spare = [self.gn_b, self.gn_c]
        nblk = len(bb.blocks)
        for i in reversed(range(nblk)):
            bw, c = bb.blocks[i], self.blk[i]
            if i + 1 < nblk:
                x2, awn, invn = self.blk[i + 1].x_in, bb.blocks[i + 1].norm_1.aw, self.blk[i + 1].inv1
            else:
                x2, awn, invn = self.x_final, bb.final_norm.aw, self.inv_f
            g_x1 = spare[0] if res is not spare[0] else spare[1]
            nat.spectral_block_bwd(g_n, x2, awn, invn, res, c.x1, bw.norm_2.aw, c.inv2, c.a_s,
                                   c.h, bw.atom_wise.fused_bwd, g_x1)
            self._edgewise_bwd(bw, c, g_x1, g_n)          # g_n <- adjoint of this block's n1
            res = g_x1
        c0, bw0 = self.blk[0], bb.blocks[0]
        gcur = spare[0] if res is not spare[0] else spare[1]
        nat.rmsnorm_sh_bwd(g_n, c0.x_in, bw0.norm_1.aw, c0.inv1, res, gcur)
        self._backward_tail(gcur)

    def _backward_tail(self, gcur):
        """Edge-degree init backward, the radial MLPs' backward and the geometry VJP to forces,
        from the adjoint gcur of block 0's input."""
        bb, g = self.bb, self.g
        # edge-degree init backward (edge_degree.py:69-93)
        nat.rotate_env_segsum_bw(gcur, g.tgt, self.ed.out, self.coef, self.env, self.ed.g_out,
                                 self.g_coef, self.g_env, n_in=3, env_first=False,
                                 div=self.geo.rescale)
        self._radials_bwd()
        # gaussian columns of x_edge: one GEMM over the stacked first-layer adjoints
        nat.linear(self.g_a0_all, bb.rad_w0g_all, out=self.g_gauss)
        # geometry VJP -> forces (forces.py:580-589 in closed form)
        geo = self.geo
        nat.edge_geometry_bwd(self.ev, self.dist, self.g_coef, self.g_env, self.g_gauss, self.nb,
                              geo.offset, geo.coeff, geo.cutoff, self.nb, geo.jd, geo.gamma,
                              self.g_ev)
        nat.node_forces(self.g_ev, g.src_ptr, g.src_perm, g.tgt_ptr, self.forces)

    # ------------------------------------------------------------------ step
    def _step(self, compute_stress):
        self._forward()
        self._backward()
        if compute_stress:
            nat.virial(self.ev, self.g_ev, self.virial_work, self.virial_buf)

    def run(self, pos, compute_stress=False, eager=False):
        """Enqueue one step; results stay on the device (energy_buf, forces, virial_buf).
        ``eager`` launches the kernels one by one instead of replaying the graph."""
        self.pos.copy_(torch.as_tensor(pos, dtype=torch.float32).reshape(self.N, 3),
                       non_blocking=True)
        if self.use_graph and not eager:
            self._graphs.run(bool(compute_stress))
        else:
            self._step(compute_stress)

    def segment_energies(self, natoms):
        """Raw energies of the systems of a disjoint batch (contiguous node ranges of sizes
        ``natoms``), each the same device sum over its nodes as a single system's energy
        (Backbone.energy_batch, model.py:241-247); call after ``run``."""
        natoms = tuple(int(n) for n in natoms)
        if sum(natoms) != self.N or min(natoms, default=1) < 0:
            raise ValueError("natoms do not add up to the node count")
        ptr = getattr(self, "_seg_ptr", None)
        if ptr is None or ptr[0] != natoms:
            offs = [0]
            for n in natoms:
                offs.append(offs[-1] + n)
            self._seg_ptr = ptr = (natoms, torch.tensor(offs, dtype=torch.int32,
                                                        device=self.device))
        out = torch.empty(len(natoms), device=self.device, dtype=torch.float32)
        nat.segment_sum(self.node_e.view(-1), ptr[1], out)
        return out

    def __call__(self, pos, compute_stress=False):
        self.run(pos, compute_stress)
        E = float(self.energy_buf.item())
        F = self.forces.clone()
        if not torch.as_tensor(pos).is_cuda:
            F = F.cpu()
        if compute_stress:
            V = self.virial_buf.reshape(3, 3).clone()
            return E, F, (V if torch.as_tensor(pos).is_cuda else V.cpu())
        return E, F
