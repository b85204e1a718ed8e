"""Isolated edgewise step (the C2 workload): gather source node features, rotate into the edge
frame, one SO(2) convolution, rotate back, scatter-add to destinations -- and the VJP of that map
with respect to the edge vectors.

This is the message-passing core of the reference's ``Edgewise`` block (edgewise.py:52-86:
gather, ``rotation.rotate`` / fused_rotate, ``SO2Convolution``, inverse rotate, segment sum)
without the radial MLP, gate and envelope, with the backward of forces.py:352-418 restricted to
the rotation (Wigner) adjoint and closed by the Wigner VJP of geometry.py:87-155.  Kernels:
``tta_edge_wigner``, ``tta_gather_rotate_src``, split / fp32 GEMMs on the fused
``[[Wa, Wb], [-Wb, Wa]]`` blocks, ``tta_rotate_env_segsum``; backward
``tta_rotate_env_segsum_bw``, transposed GEMMs, ``tta_gather_rotate_src_bw``,
``tta_edge_geometry_bwd``.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _native as nat
from .model import PRECISIONS, SO2Weights


class EdgewiseStep:
    """``EdgewiseStep(weights, prefix, jd, src, tgt, num_nodes, C, device, precision)``;
    ``out, g_ev = step(x, ev, g_out)`` with x [N, 9, C], ev [E, 3] (reference edge order),
    g_out [N, 9, C] the upstream adjoint of the scattered output."""

    def __init__(self, weights, prefix, jd, src, tgt, num_nodes, C=128, device="cuda",
                 precision="f32", gamma=0.0):
        nat.load()
        if precision not in PRECISIONS:
            raise RuntimeError(f"precision must be one of {sorted(PRECISIONS)}")
        dev = torch.device(device)
        self.dev, self.C, self.N, self.gamma = dev, int(C), int(num_nodes), float(gamma)
        self.so2 = SO2Weights(weights, prefix, dev, self.C, self.C, 0, 0, PRECISIONS[precision])
        self.jd = torch.cat([torch.as_tensor(j, dtype=torch.float32).reshape(-1) for j in jd]).to(dev)
        s = torch.as_tensor(src).to("cpu", torch.int64).numpy()
        t = torch.as_tensor(tgt).to("cpu", torch.int64).numpy()
        E = int(s.shape[0])
        if E and (min(s.min(), t.min()) < 0 or max(s.max(), t.max()) >= self.N):
            raise ValueError("edge index out of range")
        order = np.argsort(t, kind="stable")
        self.order = torch.from_numpy(order).to(dev)
        self.inv_order = torch.from_numpy(np.argsort(order, kind="stable")).to(dev)
        ptr = np.zeros(self.N + 1, np.int64)
        ptr[1:] = np.cumsum(np.bincount(t[order], minlength=self.N))
        i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).to(dev)
        self.src, self.tgt, self.tgt_ptr = i32(s[order]), i32(t[order]), i32(ptr)
        self.E = E
        f = lambda *shape: torch.empty(*shape, device=dev, dtype=torch.float32)
        C = self.C
        self.zero_idx = torch.zeros(E, dtype=torch.int32, device=dev)
        self.origin = torch.zeros(1, 3, device=dev)
        self.ev, self.dist, self.coef = f(E, 3), f(E), f(E, 35)
        self.env = torch.ones(E, device=dev)
        self.xe, self.ms, self.out = f(E, 9 * C), f(E, 9 * C), f(self.N, 9, C)
        self.g_m, self.g_xe = f(E, 9 * C), f(E, 9 * C)
        self.g_coef, self.g_env, self.g_ev = f(E, 35), f(E), f(E, 3)

    def forward(self, x, ev_sorted):
        C = self.C
        # ev = pos[0] - pos[0] + shift: the Wigner kernel reads the edge vector from the shift
        nat.edge_wigner(self.origin, self.zero_idx, self.zero_idx, ev_sorted, self.jd, self.gamma,
                        self.ev, self.dist, self.coef)
        nat.gather_rotate_src(x, self.src, self.coef, self.xe.view(self.E, 9, C))
        s = self.so2
        nat.linear_group([(self.xe[:, :3 * C], s.wm0_t, s.bm0, self.ms[:, :3 * C]),
                          (self.xe[:, 3 * C:7 * C], s.w1, None, self.ms[:, 3 * C:7 * C]),
                          (self.xe[:, 7 * C:], s.w2, None, self.ms[:, 7 * C:])])
        nat.rotate_env_segsum(self.ms.view(self.E, 9, C), self.coef, self.env, self.tgt_ptr, None,
                              self.out, n_in=9, env_first=True, div=1.0)
        return self.out

    def backward(self, x, g_out):
        C = self.C
        nat.fill(self.g_coef, 0.0)
        nat.fill(self.g_env, 0.0)
        nat.rotate_env_segsum_bw(g_out, self.tgt, self.ms.view(self.E, 9, C), self.coef, self.env,
                                 self.g_m.view(self.E, 9, C), self.g_coef, self.g_env, n_in=9,
                                 env_first=True, div=1.0)
        s = self.so2
        nat.linear_group([(self.g_m[:, :3 * C], s.wm0, None, self.g_xe[:, :3 * C]),
                          (self.g_m[:, 3 * C:7 * C], s.w1_t, None, self.g_xe[:, 3 * C:7 * C]),
                          (self.g_m[:, 7 * C:], s.w2_t, None, self.g_xe[:, 7 * C:])])
        nat.gather_rotate_src_bw(self.g_xe.view(self.E, 9, C), x, self.src, self.coef, None,
                                 self.g_coef)
        nat.edge_geometry_bwd(self.ev, self.dist, self.g_coef, None, None, 0, None, 0.0, 1.0, 0,
                              self.jd, self.gamma, self.g_ev)
        return self.g_ev

    def __call__(self, x, ev, g_out):
        """Reference edge order in and out: ev [E, 3] -> (out [N, 9, C], g_ev [E, 3])."""
        x = torch.as_tensor(x, dtype=torch.float32).to(self.dev).contiguous()
        ev_s = torch.as_tensor(ev, dtype=torch.float32).to(self.dev)[self.order].contiguous()
        g = torch.as_tensor(g_out, dtype=torch.float32).to(self.dev).contiguous()
        out = self.forward(x, ev_s)
        g_ev = self.backward(x, g)
        return out, g_ev[self.inv_order]
