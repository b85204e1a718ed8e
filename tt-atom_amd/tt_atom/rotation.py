"""Per-op entry points of the reference's rotation module (rotation.py:188-270) over fp32
torch tensors on the device: the packed-coefficient bookkeeping (``pack``, ``gather_coef``,
``scatter_coef``; torch indexing on whatever device the tensors are on) and the rotation by a
per-edge matrix of fixed sparsity with its VJP (``rotate``, ``rotate_bw``), which run the
sparse-pattern HIP kernels of csrc/pattern.hip.

The signatures are the reference's; its ``ttnn`` and ``device`` arguments are accepted and not
used (the tensors carry their device), and the tensors are row-major fp32 instead of tiled
bf16.  The fused step (tt_atom.trace) does not go through here: it runs the gather, rotation and
radial product of the message block as one kernel (tta_gather_rotate).  Shapes the kernels do
not take (more than 64 coefficient blocks on a side, more than 512 nonzeros) raise
RuntimeError, as the reference does for shapes its kernel cannot run (rotation.py:97-102).
"""
from __future__ import annotations

import torch

from . import _native as nat

__all__ = ["gather_coef", "pack", "rotate", "rotate_bw", "scatter_coef"]

_MAX_BLOCKS, _MAX_NNZ = 64, 512


def gather_coef(wigner: torch.Tensor, ii: torch.Tensor, jj: torch.Tensor):
    """The packed coefficients ``[E, nnz]`` of ``wigner`` ``[E, n_out, n_in]`` at a known pattern
    ``(ii, jj)`` (rotation.py:188-193): ``wigner[:, ii, jj]``, the same values ``pack`` returns."""
    return wigner[:, ii, jj].contiguous()


def pack(wigner: torch.Tensor, tol: float = 1e-6):
    """``[E, n_out, n_in]`` -> (``ij``: the structural nonzeros as (out, in) pairs in row-major
    order, ``coef`` ``[E, nnz]``) (rotation.py:196-208).  An entry is structural when its
    magnitude exceeds ``tol`` on some edge; dropping the others is exact for this topology."""
    nz = (wigner.abs().amax(dim=0) > tol).nonzero(as_tuple=False)
    ij = [(int(i), int(j)) for i, j in nz.tolist()]
    return ij, wigner[:, nz[:, 0], nz[:, 1]].contiguous()


def scatter_coef(g_coef: torch.Tensor, ij, n_out: int, n_in: int = None) -> torch.Tensor:
    """``[E, nnz]`` coefficient adjoints -> dense ``[E, n_out, n_in]`` with zeros off the pattern
    (rotation.py:263-270)."""
    n_in = n_out if n_in is None else n_in
    out = torch.zeros(g_coef.shape[0], n_out, n_in, dtype=g_coef.dtype, device=g_coef.device)
    if ij:
        ii = torch.tensor([i for i, _ in ij], device=g_coef.device)
        jj = torch.tensor([j for _, j in ij], device=g_coef.device)
        out[:, ii, jj] = g_coef
    return out


def _grouped(ij, n_rows, by_out):
    """The pattern grouped by output row (``by_out``) or input column: (ptr, k, other side)."""
    key = (lambda p: p[1][0]) if by_out else (lambda p: p[1][1])
    order = sorted(enumerate(ij), key=key)           # stable: pattern order within a group
    ptr = [0] * (n_rows + 1)
    for _, (i, j) in order:
        ptr[(i if by_out else j) + 1] += 1
    for r in range(n_rows):
        ptr[r + 1] += ptr[r]
    k = [q for q, _ in order]
    other = [(j if by_out else i) for _, (i, j) in order]
    return ptr, k, other


def _check(name, x, coef, ij, n_in, n_out, W):
    if len(ij) > _MAX_NNZ or n_in > _MAX_BLOCKS or n_out > _MAX_BLOCKS:
        raise RuntimeError(f"{name}: unsupported shape (n_in={n_in}, n_out={n_out}, "
                           f"nnz={len(ij)}; at most {_MAX_BLOCKS} blocks a side, {_MAX_NNZ} "
                           "nonzeros)")
    for i, j in ij:
        if not (0 <= i < n_out and 0 <= j < n_in):
            raise RuntimeError(f"{name}: pattern entry ({i}, {j}) outside [{n_out}, {n_in}]")
    E = x.shape[0]
    if x.dim() != 2 or x.shape[1] != n_in * W:
        raise RuntimeError(f"{name}: expected [E, {n_in * W}] input, got {tuple(x.shape)}")
    if coef.shape != (E, len(ij)):
        raise RuntimeError(f"{name}: coef must be [{E}, {len(ij)}], got {tuple(coef.shape)}")
    return E


def rotate(ttnn, x_flat, ij, coef, n_in, W, device=None, n_out=None):
    """``x_flat`` ``[E, n_in*W]`` -> ``[E, n_out*W]``: each edge's W-channel blocks multiplied by
    its packed matrix, out block i = sum over pattern pairs (i, j) of coef[:, k] x block j
    (rotation.py:211-222).  ``n_out`` defaults to ``n_in``."""
    n_out = n_in if n_out is None else n_out
    E = _check("rotate", x_flat, coef, ij, n_in, n_out, W)
    ptr, k, blk = _grouped(ij, n_out, by_out=True)
    out = torch.empty(E, n_out * W, device=x_flat.device, dtype=torch.float32)
    nat.rotate_pattern(x_flat.contiguous(), coef.contiguous(), out, ptr, k, blk, E=E, n_in=n_in,
                       n_out=n_out, W=W)
    return out


def rotate_bw(ttnn, x_in_flat, g_out_flat, ij, coef, n_in, W, device=None, n_out=None):
    """VJP of :func:`rotate` (rotation.py:225-260): (adjoint of ``x_in`` ``[E, n_in*W]``, adjoint
    of the packed coefficients ``[E, nnz]``).  The input adjoint is the same rotation with the
    pattern grouped by input block; the coefficient adjoint is gc[:, k] = sum over channels of
    g_out block i times x_in block j for pair k = (i, j)."""
    n_out = n_in if n_out is None else n_out
    E = _check("rotate_bw", x_in_flat, coef, ij, n_in, n_out, W)
    if g_out_flat.shape != (E, n_out * W):
        raise RuntimeError(f"rotate_bw: g_out must be [{E}, {n_out * W}]")
    ptr, k, blk = _grouped(ij, n_in, by_out=False)
    g_out = g_out_flat.contiguous()
    g_in = torch.empty(E, n_in * W, device=g_out.device, dtype=torch.float32)
    nat.rotate_pattern(g_out, coef.contiguous(), g_in, ptr, k, blk, E=E, n_in=n_out, n_out=n_in,
                       W=W)
    gc = torch.empty(E, len(ij), device=g_out.device, dtype=torch.float32)
    nat.rotate_pattern_gc(g_out, x_in_flat.contiguous(), gc, [i for i, _ in ij],
                          [j for _, j in ij], E=E, n_in=n_in, n_out=n_out, W=W)
    return g_in, gc
