"""ctypes boundary to ``libttatom_hip.so`` (the C ABI declared in ``include/tt_atom_hip.h``).

Every wrapper takes torch tensors that live on the current HIP device, checks dtype / size /
contiguity on the host, passes raw device pointers plus the current torch stream, and raises
``RuntimeError`` with the library's message on a non-zero status.  There is no fallback: if
the library is missing or the device is not a gfx950 the call fails loudly.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libttatom_hip.so"

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double


class GemmProblem(ctypes.Structure):
    """tta_gemm_problem (include/tt_atom_hip_types.h): one product of a grouped GEMM launch."""
    _fields_ = [("A", _P), ("B", _P), ("C", _P), ("bias", _P), ("C2", _P), ("aux", _P),
                ("M", _I64), ("N", _I64), ("K", _I64), ("lda", _I64), ("ldb", _I64),
                ("ldc", _I64), ("epilogue", _I64)]


class CellGrid(ctypes.Structure):
    """tta_cell_grid (include/tt_atom_hip_types.h): bins of the cell-list neighbour search."""
    _fields_ = [("origin", _F * 3), ("inv_h", _F), ("dims", _I * 3)]


# name -> argtypes (all return int status unless listed in _RESTYPE)
_SIGS = {
    "tta_version": [],
    "tta_last_error": [],
    "tta_check_device": [ctypes.c_char_p, _I64],
    "tta_gemm_f32": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                     _I64, _I64, _I64, _I, _P],
    "tta_gather_rotate": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_gather_rotate_bw_dst": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_node_gather_sum_dst": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_gather_rotate_bw_srcwalk": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_gather_rotate_bw_tgtwalk": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                     _I64, _P],
    "tta_gather_rotate_bw": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_rotate_env_segsum": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _F, _P],
    "tta_rotate_env_segsum_bw": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _F,
                                 _P],
    "tta_node_gather_sum": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_gate_fwd": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P],
    "tta_gate_bwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P],
    "tta_gate_gating_bwd": [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P],
    "tta_rotate_pattern": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P],
    "tta_rotate_pattern_gc": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P],
    "tta_segment_sum_table": [_P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "tta_ln_silu_fwd": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P],
    "tta_ln_silu_bwd": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P],
    "tta_rmsnorm_sh_fwd": [_P, _P, _P, _P, _P, _P, _I64, _I64, _F, _P],
    "tta_rmsnorm_sh_bwd": [_P, _P, _P, _P, _P, _P, _I64, _I64, _P],
    "tta_silu_bwd": [_P, _P, _P, _I64, _P],
    "tta_sum": [_P, _I64, _I64, _P, _P],
    "tta_fill": [_P, _I64, _F, _P],
    "tta_edge_wigner": [_P, _P, _P, _P, _P, _F, _P, _P, _P, _I64, _I64, _P],
    "tta_edge_geometry_fwd": [_P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _F, _F, _I64, _I64,
                              _P, _P, _P, _P, _P, _I64, _I64, _P],
    "tta_edge_features": [_P, _P, _P, _P, _P, _P, _F, _F, _I64, _I64, _P, _P, _I64, _P],
    "tta_edge_geometry_bwd": [_P, _P, _P, _P, _P, _I64, _P, _F, _F, _I64, _P, _F, _P, _I64, _P],
    "tta_node_forces": [_P, _P, _P, _P, _P, _I64, _I64, _P],
    "tta_virial": [_P, _P, _I64, _P, _P, _P],
    "tta_virial_noalloc": [_P, _P, _I64, _P, _P],
    "tta_spectral_block_fwd": [_P] * 18 + [_I64, _I64, _I64, _F, _P],
    "tta_spectral_block_bwd": [_P] * 14 + [_I64, _I64, _I64, _P],
    "tta_energy_head_fwd": [_P] * 10 + [_I64, _I64, _I64, _P],
    "tta_energy_head_bwd": [_P] * 6 + [_I64, _I64, _I64, _P],
    "tta_segment_sum": [_P, _P, _I64, _P, _P],
    "tta_gemm_f32_gather": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64,
                            _P, _P, _I64, _I64, _I, _P],
    "tta_orb_edge_features": [_P, _P, _P, _P, _F, _I64, _P, _P, _P, _I64, _I64, _P],
    "tta_orb_edge_features_bwd": [_P, _P, _P, _F, _I64, _P, _I64, _P],
    "tta_rms_residual": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _F, _P],
    "tta_rms_bwd": [_P, _P, _P, _P, _P, _I64, _I64, _P],
    "tta_orb_segsum": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_orb_edge_bwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                         _P],
    "tta_orb_node_segsum2": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_segment_mean": [_P, _P, _P, _I64, _I64, _P],
    "tta_segment_mean_bwd": [_P, _P, _P, _P, _I64, _I64, _P],
    "tta_segment_center": [_P, _P, _P, _I64, _I64, _P],
    "tta_add_rows": [_P, _I64, _P, _I64, _I64, _I64, _P],
    "tta_gather_rotate_src": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_gather_rotate_src_bw": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "tta_pack_b_elems": [_I64, _I64, _I],
    "tta_pack_b": [_P, _I64, _I64, _I64, _I, _P, _I64, _P],
    "tta_gemm_bf16x": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P, _I64, _P, _P,
                       _I64, _I64, _I, _P],
    "tta_gemm_bf16x_group": [ctypes.POINTER(GemmProblem), _I64, _I, _P],
    "tta_gemm_f32_group": [ctypes.POINTER(GemmProblem), _I64, _P],
    "tta_gemm_f32_splitk_work": [ctypes.POINTER(GemmProblem), _I64],
    "tta_gemm_bf16x_splitk_work": [ctypes.POINTER(GemmProblem), _I64],
    "tta_gemm_bf16x_group_splitk": [ctypes.POINTER(GemmProblem), _I64, _I, _P, _I64, _P],
    "tta_gemm_bf16x_group_gate": [ctypes.POINTER(GemmProblem), _I64, _I, _P, _P, _I64, _P, _I64,
                                  _I64, _P, _P, _I64, _P],
    "tta_gemm_bf16x_group_gate_bwd": [ctypes.POINTER(GemmProblem), _I64, _I, _P, _P, _I64, _P,
                                      _I64, _I64, _P, _P, _I64, _P],
    "tta_gemm_f32_group_splitk": [ctypes.POINTER(GemmProblem), _I64, _P, _I64, _P],
    "tta_radius_graph_thresholds": [_P, _I64, _P, _P, _P, _I64, _P, _P, _I, _D, _F, _F, _I, _P,
                                    _P, _P, _P, _P],
    "tta_radius_graph_count": [_P, _I64, _P, _P, _P, _I64, _P, _P, _I, _D, _F, _F, _P, _P, _P,
                               _P, _P],
    "tta_radius_graph_write": [_P, _I64, _P, _P, _P, _I64, _P, _P, _I, _D, _F, _F, _P, _P, _P,
                               _P, _P, _P, _P, _P],
    "tta_cell_list_workspace": [_I64, _I64],
    "tta_cell_list_build": [_P, _I64, _P, _I64, _I, ctypes.POINTER(CellGrid), _P, _P, _P, _P],
    "tta_radius_graph_cells_thresholds": [_P, _I64, _P, _I64, _I, ctypes.POINTER(CellGrid), _P,
                                          _P, _D, _F, _F, _I, _P, _P, _P, _P],
    "tta_radius_graph_cells_count": [_P, _I64, _P, _I64, _I, ctypes.POINTER(CellGrid), _P, _P,
                                     _D, _F, _F, _P, _P, _P, _P, _P],
    "tta_radius_graph_cells_write": [_P, _I64, _P, _I64, _I, ctypes.POINTER(CellGrid), _P, _P,
                                     _D, _F, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P],
}
_RESTYPE = {"tta_last_error": ctypes.c_char_p, "tta_pack_b_elems": ctypes.c_int64,
            "tta_cell_list_workspace": ctypes.c_int64, "tta_gemm_f32_splitk_work": ctypes.c_int64,
            "tta_gemm_bf16x_splitk_work": ctypes.c_int64}

EXPORTS = tuple(_SIGS)

_lib = None


def load(require_device=True):
    """Load the library (once).  torch's HIP runtime is initialised first so the library binds to
    that already-loaded runtime (same SONAME) and torch streams are valid handles for it."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python __graft_entry__.py` "
                           "(build()) or `make -C tt-atom_amd/csrc`")
    if require_device:
        if not torch.cuda.is_available():
            raise RuntimeError("tt_atom (MI355X build) needs a HIP device; none is visible")
        torch.cuda.init()
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    if require_device:
        buf = ctypes.create_string_buffer(64)
        if lib.tta_check_device(buf, 64) != 0:
            raise RuntimeError(lib.tta_last_error().decode())
    _lib = lib
    return lib


def load_symbols_only():
    """Load without touching a device (CPU tests: symbol / ABI checks only)."""
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    return lib


def _call(name, *args):
    lib = load()
    st = getattr(lib, name)(*args)
    if st != 0:
        raise RuntimeError(f"{name}: {lib.tta_last_error().decode()}")


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t, dtype=torch.float32, numel=None, name="tensor", contiguous=True):
    if t is None:
        return None
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype}, got {t.dtype}")
    if contiguous and not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if numel is not None and t.numel() != numel:
        raise RuntimeError(f"{name} has {t.numel()} elements, expected {numel}")
    return t.data_ptr()


def _i32(t, numel=None, name="index"):
    return _ptr(t, torch.int32, numel, name)


def _host_idx8(idx, name="idx8"):
    """The 8-entry gate index table as host memory (the entry points read it on the host while
    they build the launch): a sequence of ints or a tensor (a device tensor is copied back, so
    pass a sequence inside a graph capture)."""
    vals = idx.tolist() if isinstance(idx, torch.Tensor) else list(idx)
    if len(vals) != 8:
        raise RuntimeError(f"{name} must have 8 entries, got {len(vals)}")
    return (ctypes.c_int * 8)(*(int(v) for v in vals))


def _rows(t, rows, ld, width, name="tensor"):
    """Pointer of a row-strided fp32 view; checks that rows x width at stride ld stay inside the
    tensor's storage (the kernels index ptr[r * ld + c] for r < rows, c < width)."""
    if not t.is_cuda or t.dtype != torch.float32:
        raise RuntimeError(f"{name} must be an fp32 device tensor")
    if rows == 0:
        return t.data_ptr()
    need = t.storage_offset() + (rows - 1) * ld + width
    if ld < width or need * 4 > t.untyped_storage().nbytes():
        raise RuntimeError(f"{name}: {rows} rows of {width} at stride {ld} exceed its storage")
    return t.data_ptr()


# ----------------------------------------------------------------------------- GEMM
EPI_STORE, EPI_SILU, EPI_ACCUM, EPI_PRE_SILU, EPI_SILU_GRAD = 0, 1, 2, 3, 4
EPI_SIGMOID = 5
EPI_GATE, EPI_GATE_BWD = 6, 7  # tta_gemm_bf16x_group_gate / _gate_bwd only

# Optional measurement hook: when set, every GEMM launch is bracketed by
# ``probe.before(flops, nbytes, kind)`` and ``probe.after()`` (the benchmark records HIP events on
# the launch stream there).  nbytes is the algorithmic traffic: A, B and C once (C twice when
# accumulated, plus the second output / auxiliary input of epilogues 3 and 4); kind is "f32" for
# the fp32 MFMA kernel and MODE_KIND[mode] for the split kernel.  The gated SO(2) launches pass
# ``part="gate"`` as well (a probe may file them separately within their family).
_gemm_probe = None


def set_gemm_probe(probe):
    global _gemm_probe
    _gemm_probe = probe


def _span(t, name, rows, ld, width, batch=1, stride=0):
    """Checks that an fp32 device tensor's storage holds rows x width at row stride ld, for
    `batch` copies `stride` elements apart, starting at the tensor's own offset."""
    if t is None:
        return
    if not t.is_cuda or t.dtype != torch.float32:
        raise RuntimeError(f"gemm: {name} must be an fp32 device tensor")
    if rows <= 0 or width <= 0 or batch <= 0:
        return
    need = t.storage_offset() + (batch - 1) * stride + (rows - 1) * ld + width
    if ld < 0 or stride < 0 or need * 4 > t.untyped_storage().nbytes():
        raise RuntimeError(f"gemm: {name} is too small for {batch} x {rows} x {width} at row "
                           f"stride {ld} (batch stride {stride})")


def gemm(A, B, C, *, M, N, K, lda, ldb, ldc, bias=None, epilogue=EPI_STORE, C2=None, aux=None,
         batch=1, sA=0, sB=0, sC=0, sBias=0):
    """C = epi(A @ B + bias) on raw strided views (A/B/C are base tensors; offsets are applied
    by the caller through ``narrow``/slicing of contiguous storage -> data_ptr)."""
    # every operand must hold its whole strided extent: the kernel indexes C2 and aux with C's
    # row stride and batch stride
    _span(A, "A", M, lda, K, batch, sA)
    _span(B, "B", K, ldb, N, batch, sB)
    _span(C, "C", M, ldc, N, batch, sC)
    _span(C2, "C2", M, ldc, N, batch, sC)
    _span(aux, "aux", M, ldc, N, batch, sC)
    _span(bias, "bias", 1, N, N, batch, sBias)
    probe = _gemm_probe
    if probe is not None:
        c_passes = 1 + (epilogue in (EPI_ACCUM, EPI_PRE_SILU, EPI_SILU_GRAD))
        nbytes = 4.0 * (M * K * (batch if sA else 1) + K * N * (batch if sB else 1)
                        + c_passes * M * N * batch)
        probe.before(2.0 * M * N * K * batch, nbytes, "f32")
    _call("tta_gemm_f32", A.data_ptr(), B.data_ptr(), C.data_ptr(),
          None if bias is None else bias.data_ptr(), None if C2 is None else C2.data_ptr(),
          None if aux is None else aux.data_ptr(), M, N, K, lda, ldb, ldc, batch, sA, sB, sC,
          sBias, epilogue, _stream())
    if probe is not None:
        probe.after()


# Split MFMA GEMM modes (tta_gemm_bf16x): 6 = fp32-accurate with three bf16 planes per operand
# (six products), 16 = fp32-accurate with two power-of-two-scaled fp16 planes per operand (three
# products), 3 = two bf16 planes / three products, 1 = bf16 operands.
SPLIT_F32, SPLIT_F16X3, SPLIT_3, SPLIT_BF16 = 6, 16, 3, 1
# kernel-family name per mode, as the measurement hook reports it
MODE_KIND = {6: "bf16x6", 16: "f16x3", 3: "bf16x3", 1: "bf16x1"}
# mode-16 products that tta_gemm_bf16x(_group) runs on its short-K panel kernel (K <= 128, one
# 32-wide k-slab count for the whole group, plain or SiLU epilogue, no row gathers, at least 128
# columns, 16-byte aligned rows and operands, ldc < 2^22) are reported as their own family
PANEL_KIND = "f16x3-panel"


def _panel_item(M, N, K, ldc, epilogue, ptrs, gather=False):
    al = all(q is None or q % 16 == 0 for q in ptrs)
    return (K <= 128 and epilogue in (EPI_STORE, EPI_SILU) and not gather and N >= 128
            and N % 4 == 0 and ldc % 4 == 0 and ldc < (1 << 22) and al)


class PackedWeight:
    """A constant GEMM operand w_t [K, N] (fp32, row-major) plus its bf16-plane packing for the
    split kernel (``mode`` 6, 16, 3 or 1; None keeps only the fp32 matrix for the fp32-MFMA
    kernel).  ``shape`` / ``T``-free: it stands wherever a [K, N] weight is passed to linear()."""

    def __init__(self, w_t, mode=SPLIT_F32):
        if w_t.dim() != 2 or w_t.dtype != torch.float32 or not w_t.is_cuda:
            raise RuntimeError("PackedWeight: w_t must be a 2-D fp32 device tensor")
        self.w_t = w_t
        self.mode = mode
        self.packed = None
        K, N = w_t.shape
        if mode is not None and K % 4 == 0:
            n = load().tta_pack_b_elems(K, N, mode)
            self.packed = torch.empty(n, dtype=torch.int16, device=w_t.device)
            _call("tta_pack_b", _ptr(w_t, name="w_t", contiguous=False), K, N, _ld(w_t, "w_t"),
                  mode, self.packed.data_ptr(), n, _stream())

    @property
    def shape(self):
        return self.w_t.shape


def _same_rows(out, out2, aux, where):
    """out2 and aux are written / read at out's row stride by the GEMM epilogues."""
    ldc = _ld(out, "out")
    for t, nm in ((out2, "out2"), (aux, "aux")):
        if t is not None and (t.shape != out.shape or _ld(t, nm) != ldc):
            raise RuntimeError(f"{where}: {nm} must have out's shape and row stride")


def _gemm_bf16x(x, pw, out, bias, epilogue, out2, aux, P=None, idx0=None, idx1=None, off1=0):
    M, K = x.shape
    N = pw.w_t.shape[1]
    _same_rows(out, out2, aux, "linear")
    _span(x, "x", M, _ld(x, "x"), K)
    for t, nm in ((out, "out"), (out2, "out2"), (aux, "aux")):
        _span(t, nm, M, _ld(out, "out"), N)
    probe = _gemm_probe
    if probe is not None:
        c_passes = 1 + (epilogue in (EPI_ACCUM, EPI_PRE_SILU, EPI_SILU_GRAD)) + (2 if P is not None else 0)
        panel = pw.mode == 16 and _panel_item(
            M, N, K, _ld(out, "out"), epilogue,
            [out.data_ptr(), None if bias is None else bias.data_ptr()], gather=P is not None)
        probe.before(2.0 * M * N * K, 4.0 * (M * K + K * N + c_passes * M * N),
                     PANEL_KIND if panel else MODE_KIND[pw.mode])
    _call("tta_gemm_bf16x", x.data_ptr(), pw.packed.data_ptr(), out.data_ptr(),
          None if bias is None else _ptr(bias, numel=N, name="bias"),
          None if out2 is None else out2.data_ptr(), None if aux is None else aux.data_ptr(),
          M, N, K, _ld(x, "x"), _ld(out, "out"), pw.mode,
          None if P is None else _ptr(P, name="P"), 0 if P is None else _ld(P, "P"),
          None if idx0 is None else _i32(idx0, M), None if idx1 is None else _i32(idx1, M),
          off1, 0 if P is None else P.shape[0], epilogue, _stream())
    if probe is not None:
        probe.after()


def _split_ok(x, pw, min_rows=4096):
    """The split kernel (128 x 128 x 32 tiles) runs edge-level GEMMs; short-K or small-M
    products stay on the fp32 MFMA kernel, whose smaller tiles fill the chip better there
    (small-M products of packed weights may take the split kernel's split-K form instead:
    ``_small_split``)."""
    M, K = x.shape
    return (isinstance(pw, PackedWeight) and pw.packed is not None and M >= min_rows
            and K >= 128 and K % 4 == 0 and x.data_ptr() % 16 == 0 and _ld(x, "x") % 4 == 0
            and _ld(x, "x") < (1 << 21))


def _fp32_tiles(shapes):
    return sum(-(-M // 32) * -(-N // 64) for M, N in shapes)


def _small_split(items):
    """items = [(x, PackedWeight, bias, out, epilogue, out2, aux)] of products with M < 4096:
    the split kernel's split-K launch (tta_gemm_bf16x_group_splitk) when the fp32 kernel would run
    them unsplit at its matrix rate (160 or more of its 32 x 64 tiles in all: its split-K form
    takes smaller launches) and the split kernel's rule splits them.  Returns False, having
    launched nothing, otherwise."""
    if not all(isinstance(w, PackedWeight) and w.packed is not None and w.mode == items[0][1].mode
               and x.shape[0] < 4096 and x.shape[1] >= 256 and _split_ok(x, w, min_rows=1)
               for x, w, *_ in items):
        return False
    if _fp32_tiles([(x.shape[0], w.shape[1]) for x, w, *_ in items]) < 160:
        return False
    probs = (GemmProblem * len(items))()
    flops = nbytes = 0.0
    for i, (x, w, bias, out, epi, out2, aux) in enumerate(items):
        M, K = x.shape
        N = w.shape[1]
        ldc = _ld(out, "out")
        probs[i] = GemmProblem(
            _rows(x, M, _ld(x, "x"), K, "x"), w.packed.data_ptr(), _rows(out, M, ldc, N, "out"),
            None if bias is None else _ptr(bias, numel=N, name="bias"),
            None if out2 is None else _rows(out2, M, _ld(out2, "out2"), N, "out2"),
            None if aux is None else _rows(aux, M, _ld(aux, "aux"), N, "aux"),
            M, N, K, _ld(x, "x"), 0, ldc, epi)
        flops += 2.0 * M * N * K
        nbytes += 4.0 * (M * K + K * N + (1 + (epi in (EPI_ACCUM, EPI_PRE_SILU, EPI_SILU_GRAD)))
                         * M * N)
    need = load().tta_gemm_bf16x_splitk_work(probs, len(items))
    if need < 0:
        raise RuntimeError("tta_gemm_bf16x_splitk_work: bad product list")
    if need == 0:
        return False
    work = torch.empty(need, device=items[0][0].device, dtype=torch.float32)
    probe = _gemm_probe
    if probe is not None:
        probe.before(flops, nbytes, MODE_KIND[items[0][1].mode])
    _call("tta_gemm_bf16x_group_splitk", probs, len(items), items[0][1].mode, work.data_ptr(),
          work.numel(), _stream())
    if probe is not None:
        probe.after()
    return True


def linear_group_gate(items, c0, sig, x0, idx8, H, backward=False):
    """The coefficient products of an SO(2) convolution with its gate applied as they are
    written (tta_gemm_bf16x_group_gate): ``items`` = [(x, PackedWeight, bias, out)], product i's
    columns being coefficients c0[i], c0[i] + 1, ... of H channels each; ``sig`` [M, L * H]
    the sigmoid of the convolution's gating columns (any row stride; linear() with
    EPI_SIGMOID), ``x0`` [M, H] receives coefficient 0's pre-activation.  ``backward``: the
    adjoint products with the gate's input adjoint applied instead
    (tta_gemm_bf16x_group_gate_bwd; x0 is read).  Launches with fewer than 4096 rows take the
    split-K form when the library's rule splits them."""
    if not items or len(items) > MAX_GROUP or len(c0) != len(items):
        raise RuntimeError("linear_group_gate: 1..8 products, one first coefficient each")
    mode = items[0][1].mode
    probs = (GemmProblem * len(items))()
    flops = nbytes = 0.0
    L = max(_host_idx8(idx8)) + 1
    M = items[0][0].shape[0]
    for i, (x, w, bias, out) in enumerate(items):
        if not (isinstance(w, PackedWeight) and w.packed is not None and w.mode == mode
                and x.shape[1] % 4 == 0 and x.data_ptr() % 16 == 0 and _ld(x, "x") % 4 == 0
                and _ld(x, "x") < (1 << 21)):
            raise RuntimeError("linear_group_gate: every product needs a packed weight of one "
                               "mode and a 16-byte aligned x with K, row stride multiples of 4")
        Mi, K = x.shape
        N = w.shape[1]
        if Mi != M or K != w.shape[0] or out.shape != (M, N) or N % H:
            raise RuntimeError("linear_group_gate: shape mismatch")
        ldc = _ld(out, "out")
        probs[i] = GemmProblem(_rows(x, M, _ld(x, "x"), K, "x"), w.packed.data_ptr(),
                               _rows(out, M, ldc, N, "out"),
                               None if bias is None else _ptr(bias, numel=N, name="bias"),
                               None, None, M, N, K, _ld(x, "x"), 0, ldc,
                               EPI_GATE_BWD if backward else EPI_GATE)
        flops += 2.0 * M * N * K
        # A, B, the output and a gating sigmoid per gated output (coefficient 0: its x0 copy)
        nbytes += 4.0 * (M * K + K * N + 2 * M * N)
    gp = _rows(sig, M, _ld(sig, "sig"), L * H, "sig")
    xp = _rows(x0, M, _ld(x0, "x0"), H, "x0")
    work = None
    if M < 4096:
        need = load().tta_gemm_bf16x_splitk_work(probs, len(items))
        if need < 0:
            raise RuntimeError("tta_gemm_bf16x_splitk_work: bad product list")
        if need > 0:
            work = torch.empty(need, device=items[0][0].device, dtype=torch.float32)
    probe = _gemm_probe
    if probe is not None:
        probe.before(flops, nbytes, MODE_KIND[mode], part="gate")
    _call("tta_gemm_bf16x_group_gate_bwd" if backward else "tta_gemm_bf16x_group_gate", probs,
          len(items), mode,
          (ctypes.c_int64 * len(items))(*c0), gp, _ld(sig, "sig"), xp, _ld(x0, "x0"), H,
          _host_idx8(idx8), None if work is None else work.data_ptr(),
          0 if work is None else work.numel(), _stream())
    if probe is not None:
        probe.after()


def _gemm_f32_splitk(items):
    """items = [(x, w_t, bias, out, epilogue, out2, aux)] of fp32 row-major products: one
    tta_gemm_f32_group_splitk call (k chunks run as separate workgroups, then a reduction) with
    a workspace from the caching allocator, when the library's rule splits any of them (grids
    too small to fill the GPU, K >= 256).  Returns False, having launched nothing, otherwise."""
    probs = (GemmProblem * len(items))()
    flops = nbytes = 0.0
    for i, (x, w, bias, out, epi, out2, aux) in enumerate(items):
        M, K = x.shape
        N = w.shape[1]
        ldc = _ld(out, "out")
        probs[i] = GemmProblem(
            _rows(x, M, _ld(x, "x"), K, "x"), _rows(w, K, _ld(w, "w_t"), N, "w_t"),
            _rows(out, M, ldc, N, "out"),
            None if bias is None else _ptr(bias, numel=N, name="bias"),
            None if out2 is None else _rows(out2, M, _ld(out2, "out2"), N, "out2"),
            None if aux is None else _rows(aux, M, _ld(aux, "aux"), N, "aux"),
            M, N, K, _ld(x, "x"), _ld(w, "w_t"), ldc, epi)
        flops += 2.0 * M * N * K
        nbytes += 4.0 * (M * K + K * N + (1 + (epi in (EPI_ACCUM, EPI_PRE_SILU, EPI_SILU_GRAD)))
                         * M * N)
    need = load().tta_gemm_f32_splitk_work(probs, len(items))
    if need < 0:
        raise RuntimeError("tta_gemm_f32_splitk_work: bad product list")
    if need == 0:
        return False
    work = torch.empty(need, device=items[0][0].device, dtype=torch.float32)
    probe = _gemm_probe
    if probe is not None:
        probe.before(flops, nbytes, "f32")
    _call("tta_gemm_f32_group_splitk", probs, len(items), work.data_ptr(), work.numel(),
          _stream())
    if probe is not None:
        probe.after()
    return True


def linear(x, w_t, bias=None, out=None, epilogue=EPI_STORE, out2=None, aux=None):
    """y = x @ w_t (+ bias) for 2-D row-major x [M, K] (any row stride) and w_t [K, N] (a tensor
    or a PackedWeight; a packed weight runs on the split kernel when the shapes allow)."""
    M, K = x.shape
    K2, N = w_t.shape
    if K != K2:
        raise RuntimeError(f"linear: inner dims {K} vs {K2}")
    if out is None:
        out = torch.empty(M, N, device=x.device, dtype=torch.float32)
    _same_rows(out, out2, aux, "linear")
    if isinstance(w_t, PackedWeight):
        if _split_ok(x, w_t):
            _gemm_bf16x(x, w_t, out, bias, epilogue, out2, aux)
            return out
        if _small_split([(x, w_t, bias, out, epilogue, out2, aux)]):
            return out
        w_t = w_t.w_t
    if M < 4096 and K >= 256 and _gemm_f32_splitk([(x, w_t, bias, out, epilogue, out2, aux)]):
        return out
    gemm(x, w_t, out, M=M, N=N, K=K, lda=_ld(x, "x"), ldb=_ld(w_t, "w_t"), ldc=_ld(out, "out"),
         bias=bias, epilogue=epilogue, C2=out2, aux=aux)
    return out


MAX_GROUP = 8


def linear_group(items):
    """Several independent products y = x @ w_t (+ bias) in one launch: ``items`` = [(x, w_t,
    bias, out, epilogue, out2, aux)] (the last three optional).  All on the split kernel
    when every product qualifies for it (same plane mode), all on the fp32 kernel when none
    does; a mix runs one launch per product."""
    items = [tuple(it) + (EPI_STORE, None, None)[len(it) - 4:] for it in items]
    for x, w, bias, out, epi, out2, aux in items:
        if x.shape[1] != w.shape[0] or out.shape != (x.shape[0], w.shape[1]):
            raise RuntimeError("linear_group: shape mismatch")
        _same_rows(out, out2, aux, "linear_group")
    split = [isinstance(w, PackedWeight) and _split_ok(x, w) for x, w, *_ in items]
    modes = {w.mode for (x, w, *_), sp in zip(items, split) if sp}
    if len(items) > MAX_GROUP or (any(split) and not all(split)) or len(modes) > 1:
        for x, w, bias, out, epi, out2, aux in items:
            linear(x, w, bias, out, epi, out2, aux)
        return
    if not any(split) and _small_split(items):
        return
    if not split[0] and any(x.shape[1] >= 256 for x, *_ in items) and _gemm_f32_splitk(
            [(x, w.w_t if isinstance(w, PackedWeight) else w, *rest) for x, w, *rest in items]):
        return
    probs = (GemmProblem * len(items))()
    flops = nbytes = 0.0
    panel = split[0] and items[0][1].mode == 16 and len({(x.shape[1] + 31) // 32 for x, *_ in items}) == 1
    for x, w, bias, out, epi, out2, aux in items:
        panel = panel and _panel_item(x.shape[0], w.shape[1], x.shape[1], _ld(out, "out"), epi,
                                      [out.data_ptr(), None if bias is None else bias.data_ptr()])
    for i, (x, w, bias, out, epi, out2, aux) in enumerate(items):
        M, K = x.shape
        N = w.shape[1]
        wt = w if split[0] else (w.w_t if isinstance(w, PackedWeight) else w)
        ldc = _ld(out, "out")
        probs[i] = GemmProblem(
            _rows(x, M, _ld(x, "x"), K, "x"),
            wt.packed.data_ptr() if split[0] else _rows(wt, K, _ld(wt, "w_t"), N, "w_t"),
            _rows(out, M, ldc, N, "out"),
            None if bias is None else _ptr(bias, numel=N, name="bias"),
            None if out2 is None else _rows(out2, M, _ld(out2, "out2"), N, "out2"),
            None if aux is None else _rows(aux, M, _ld(aux, "aux"), N, "aux"),
            M, N, K, _ld(x, "x"), 0 if split[0] else _ld(wt, "w_t"), ldc, epi)

        c_passes = 1 + (epi in (EPI_ACCUM, EPI_PRE_SILU, EPI_SILU_GRAD))
        flops += 2.0 * M * N * K
        nbytes += 4.0 * (M * K + K * N + c_passes * M * N)
    probe = _gemm_probe
    if probe is not None:
        probe.before(flops, nbytes, (PANEL_KIND if panel else MODE_KIND[items[0][1].mode])
                     if split[0] else "f32")
    if split[0]:
        _call("tta_gemm_bf16x_group", probs, len(items), items[0][1].mode, _stream())
    else:
        _call("tta_gemm_f32_group", probs, len(items), _stream())
    if probe is not None:
        probe.after()


def _ld(t, name):
    """Leading dimension of a row-major 2-D view (strides of size-1 dims do not matter)."""
    if t.dim() != 2:
        raise RuntimeError(f"linear: {name} must be 2-D")
    if t.shape[1] > 1 and t.stride(1) != 1:
        raise RuntimeError(f"linear: {name} must be row-major")
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


# ----------------------------------------------------------------------------- rotation
# Optional measurement hook for the HBM-bound edge kernels: ``probe.before(kernel, nbytes,
# compulsory)`` / ``probe.after()`` around each launch.  nbytes = algorithmic bytes (every operand
# read or written once per use: gathered node rows count once per edge); compulsory = every
# distinct operand byte once (a gathered node tensor counts once), the least HBM traffic the
# launch can have.  They differ only for the kernels that gather node rows per edge or read an
# edge row twice.
_hbm_probe = None


def set_hbm_probe(probe):
    global _hbm_probe
    _hbm_probe = probe


def _pick_v(W):
    """Vector width of the rotation kernels for rows of W channels (pick_v in csrc/rotate.hip)."""
    return 4 if W >= 256 else 2 if W >= 128 else 1


def bw_walk_width_ok(C):
    """Whether the node walks of the rotation backward (gather_rotate_bw_dst / _nodes) take rows
    of C channels: every channel of a half in one lane vector of a wavefront, C / V <= 64 with
    C a multiple of 4, i.e. C <= 64, C = 128 or C = 256 (bw_walk_check in csrc/rotate.hip)."""
    return C > 0 and C % 4 == 0 and C // _pick_v(C) <= 64


def _tf(b):
    return "true" if b else "false"


def _al16(*ts):
    return all(t is None or t.data_ptr() % 16 == 0 for t in ts)


def _ln_variant(n, vec):
    """(G, NPL, VEC) of the LayerNorm-SiLU launch for rows of n (tta_ln_silu_fwd/_bwd)."""
    if n <= 32:
        return 32, 1, False
    if n <= 64:
        return 32, 2, False
    if n <= 128:
        return 16, 8, vec
    if n <= 256:
        return 64, 4, vec
    return 64, 8, False


def _hbm_call(kernel, nbytes, name, *args, compulsory=None):
    probe = _hbm_probe
    if probe is not None:
        probe.before(kernel, float(nbytes), float(nbytes if compulsory is None else compulsory))
    _call(name, *args)
    if probe is not None:
        probe.after()


def gather_rotate(x, src, tgt, coef, rad, out):
    N, nsph, C = x.shape
    E = src.numel()
    edge = 4 * (35 + (12 * C if rad is not None else 0) + 18 * C) + 8
    nbytes = E * (edge + 4 * 18 * C)
    _hbm_call(f"k_gather_rotate<{_pick_v(2 * C)},{_tf(rad is not None)},2>", nbytes, "tta_gather_rotate", _ptr(x, numel=N * 9 * C, name="x"),
              _i32(src, E), _i32(tgt, E),
              _ptr(coef, numel=E * 35, name="coef"), _ptr(rad, numel=E * 12 * C, name="rad"),
              _ptr(out, numel=E * 18 * C, name="out"), N, E, C, _stream(),
              compulsory=E * edge + 4 * N * 9 * C)
    return out


def gather_rotate_src(x, src, coef, out):
    N, _, C = x.shape
    E = src.numel()
    _hbm_call(f"k_gather_rotate<{_pick_v(C)},false,1>", E * (4 * (9 * C + 35 + 9 * C) + 4), "tta_gather_rotate_src",
              _ptr(x, numel=N * 9 * C, name="x"), _i32(src, E),
              _ptr(coef, numel=E * 35, name="coef"), _ptr(out, numel=E * 9 * C, name="out"), N, E, C,
              _stream(), compulsory=E * (4 * (35 + 9 * C) + 4) + 4 * N * 9 * C)
    return out


def gather_rotate_src_bw(g_out, x, src, coef, g_in, g_coef):
    N, _, C = x.shape
    E = src.numel()
    edge = 4 * (9 * C + 35 + 70 + (9 * C if g_in is not None else 0)) + 4
    _hbm_call(f"k_gather_rotate_bw<{_pick_v(C)},false,1>", E * (edge + 4 * 9 * C), "tta_gather_rotate_src_bw",
              _ptr(g_out, numel=E * 9 * C, name="g_out"),
              _ptr(x, numel=N * 9 * C, name="x"), _i32(src, E), _ptr(coef, numel=E * 35, name="coef"),
              None if g_in is None else _ptr(g_in, numel=E * 9 * C, name="g_in"),
              _ptr(g_coef, numel=E * 35, name="g_coef"), N, E, C, _stream(),
              compulsory=E * edge + 4 * N * 9 * C)


def gather_rotate_bw(g_xf, rad, x, src, tgt, coef, g_rad, g_mcat, g_coef):
    N, _, C = x.shape
    E = src.numel()
    edge = 4 * (18 * C + (24 * C if rad is not None else 0) + 35 + 70 + 18 * C) + 8
    nbytes = E * (edge + 4 * 18 * C)
    _hbm_call(f"k_gather_rotate_bw<{_pick_v(2 * C)},{_tf(rad is not None)},2>", nbytes, "tta_gather_rotate_bw",
              _ptr(g_xf, numel=E * 18 * C, name="g_xf"),
              _ptr(rad, numel=E * 12 * C, name="rad"), _ptr(x, numel=N * 9 * C, name="x"),
              _i32(src, E), _i32(tgt, E), _ptr(coef, numel=E * 35, name="coef"),
              _ptr(g_rad, numel=E * 12 * C, name="g_rad"), _ptr(g_mcat, numel=E * 18 * C, name="g_mcat"),
              _ptr(g_coef, numel=E * 35, name="g_coef"), N, E, C, _stream(),
              compulsory=E * edge + 4 * N * 9 * C)


def gather_rotate_bw_dst(g_xf, rad, x, src, tgt_ptr, coef, g_rad, g_mcat, g_coef, tsum):
    """gather_rotate_bw walked by destination node (edges sorted by destination, tgt_ptr their
    CSR offsets): g_mcat gets its source half only, and tsum [N, 9, C] receives the destination
    half already summed per node (the sum node_gather_sum would form, bit for bit).  C <= 256."""
    N, _, C = x.shape
    E = src.numel()
    edge = 4 * (18 * C + 24 * C + 35 + 70 + 9 * C) + 4
    _hbm_call(f"k_gather_rotate_bw_dst<{_pick_v(C)}>", E * (edge + 4 * 9 * C) + 4 * N * 9 * C,
              "tta_gather_rotate_bw_dst",
              _ptr(g_xf, numel=E * 18 * C, name="g_xf"), _ptr(rad, numel=E * 12 * C, name="rad"),
              _ptr(x, numel=N * 9 * C, name="x"), _i32(src, E), _i32(tgt_ptr, N + 1, "tgt_ptr"),
              _ptr(coef, numel=E * 35, name="coef"), _ptr(g_rad, numel=E * 12 * C, name="g_rad"),
              _ptr(g_mcat, numel=E * 18 * C, name="g_mcat"), _ptr(g_coef, numel=E * 35, name="g_coef"),
              _ptr(tsum, numel=N * 9 * C, name="tsum"), N, E, C, _stream(),
              compulsory=E * edge + 4 * N * 9 * C * 2)


def node_gather_sum_dst(g_mcat, src_ptr, src_perm, tsum, res, out):
    """node_gather_sum with the destination sums precomputed (tsum from gather_rotate_bw_dst)."""
    N, _, C = out.shape
    E = src_perm.numel()
    nbytes = 4 * (E * 9 * C + (N + 1) + E + N * 9 * C * (2 + (res is not None)))
    _hbm_call(f"k_node_gather_sum<{_pick_v(C)}>", nbytes, "tta_node_gather_sum_dst",
              _ptr(g_mcat, numel=E * 18 * C, name="g_mcat"),
              _i32(src_ptr, N + 1, "src_ptr"), _i32(src_perm, E, "src_perm"),
              _ptr(tsum, numel=N * 9 * C, name="tsum"), _ptr(res, numel=N * 9 * C, name="res"),
              _ptr(out, numel=N * 9 * C, name="out"), N, E, C, _stream())
    return out


def gather_rotate_bw_nodes(g_xf, rad, x, src_ptr, src_perm, tgt_ptr, coef, g_rad, g_coef,
                           coef_half, ssum, res, out):
    """The backward of gather_rotate (rad given) walked from both ends of every edge: the source
    walk (outgoing edges of each node through src_ptr / src_perm, source half of the channels)
    writes ssum [N, 9, C] and the source half's coefficient sums coef_half [E, 35]; the
    destination walk (incoming edges, tgt_ptr, destination half) writes out [N, 9, C] =
    (ssum + its sum) + res and accumulates g_coef.  Both write their half of g_rad.  g_rad and
    out are the bits of gather_rotate_bw_dst + node_gather_sum_dst (g_coef to fp32 rounding),
    without the [E, 9, C] gather adjoint.  bw_walk_width_ok(C) must hold."""
    N, _, C = x.shape
    E = src_perm.numel()
    V = _pick_v(C)
    chk = dict(g_xf=(g_xf, E * 18 * C), rad=(rad, E * 12 * C), g_rad=(g_rad, E * 12 * C),
               coef=(coef, E * 35), g_coef=(g_coef, E * 35), coef_half=(coef_half, E * 35))
    p = {k: _ptr(t, numel=n, name=k) for k, (t, n) in chk.items()}
    xp = _ptr(x, numel=N * 9 * C, name="x")
    sp = _ptr(ssum, numel=N * 9 * C, name="ssum")
    # per edge: the half rows of g_xf and rad read, of g_rad written; the coefficients (and the
    # source walk's sums, and g_coef read and written); per node: its own row, the sums
    e_src = 4 * (21 * C + 35 + 35 + 1)
    _hbm_call(f"k_gather_rotate_bw_walk<{V},false>", E * e_src + 4 * N * (18 * C + 1),
              "tta_gather_rotate_bw_srcwalk", p["g_xf"], p["rad"], xp,
              _i32(src_ptr, N + 1, "src_ptr"), _i32(src_perm, E, "src_perm"), p["coef"],
              p["g_rad"], p["coef_half"], sp, N, E, C, _stream())
    e_tgt = 4 * (21 * C + 4 * 35)
    _hbm_call(f"k_gather_rotate_bw_walk<{V},true>",
              E * e_tgt + 4 * N * ((27 + 9 * (res is not None)) * C + 1),
              "tta_gather_rotate_bw_tgtwalk", p["g_xf"], p["rad"], xp,
              _i32(tgt_ptr, N + 1, "tgt_ptr"), p["coef"], p["g_rad"], p["g_coef"],
              p["coef_half"], sp, _ptr(res, numel=N * 9 * C, name="res"),
              _ptr(out, numel=N * 9 * C, name="out"), N, E, C, _stream())
    return out


def rotate_env_segsum(m, coef, env, tgt_ptr, res, out, *, n_in, env_first, div=1.0):
    N, _, C = out.shape
    E = coef.shape[0]
    nbytes = 4 * (E * (n_in * C + 36) + (N + 1) + N * 9 * C * (1 + (res is not None)))
    _hbm_call(f"k_rotate_env_segsum<{_pick_v(C)},{n_in},{_tf(env_first)}>", nbytes, "tta_rotate_env_segsum",
              _ptr(m, numel=E * n_in * C, name="m"),
              _ptr(coef, numel=E * 35, name="coef"), _ptr(env, numel=E, name="env"),
              _i32(tgt_ptr, N + 1, "tgt_ptr"), _ptr(res, numel=N * 9 * C, name="res"),
              _ptr(out, numel=N * 9 * C, name="out"), N, E, C, n_in, int(env_first), float(div),
              _stream())
    return out


def rotate_env_segsum_bw(g_node, tgt, m, coef, env, g_m, g_coef, g_env, *, n_in, env_first,
                         div=1.0):
    N, _, C = g_node.shape
    E = tgt.numel()
    nbytes = 4 * E * (9 * C + 1 + 2 * n_in * C + 35 + 1 + 70 + 2)
    _hbm_call(f"k_rotate_env_segsum_bw<{_pick_v(C)},{n_in},{_tf(env_first)}>", nbytes, "tta_rotate_env_segsum_bw",
              _ptr(g_node, numel=N * 9 * C, name="g_node"), _i32(tgt, E),
              _ptr(m, numel=E * n_in * C, name="m"), _ptr(coef, numel=E * 35, name="coef"),
              _ptr(env, numel=E, name="env"), _ptr(g_m, numel=E * n_in * C, name="g_m"),
              _ptr(g_coef, numel=E * 35, name="g_coef"), _ptr(g_env, numel=E, name="g_env"), N, E, C,
              n_in, int(env_first), float(div), _stream(),
              compulsory=nbytes - 4 * E * 9 * C + 4 * N * 9 * C)


def node_gather_sum(g_mcat, src_ptr, src_perm, tgt_ptr, res, out):
    N, _, C = out.shape
    E = src_perm.numel()
    nbytes = 4 * (E * 18 * C + 2 * (N + 1) + E + N * 9 * C * (1 + (res is not None)))
    _hbm_call(f"k_node_gather_sum<{_pick_v(C)}>", nbytes, "tta_node_gather_sum",
              _ptr(g_mcat, numel=E * 18 * C, name="g_mcat"),
              _i32(src_ptr, N + 1, "src_ptr"), _i32(src_perm, E, "src_perm"),
              _i32(tgt_ptr, N + 1, "tgt_ptr"), _ptr(res, numel=N * 9 * C, name="res"),
              _ptr(out, numel=N * 9 * C, name="out"), N, E, C, _stream())
    return out


# ----------------------------------------------------------------------------- row-wise
def gate_fwd(x, gating, y, idx8, *, R, H, L, ldx=None, ldg=None):
    """x rows [9*H] at stride ldx, gating rows [L*H] at stride ldg, y contiguous [R, 9, H]."""
    ldx = 9 * H if ldx is None else ldx
    ldg = L * H if ldg is None else ldg
    _hbm_call("k_gate_fwd", 4 * R * H * (18 + L), "tta_gate_fwd",
              _rows(x, R, ldx, 9 * H, "x"), _rows(gating, R, ldg, L * H, "gating"),
              _ptr(y, numel=R * 9 * H, name="y"), R, H, L, ldx, ldg, _host_idx8(idx8), _stream())
    return y


def gate_bwd(g_y, x, gating, g_x, g_gating, idx8, *, R, H, L, ldx=None, ldg=None):
    """g_x shares x's row stride, g_gating shares gating's."""
    ldx = 9 * H if ldx is None else ldx
    ldg = L * H if ldg is None else ldg
    _hbm_call("k_gate_bwd", 4 * R * H * (27 + 2 * L), "tta_gate_bwd",
              _ptr(g_y, numel=R * 9 * H, name="g_y"), _rows(x, R, ldx, 9 * H, "x"),
              _rows(gating, R, ldg, L * H, "gating"), _rows(g_x, R, ldx, 9 * H, "g_x"),
              _rows(g_gating, R, ldg, L * H, "g_gating"), R, H, L, ldx, ldg, _host_idx8(idx8),
              _stream())


def gate_gating_bwd(g_x, y, sig, g_gating, idx8, *, R, H, L):
    """The gating adjoint from the gate's input adjoint g_x (written by linear_group_gate with
    backward=True), the gated rows y (contiguous [R, 9, H]) and the gating sigmoids sig
    (tta_gate_gating_bwd); g_x, sig and g_gating are row-strided 2-D views."""
    ldgx, ldg, ldgg = (_ld(t, nm) for t, nm in ((g_x, "g_x"), (sig, "sig"), (g_gating, "g_gating")))
    _hbm_call("k_gate_gating_bwd", 4 * R * H * (16 + 2 * L), "tta_gate_gating_bwd",
              _rows(g_x, R, ldgx, 9 * H, "g_x"), _ptr(y, numel=R * 9 * H, name="y"),
              _rows(sig, R, ldg, L * H, "sig"), _rows(g_gating, R, ldgg, L * H, "g_gating"),
              R, H, L, ldgx, ldg, ldgg, _host_idx8(idx8), _stream())


def _host_i32(vals, name):
    vals = [int(v) for v in vals]
    return (ctypes.c_int * max(1, len(vals)))(*vals)


def rotate_pattern(x, coef, out, ptr, k, blk, *, E, n_in, n_out, W):
    """out [E, n_out, W] = the sparse-pattern rotation of x [E, n_in, W] by coef [E, nnz]
    (tta_rotate_pattern): the terms of output block r are q in [ptr[r], ptr[r+1]), coefficient
    column k[q] times input block blk[q] (host sequences)."""
    nnz = len(k)
    if len(ptr) != n_out + 1 or len(blk) != nnz:
        raise RuntimeError("rotate_pattern: ptr needs n_out + 1 entries and blk one per term")
    _hbm_call("k_rotate_pattern", 4 * E * ((n_in + n_out) * W + nnz), "tta_rotate_pattern",
              _ptr(x, numel=E * n_in * W, name="x"), _ptr(coef, numel=E * nnz, name="coef"),
              _ptr(out, numel=E * n_out * W, name="out"), E, n_in, n_out, W, nnz,
              _host_i32(ptr, "ptr"), _host_i32(k, "k"), _host_i32(blk, "blk"), _stream())


def rotate_pattern_gc(g_out, x_in, gc, ii, jj, *, E, n_in, n_out, W):
    """gc [E, nnz]: gc[e, k] = sum_w g_out[e, ii[k], w] x_in[e, jj[k], w]
    (tta_rotate_pattern_gc)."""
    nnz = len(ii)
    if len(jj) != nnz:
        raise RuntimeError("rotate_pattern_gc: ii and jj differ in length")
    _hbm_call("k_rotate_pattern_gc", 4 * E * ((n_in + n_out) * W + nnz), "tta_rotate_pattern_gc",
              _ptr(g_out, numel=E * n_out * W, name="g_out"),
              _ptr(x_in, numel=E * n_in * W, name="x_in"), _ptr(gc, numel=E * nnz, name="gc"),
              E, n_in, n_out, W, nnz, _host_i32(ii, "ii"), _host_i32(jj, "jj"), _stream())


def segment_sum_table(msg, gather, out, *, N, Dmax, W):
    """out [N, W] = per-node sums of msg [n_msg, W] rows over the [N, Dmax] int32 gather table
    (entries outside [0, n_msg) add nothing; tta_segment_sum_table)."""
    n_msg = msg.shape[0] if msg.dim() == 2 else msg.numel() // max(W, 1)
    _hbm_call("k_segment_sum_table", 4 * (N * Dmax + 2 * N * W + N * Dmax * W),
              "tta_segment_sum_table", _ptr(msg, numel=n_msg * W, name="msg"),
              _i32(gather, N * Dmax, "gather"), _ptr(out, numel=N * W, name="out"), n_msg, N,
              Dmax, W, _stream())


def ln_silu_fwd(a, gamma, beta, nrm, s, *, R, n, groups=1, lda=None, lds=None, eps=1e-5):
    """``groups`` LayerNorms of width n side by side per row (gamma / beta [groups * n]).
    ``nrm`` (the LayerNorm output) may be None: then it is not written, and ln_silu_bwd
    recomputes it."""
    w = groups * n
    lda = w if lda is None else lda
    lds = w if lds is None else lds
    G, NPL, VEC = _ln_variant(n, n in (128, 256) and lda % 4 == 0 and lds % 4 == 0
                              and _al16(a, gamma, beta, nrm, s))
    _hbm_call(f"k_ln_silu_fwd<{G},{NPL},{_tf(VEC)}>", 4 * ((2 + (nrm is not None)) * R * w + 2 * w),
              "tta_ln_silu_fwd",
              _rows(a, R, lda, w, "a"), _ptr(gamma, numel=w), _ptr(beta, numel=w),
              None if nrm is None else _rows(nrm, R, lda, w, "nrm"), _rows(s, R, lds, w, "s"),
              R, n, groups, lda, lds, eps, _stream())


def ln_silu_bwd(g, a, nrm, gamma, g_a, *, R, n, groups=1, ldg=None, lda=None, ldo=None,
                eps=1e-5, beta=None):
    """Backward of silu(layer_norm(a)); with ``nrm`` None the LayerNorm output is recomputed
    from a, gamma and ``beta`` (the same values the forward produced)."""
    w = groups * n
    ldg = w if ldg is None else ldg
    lda = w if lda is None else lda
    ldo = w if ldo is None else ldo
    if nrm is None and beta is None:
        raise RuntimeError("ln_silu_bwd: nrm, or beta to recompute it, is required")
    nbytes = 4 * (4 * R * w + w) if nrm is not None else 4 * (3 * R * w + 2 * w)
    G, NPL, VEC = _ln_variant(n, n in (128, 256) and ldg % 4 == 0 and lda % 4 == 0
                              and ldo % 4 == 0 and _al16(g, a, nrm, gamma, beta, g_a))
    _hbm_call(f"k_ln_silu_bwd<{G},{NPL},{_tf(nrm is None)},{_tf(VEC)}>", nbytes, "tta_ln_silu_bwd",
              _rows(g, R, ldg, w, "g"), _rows(a, R, lda, w, "a"),
              None if nrm is None else _rows(nrm, R, lda, w, "nrm"), _ptr(gamma, numel=w),
              None if beta is None else _ptr(beta, numel=w), _rows(g_a, R, ldo, w, "g_a"), R, n,
              groups, ldg, lda, ldo, eps, _stream())


def rmsnorm_sh_fwd(x, aw, ab, add0, y, inv, eps=1e-5):
    N, _, C = x.shape
    _call("tta_rmsnorm_sh_fwd", _ptr(x, numel=N * 9 * C, name="x"), _ptr(aw, numel=3 * C),
          _ptr(ab, numel=C), _ptr(add0, numel=N * C, name="add0"), _ptr(y, numel=N * 9 * C),
          _ptr(inv, numel=N, name="inv"), N, C, eps, _stream())


def rmsnorm_sh_bwd(g, x, aw, inv, res, out):
    N, _, C = x.shape
    _call("tta_rmsnorm_sh_bwd", _ptr(g, numel=N * 9 * C, name="g"), _ptr(x, numel=N * 9 * C),
          _ptr(aw, numel=3 * C), _ptr(inv, numel=N), _ptr(res, numel=N * 9 * C, name="res"),
          _ptr(out, numel=N * 9 * C), N, C, _stream())


def silu_bwd(g, x, out):
    n = g.numel()
    _call("tta_silu_bwd", _ptr(g, numel=n), _ptr(x, numel=n), _ptr(out, numel=n), n, _stream())


def reduce_sum(x, n, stride, out):
    """out[0] = sum of x[0], x[stride], ..., x[(n - 1) * stride] (x fp32 on the device)."""
    if stride < 1:
        raise RuntimeError("reduce_sum: stride must be >= 1")
    _call("tta_sum", _rows(x, n, stride, 1, "x"), n, stride, _ptr(out, numel=1), _stream())


def segment_sum(x, ptr, out):
    """out[k] = sum of x over [ptr[k], ptr[k+1]) (x contiguous fp32, ptr int32 [K + 1])."""
    K = out.numel()
    n = x.numel()
    _call("tta_segment_sum", _ptr(x, numel=n, name="x"), _i32(ptr, K + 1, "ptr"), K,
          _ptr(out, numel=K), _stream())


def fill(out, value):
    _call("tta_fill", _ptr(out), out.numel(), float(value), _stream())


# ----------------------------------------------------------------------------- geometry
def edge_wigner(pos, src, tgt, shift, jd, gamma, ev, dist, coef):
    N = pos.shape[0]
    E = src.numel()
    sh = 12 if shift is not None else 0
    # per edge: src / tgt, two gathered positions, the shift; out ev, dist, 35 coefficients
    _hbm_call("k_edge_wigner", E * (8 + 24 + sh + 12 + 4 + 140) + 140, "tta_edge_wigner",
              _ptr(pos, numel=N * 3, name="pos"), _i32(src, E), _i32(tgt, E),
              _ptr(shift, numel=E * 3, name="shift"), _ptr(jd, numel=35, name="jd"), float(gamma),
              _ptr(ev, numel=E * 3), _ptr(dist, numel=E), _ptr(coef, numel=E * 35), N, E,
              _stream(), compulsory=E * (8 + sh + 12 + 4 + 140) + 12 * N + 140)


def edge_features(dist, zsrc, ztgt, src_emb, tgt_emb, offsets, coeff, cutoff, nb, ec, x_edge, env):
    E = dist.numel()
    v4 = nb % 4 == 0 and ec % 4 == 0 and _al16(x_edge, offsets, src_emb, tgt_emb)
    # per edge: dist, two species, two gathered embedding rows; out x_edge row and envelope
    _hbm_call("k_edge_features_v4" if v4 else "k_edge_features",
              E * (4 + 8 + 8 * ec + 4 * (nb + 2 * ec) + 4) + 4 * nb, "tta_edge_features",
              _ptr(dist, numel=E), _i32(zsrc, E), _i32(ztgt, E),
              _ptr(src_emb, name="src_emb"), _ptr(tgt_emb, name="tgt_emb"),
              _ptr(offsets, numel=nb, name="offsets"), float(coeff), float(cutoff), nb, ec,
              _ptr(x_edge, numel=E * (nb + 2 * ec), name="x_edge"), _ptr(env, numel=E), E,
              _stream(), compulsory=E * (4 + 8 + 4 * (nb + 2 * ec) + 4) + 4 * nb
              + 4 * sum(t.numel() for t in (src_emb, tgt_emb) if t is not None))


def edge_geometry_fwd(pos, src, tgt, shift, jd, gamma, zsrc, ztgt, src_emb, tgt_emb, offsets,
                      coeff, cutoff, nb, ec, ev, dist, coef, x_edge, env):
    """edge_wigner + edge_features in one launch (same results)."""
    N = pos.shape[0]
    E = src.numel()
    v4 = (nb % 4 == 0 and ec % 4 == 0 and nb + 2 * ec < (1 << 14)
          and _al16(x_edge, offsets, src_emb, tgt_emb))
    if not v4:
        edge_wigner(pos, src, tgt, shift, jd, gamma, ev, dist, coef)
        edge_features(dist, zsrc, ztgt, src_emb, tgt_emb, offsets, coeff, cutoff, nb, ec,
                      x_edge, env)
        return
    sh = 12 if shift is not None else 0
    W = nb + 2 * ec
    # per edge: src / tgt, two gathered positions, the shift, two species, two gathered
    # embedding rows; out ev, dist, 35 coefficients, the x_edge row and the envelope
    _hbm_call("k_edge_geometry_fwd",
              E * (8 + 24 + sh + 8 + 8 * ec + 12 + 4 + 140 + 4 * W + 4) + 140 + 4 * nb,
              "tta_edge_geometry_fwd",
              _ptr(pos, numel=N * 3, name="pos"), _i32(src, E), _i32(tgt, E),
              _ptr(shift, numel=E * 3, name="shift"), _ptr(jd, numel=35, name="jd"), float(gamma),
              _i32(zsrc, E), _i32(ztgt, E), _ptr(src_emb, name="src_emb"),
              _ptr(tgt_emb, name="tgt_emb"), _ptr(offsets, numel=nb, name="offsets"),
              float(coeff), float(cutoff), nb, ec, _ptr(ev, numel=E * 3),
              _ptr(dist, numel=E), _ptr(coef, numel=E * 35),
              _ptr(x_edge, numel=E * W, name="x_edge"), _ptr(env, numel=E), N, E, _stream(),
              compulsory=E * (8 + sh + 8 + 12 + 4 + 140 + 4 * W + 4) + 12 * N + 140 + 4 * nb
              + 4 * sum(t.numel() for t in (src_emb, tgt_emb) if t is not None))


def edge_geometry_bwd(ev, dist, g_coef, g_env, g_gauss, ldg, offsets, coeff, cutoff, nb, jd,
                      gamma, g_ev):
    E = dist.numel()
    if g_gauss is not None and (ldg < nb or offsets is None or offsets.numel() < nb):
        raise RuntimeError("edge_geometry_bwd: g_gauss needs ldg >= nb and nb offsets")
    v4 = (g_gauss is not None and nb % 4 == 0 and ldg % 4 == 0 and _al16(g_gauss, offsets))
    kern = f"k_edge_geometry_bwd<{256 if E >= 256 * 512 else 64},{_tf(v4)}>"
    # per edge: ev, dist, g_coef, g_env, the Gaussian-adjoint row; out g_ev
    per = 12 + 4 + (140 if g_coef is not None else 0) + (4 if g_env is not None else 0) + \
        (4 * nb if g_gauss is not None else 0) + 12
    _hbm_call(kern, E * per + 4 * nb + 140, "tta_edge_geometry_bwd", _ptr(ev, numel=E * 3),
              _ptr(dist, numel=E), _ptr(g_coef, numel=E * 35, name="g_coef"),
              _ptr(g_env, numel=E, name="g_env"),
              None if g_gauss is None else _rows(g_gauss, E, ldg, nb, "g_gauss"), ldg,
              _ptr(offsets, name="offsets"), float(coeff), float(cutoff), nb,
              _ptr(jd, numel=35), float(gamma), _ptr(g_ev, numel=E * 3), E, _stream())


def node_forces(g_ev, src_ptr, src_perm, tgt_ptr, forces):
    N = forces.shape[0]
    E = src_perm.numel()
    _call("tta_node_forces", _ptr(g_ev, numel=E * 3), _i32(src_ptr, N + 1), _i32(src_perm, E),
          _i32(tgt_ptr, N + 1), _ptr(forces, numel=N * 3), N, E, _stream())


def virial(ev, g_ev, work, out):
    E = ev.shape[0]
    _call("tta_virial", _ptr(ev, numel=E * 3), _ptr(g_ev, numel=E * 3), E,
          _ptr(work, numel=256 * 9, name="work"), _ptr(out, numel=9), _stream())


def virial_noalloc(ev, g_ev, out):
    """``virial`` without a workspace: the library's per-GPU device scratch holds the partial
    sums (nothing is allocated; overlapping calls on one GPU race)."""
    E = ev.shape[0]
    _call("tta_virial_noalloc", _ptr(ev, numel=E * 3), _ptr(g_ev, numel=E * 3), E,
          _ptr(out, numel=9), _stream())


# ----------------------------------------------------------------------------- fused node stages
def node_fusable(C, H):
    """The fused node-level kernels take C and H multiples of 16 up to 128."""
    return C % 16 == 0 and H % 16 == 0 and 16 <= C <= 128 and 16 <= H <= 128


def spectral_block_fwd(x1, norm2, ff, inv2, a_s, h, x2, next_norm=None, add0=None, yn=None,
                       invn=None, eps=1e-5):
    """x2 = x1 + spectral FF of RMSNormSH_2(x1); with ``next_norm`` also yn = RMSNormSH_next(x2)
    (+ add0 on coefficient 0).  ``norm2`` / ``next_norm``: (aw [3, C], ab [C]); ``ff``: the
    per-degree weights (ws_t, bs, w1t, b1, w2t, b2)."""
    N, _, C = x1.shape
    H = ff[2].shape[2]
    nx = N * 9 * C
    awn, abn = next_norm if next_norm is not None else (None, None)
    _call("tta_spectral_block_fwd", _ptr(x1, numel=nx, name="x1"), _ptr(norm2[0], numel=3 * C),
          _ptr(norm2[1], numel=C), _ptr(ff[0], numel=C * 2 * H), _ptr(ff[1], numel=2 * H),
          _ptr(ff[2], numel=3 * C * H), _ptr(ff[3], numel=H), _ptr(ff[4], numel=3 * H * C),
          _ptr(ff[5], numel=C), _ptr(inv2, numel=N), _ptr(a_s, numel=N * 2 * H),
          _ptr(h, numel=N * 9 * H), _ptr(x2, numel=nx, name="x2"),
          None if awn is None else _ptr(awn, numel=3 * C),
          None if abn is None else _ptr(abn, numel=C),
          None if add0 is None else _ptr(add0, numel=N * C, name="add0"),
          None if yn is None else _ptr(yn, numel=nx, name="yn"),
          None if invn is None else _ptr(invn, numel=N), N, C, H, float(eps), _stream())


def spectral_block_bwd(g_n, x2, next_norm_w, invn, res, x1, aw2, inv2, a_s, h, ffb, g_x1):
    """g_x1 of one block's node-level tail from the adjoint g_n of the next norm's output;
    ``ffb``: the per-degree backward weights (w1 [3, H, C], w2 [3, C, H], ws [2H, C])."""
    N, _, C = x1.shape
    H = ffb[0].shape[1]
    nx = N * 9 * C
    _call("tta_spectral_block_bwd", _ptr(g_n, numel=nx, name="g_n"), _ptr(x2, numel=nx, name="x2"),
          _ptr(next_norm_w, numel=3 * C), _ptr(invn, numel=N),
          None if res is None else _ptr(res, numel=nx, name="res"), _ptr(x1, numel=nx, name="x1"),
          _ptr(aw2, numel=3 * C), _ptr(inv2, numel=N), _ptr(a_s, numel=N * 2 * H),
          _ptr(h, numel=N * 9 * H), _ptr(ffb[0], numel=3 * H * C), _ptr(ffb[1], numel=3 * C * H),
          _ptr(ffb[2], numel=2 * H * C), _ptr(g_x1, numel=nx, name="g_x1"), N, C, H, _stream())


def energy_head_fwd(ne, w_t, b, a1, a2, node_e):
    """Per-node energy MLP on coefficient 0 of ne [N, 9, C]: w_t = (w0t [C, H], w1t [H, H],
    w2 [H]), b = (b0, b1, b2)."""
    N, _, C = ne.shape
    H = w_t[0].shape[1]
    _call("tta_energy_head_fwd", _ptr(ne, numel=N * 9 * C, name="ne"), _ptr(w_t[0], numel=C * H),
          _ptr(b[0], numel=H), _ptr(w_t[1], numel=H * H), _ptr(b[1], numel=H),
          _ptr(w_t[2], numel=H), _ptr(b[2], numel=1), _ptr(a1, numel=N * H),
          _ptr(a2, numel=N * H), _ptr(node_e, numel=N), N, C, H, _stream())


def energy_head_bwd(a1, a2, w0, w1, w2, g_ne):
    N, H = a1.shape
    C = w0.shape[1]
    _call("tta_energy_head_bwd", _ptr(a1, numel=N * H), _ptr(a2, numel=N * H),
          _ptr(w0, numel=H * C), _ptr(w1, numel=H * H), _ptr(w2, numel=H),
          _ptr(g_ne, numel=N * 9 * C, name="g_ne"), N, C, H, _stream())


# ----------------------------------------------------------------------------- neighbour list
def radius_graph_passes(pos, lo, hi, shifts, periodic, mid2, cut2, min2, k, clo=None, chi=None):
    """The three device passes of the radius graph (thresholds with a cap, per-row counts,
    ordered write); returns (src int64 [E], tgt int64 [E], cell int32 [E] or None).  clo / chi:
    per-row image-shift ranges of a periodic batch (int32 device tensors, checked here on their
    host copies by the caller, geometry.system_graphs)."""
    N = pos.shape[0]
    dev = pos.device
    n_cells = shifts.shape[0] if periodic else 0
    lo_p = None if lo is None else _i32(lo, N, "lo")
    hi_p = None if hi is None else _i32(hi, N, "hi")
    if (clo is None) != (chi is None) or (clo is not None and not periodic):
        raise ValueError("radius graph: cell ranges go with a periodic graph, both or neither")
    clo_p = None if clo is None else _i32(clo, N, "clo")
    chi_p = None if chi is None else _i32(chi, N, "chi")
    sh_p = _ptr(shifts, numel=3 * n_cells, name="shifts") if periodic else None
    common = (_ptr(pos, numel=N * 3, name="pos"), N, lo_p, hi_p, sh_p, n_cells, clo_p, chi_p,
              int(periodic), float(mid2), float(cut2), float(min2))
    thr = (None, None, None)
    if k:
        td = torch.empty(N, device=dev, dtype=torch.float32)
        ta = torch.empty(N, device=dev, dtype=torch.int32)
        tc = torch.empty(N, device=dev, dtype=torch.int32)
        err = torch.zeros(1, device=dev, dtype=torch.int32)
        _call("tta_radius_graph_thresholds", *common, int(k), td.data_ptr(), ta.data_ptr(),
              tc.data_ptr(), err.data_ptr(), _stream())
        if int(err.item()):
            raise RuntimeError("radius graph: a receiver has more than 1024 neighbours within "
                               "the cutoff (the capped device neighbour list holds at most 1024)")
        thr = (td.data_ptr(), ta.data_ptr(), tc.data_ptr())
    counts = torch.empty(N, device=dev, dtype=torch.int32)
    _call("tta_radius_graph_count", *common, *thr, counts.data_ptr(), _stream())
    c64 = counts.to(torch.int64)
    ends = torch.cumsum(c64, 0)
    offsets = ends - c64
    E = int(ends[-1]) if N else 0
    src = torch.empty(E, device=dev, dtype=torch.int64)
    tgt = torch.empty(E, device=dev, dtype=torch.int64)
    cell = torch.empty(E, device=dev, dtype=torch.int32) if periodic else None
    if E:
        _call("tta_radius_graph_write", *common, *thr, offsets.data_ptr(), src.data_ptr(),
              tgt.data_ptr(), None if cell is None else cell.data_ptr(), _stream())
    return src, tgt, cell


CELL_ROW_MAX = 2048   # kept entries per row that the cell-list write pass sorts in LDS
CELL_MAX_K = 1024     # largest cap of the cell-list threshold selection


def radius_graph_cells(pos, shifts, periodic, grid, mid2, cut2, min2, k):
    """The cell-list radius graph of one system: the edges of ``radius_graph_passes`` (same
    order, image cells and cap) from the 27 bins around every row atom.  ``grid`` = (origin [3],
    inv_h, dims [3]) from ``geometry.cell_grid``.  A graph with a row of more than CELL_ROW_MAX
    kept entries is written by the row-scan write pass (same edges)."""
    N = pos.shape[0]
    dev = pos.device
    n_cells = shifts.shape[0] if periodic else 0
    origin, inv_h, dims = grid
    g = CellGrid((_F * 3)(*[float(v) for v in origin]), float(inv_h),
                 (_I * 3)(*[int(v) for v in dims]))
    nb = int(dims[0]) * int(dims[1]) * int(dims[2])
    P = N * n_cells if periodic else N
    if periodic and P >= (1 << 30):
        raise ValueError("cell list: N * n_cells must stay below 2^30")
    lib = load()
    work = torch.empty(int(lib.tta_cell_list_workspace(nb, P)), device=dev, dtype=torch.int32)
    bin_start = torch.empty(nb + 1, device=dev, dtype=torch.int32)
    pts = torch.empty(max(P, 1), 4, device=dev, dtype=torch.float32)
    pos_p = _ptr(pos, numel=N * 3, name="pos")
    sh_p = _ptr(shifts, numel=3 * n_cells, name="shifts") if periodic else None
    common = (pos_p, N, sh_p, n_cells, int(periodic), ctypes.byref(g))
    _call("tta_cell_list_build", *common, bin_start.data_ptr(), pts.data_ptr(), work.data_ptr(),
          _stream())
    cl = (bin_start.data_ptr(), pts.data_ptr(), float(mid2), float(cut2), float(min2))
    thr = (None, None, None)
    counts = torch.empty(N, device=dev, dtype=torch.int32)
    if k > CELL_MAX_K and N:
        # above the selection's limit the cap must be a no-op: every receiver (a row, by the
        # symmetry of the aperiodic mask) has at most k candidates
        _call("tta_radius_graph_cells_count", *common, *cl, *thr, counts.data_ptr(), _stream())
        if int(counts.max()) > k:
            raise ValueError(f"cell list: a cap of {k} > {CELL_MAX_K} neighbours is supported only "
                             "when no receiver has more than that many candidates")
        k = 0
    if k:
        td = torch.empty(N, device=dev, dtype=torch.float32)
        ta = torch.empty(N, device=dev, dtype=torch.int32)
        tc = torch.empty(N, device=dev, dtype=torch.int32)
        _call("tta_radius_graph_cells_thresholds", *common, *cl, int(k), td.data_ptr(),
              ta.data_ptr(), tc.data_ptr(), _stream())
        thr = (td.data_ptr(), ta.data_ptr(), tc.data_ptr())
    _call("tta_radius_graph_cells_count", *common, *cl, *thr, counts.data_ptr(), _stream())
    c64 = counts.to(torch.int64)
    ends = torch.cumsum(c64, 0)
    offsets = ends - c64
    E, cmax = (int(v) for v in torch.stack([ends[-1], c64.max()]).cpu()) if N else (0, 0)
    src = torch.empty(E, device=dev, dtype=torch.int64)
    tgt = torch.empty(E, device=dev, dtype=torch.int64)
    cell = torch.empty(E, device=dev, dtype=torch.int32) if periodic else None
    if not E:
        return src, tgt, cell
    out = (offsets.data_ptr(), src.data_ptr(), tgt.data_ptr(),
           None if cell is None else cell.data_ptr())
    if cmax <= CELL_ROW_MAX:
        err = torch.zeros(1, device=dev, dtype=torch.int32)
        _call("tta_radius_graph_cells_write", *common, *cl, *thr, *out, err.data_ptr(), _stream())
        if int(err.item()):
            raise RuntimeError("cell list: a row overflowed the write pass after the count pass "
                               "allowed it")
    else:
        _call("tta_radius_graph_write", pos_p, N, None, None, sh_p, n_cells, None, None,
              int(periodic), float(mid2), float(cut2), float(min2), *thr, *out, _stream())
    return src, tgt, cell


# ----------------------------------------------------------------------------- Orb-v3
def linear_gather(x, w_t, bias, out, P, idx0, idx1, off1, *, epilogue=EPI_STORE, out2=None):
    """out = epi(x @ w_t + bias + P[idx0, :N] + P[idx1, off1:off1+N]) (row-gathered node terms)."""
    M, K = x.shape
    K2, N = w_t.shape
    if K != K2 or idx0.numel() != M or idx1.numel() != M:
        raise RuntimeError("linear_gather: shape mismatch")
    if isinstance(w_t, PackedWeight):
        if _split_ok(x, w_t):
            _gemm_bf16x(x, w_t, out, bias, epilogue, out2, None, P, idx0, idx1, off1)
            return out
        w_t = w_t.w_t
    probe = _gemm_probe
    if probe is not None:
        c_passes = 1 + (epilogue in (EPI_ACCUM, EPI_PRE_SILU, EPI_SILU_GRAD))
        probe.before(2.0 * M * N * K, 4.0 * (M * K + K * N + (c_passes + 2) * M * N), "f32")
    _call("tta_gemm_f32_gather", x.data_ptr(), w_t.data_ptr(), out.data_ptr(),
          None if bias is None else _ptr(bias, numel=N, name="bias"),
          None if out2 is None else out2.data_ptr(), None, M, N, K, _ld(x, "x"),
          _ld(w_t, "w_t"), _ld(out, "out"), _ptr(P, name="P"), _ld(P, "P"),
          _i32(idx0, M), _i32(idx1, M), off1, P.shape[0], epilogue, _stream())
    if probe is not None:
        probe.after()
    return out


def orb_edge_features(pos, send, recv, shift, r_max, nb, vec, feat, cut):
    N = pos.shape[0]
    E = send.numel()
    _call("tta_orb_edge_features", _ptr(pos, numel=N * 3, name="pos"), _i32(send, E),
          _i32(recv, E), None if shift is None else _ptr(shift, numel=E * 3, name="shift"),
          float(r_max), nb, _ptr(vec, numel=E * 3), _ptr(feat, numel=E * nb * 16),
          _ptr(cut, numel=E), N, E, _stream())


def orb_edge_features_bwd(vec, g_feat, g_cut, r_max, nb, g_vec):
    E = vec.shape[0]
    _call("tta_orb_edge_features_bwd", _ptr(vec, numel=E * 3), _ptr(g_feat, numel=E * nb * 16),
          _ptr(g_cut, numel=E), float(r_max), nb, _ptr(g_vec, numel=E * 3), E, _stream())


def rms_residual(h, w, x_old, u, x_new, inv, attn_w=None, attn_b=None, sig=None, eps=1e-6):
    R, C = h.shape
    n = R * C
    nbytes = 4 * (n * (1 + (x_old is not None) + (u is not None) + (x_new is not None)) + C
                  + R * ((inv is not None) + 2 * (sig is not None)))
    _hbm_call("k_rms_residual", nbytes, "tta_rms_residual", _ptr(h, numel=n, name="h"),
              _ptr(w, numel=C, name="w"),
              None if x_old is None else _ptr(x_old, numel=n, name="x_old"),
              None if u is None else _ptr(u, numel=n, name="u"),
              None if x_new is None else _ptr(x_new, numel=n, name="x_new"),
              None if inv is None else _ptr(inv, numel=R, name="inv"),
              None if attn_w is None else _ptr(attn_w, numel=2 * C, name="attn_w"),
              None if attn_b is None else _ptr(attn_b, numel=2, name="attn_b"),
              None if sig is None else _ptr(sig, numel=2 * R, name="sig"), R, C, float(eps),
              _stream())


def rms_bwd(g, h, w, inv, g_h):
    R, C = h.shape
    _hbm_call("k_rms_bwd", 4 * (3 * R * C + R + C), "tta_rms_bwd",
              _ptr(g, numel=R * C, name="g"), _ptr(h, numel=R * C, name="h"),
              _ptr(w, numel=C, name="w"), _ptr(inv, numel=R, name="inv"),
              _ptr(g_h, numel=R * C, name="g_h"), R, C, _stream())


def orb_segsum(ue, sig, cut, send_ptr, recv_ptr, recv_perm, nodes, node_in):
    N, C = nodes.shape
    E = ue.shape[0]
    # each edge row feeds two sums (sender order, then receiver order through recv_perm)
    nbytes = 4 * (2 * E * C + 5 * E + 2 * (N + 1) + 4 * N * C)
    _hbm_call("k_segsum", nbytes, "tta_orb_segsum", _ptr(ue, numel=E * C, name="ue"),
              _ptr(sig, numel=2 * E, name="sig"), _ptr(cut, numel=E, name="cut"),
              _i32(send_ptr, N + 1), _i32(recv_ptr, N + 1), _i32(recv_perm, E),
              _ptr(nodes, numel=N * C, name="nodes"),
              _ptr(node_in, numel=N * 3 * C, name="node_in"), N, E, C, _stream(),
              compulsory=nbytes - 4 * E * C)


def orb_edge_bwd(g_e, g_node_in, ue, sig, cut, h2, inv, wn, attn_w, send, recv, g_h2, g_cut):
    E, C = ue.shape
    N = g_node_in.shape[0]
    n = E * C
    # g_e read and rewritten, two gathered node-row slices per edge, ue, h2, g_h2
    nbytes = 4 * (7 * n + 8 * E + 3 * C)
    _hbm_call("k_edge_bwd", nbytes, "tta_orb_edge_bwd", _ptr(g_e, numel=n, name="g_e"),
              _ptr(g_node_in, numel=N * 3 * C, name="g_node_in"), _ptr(ue, numel=n),
              _ptr(sig, numel=2 * E), _ptr(cut, numel=E), _ptr(h2, numel=n),
              _ptr(inv, numel=E), _ptr(wn, numel=C), _ptr(attn_w, numel=2 * C), _i32(send, E),
              _i32(recv, E), _ptr(g_h2, numel=n, name="g_h2"),
              _ptr(g_cut, numel=E, name="g_cut"), N, E, C, _stream(),
              compulsory=nbytes - 4 * 2 * n + 4 * 2 * N * C)


def orb_node_segsum2(x, send_ptr, recv_ptr, recv_perm, out):
    E, H = x.shape
    N = out.shape[0]
    nbytes = 4 * (2 * E * H + E + 2 * (N + 1) + 2 * N * H)
    _hbm_call("k_node_segsum2", nbytes, "tta_orb_node_segsum2", _ptr(x, numel=E * H, name="x"),
              _i32(send_ptr, N + 1), _i32(recv_ptr, N + 1), _i32(recv_perm, E),
              _ptr(out, numel=N * 2 * H, name="out"), N, E, H, _stream(),
              compulsory=nbytes - 4 * E * H)


def segment_mean(x, ptr, out):
    K, C = out.shape
    _call("tta_segment_mean", _ptr(x, name="x"), _i32(ptr, K + 1), _ptr(out, numel=K * C), K, C,
          _stream())


def segment_mean_bwd(g, batch, ptr, out):
    N, C = out.shape
    K = ptr.numel() - 1
    _call("tta_segment_mean_bwd", _ptr(g, numel=K * C, name="g"), _i32(batch, N), _i32(ptr, K + 1),
          _ptr(out, numel=N * C), N, C, _stream())


def segment_center(x, ptr, out):
    """out[n] = x[n] - mean of x over n's system, systems the row ranges [ptr[k], ptr[k+1])
    (ptr[K] must equal the row count); out may be x itself."""
    N, C = out.shape
    K = ptr.numel() - 1
    _call("tta_segment_center", _ptr(x, numel=N * C, name="x"), _i32(ptr, K + 1),
          _ptr(out, numel=N * C, name="out"), K, C, _stream())
    return out


def add_rows(x, y):
    """y += x for 2-D row-strided views of equal shape."""
    R, C = y.shape
    if tuple(x.shape) != (R, C):
        raise RuntimeError("add_rows: shape mismatch")
    ldx, ldy = _ld(x, "x"), _ld(y, "y")
    _call("tta_add_rows", _rows(x, R, ldx, C, "x"), ldx, _rows(y, R, ldy, C, "y"), ldy, R, C,
          _stream())
