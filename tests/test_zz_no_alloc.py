"""The allocation-free virial entry point (tta_virial_noalloc) against tta_virial, which takes a
caller workspace: same kernels, same reduction order, so the results are bit-identical.  Two
calls in a row, the second on a smaller input, check that the shared per-GPU scratch carries
nothing from one call to the next; an fp64 host sum checks both."""
import ctypes

import pytest
import torch

from tt_atom import _native as nat

pytestmark = pytest.mark.gpu


def _ref(ev, g):
    ev, g = ev.double().cpu(), g.double().cpu()
    v = ev.t() @ g
    return 0.5 * (v + v.t())


def test_virial_noalloc_equals_workspace_entry_point():
    dev = torch.device("cuda")
    gen = torch.Generator().manual_seed(11)
    lib = nat.load()
    for E in (61_440, 1_537, 0, 300_001, 5):
        print(f"virial_noalloc: E={E}", flush=True)
        ev = torch.randn(E, 3, generator=gen).to(dev)
        g = torch.randn(E, 3, generator=gen).to(dev)
        work = torch.full((256 * 9,), float("nan"), device=dev)
        a = torch.full((9,), float("nan"), device=dev)
        b = torch.full((9,), float("nan"), device=dev)
        nat.virial(ev, g, work, a)
        nat.virial_noalloc(ev, g, b)
        torch.cuda.synchronize()
        assert torch.equal(a, b), (E, a, b)
        r = _ref(ev, g).reshape(-1)
        tol = 1e-5 * max(1.0, float(r.abs().max())) + 1e-6 * (E ** 0.5)
        assert float((b.double().cpu() - r).abs().max()) <= tol
    # through the raw C ABI as well, on the current torch stream
    ev = torch.randn(1000, 3, generator=gen).to(dev)
    g = torch.randn(1000, 3, generator=gen).to(dev)
    out = torch.empty(9, device=dev)
    st = lib.tta_virial_noalloc(ctypes.c_void_p(ev.data_ptr()), ctypes.c_void_p(g.data_ptr()),
                                1000, ctypes.c_void_p(out.data_ptr()),
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    torch.cuda.synchronize()
    assert float((out.double().cpu() - _ref(ev, g).reshape(-1)).abs().max()) < 1e-4


def test_virial_noalloc_rejects_bad_sizes():
    lib = nat.load()
    assert lib.tta_virial_noalloc(None, None, -1, None, None) != 0
    assert b"outside" in lib.tta_last_error()
    assert lib.tta_virial_noalloc(None, None, 1 << 31, None, None) != 0
    assert lib.tta_virial_noalloc(None, None, 10, None, None) != 0
    assert b"null" in lib.tta_last_error()
