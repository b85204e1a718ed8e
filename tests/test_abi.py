"""The C-ABI library loads and exports every symbol include/tt_atom_hip.h declares (CPU only:
no compute call is made without a GPU)."""
import pathlib
import re

from tt_atom import _native

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "tt_atom_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int64_t|int)\s+(tta_\w+)\(", text, re.M)))


def test_header_and_bindings_agree():
    assert _declared() == sorted(_native.EXPORTS)


def test_library_exports_every_symbol():
    lib = _native.load_symbols_only()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.tta_version() == 1
    assert lib.tta_last_error() is not None


def test_argument_errors_are_reported_without_a_device():
    lib = _native.load_symbols_only()
    # invalid sizes are rejected on the host before any launch
    assert lib.tta_gemm_f32(None, None, None, None, None, None, -1, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0,
                            0, None) != 0
    assert b"negative" in lib.tta_last_error()
    assert lib.tta_gather_rotate(None, None, None, None, None, None, 1, 1, 6, None) != 0
    assert b"unsupported channel count" in lib.tta_last_error()


def test_walk_width_rule_matches_the_library():
    """The engine's choice between the node walks and the edge walk of the rotation backward
    (bw_walk_width_ok) is the library's own acceptance rule: for every width the walks either
    reject the channel count or get past it to the null-pointer check, before any launch."""
    lib = _native.load_symbols_only()
    accepted = []
    for C in range(1, 1025):
        ok = []
        for call, who in (
                (lambda: lib.tta_gather_rotate_bw_srcwalk(None, None, None, None, None, None, None,
                                                          None, None, 1, 1, C, None), b"srcwalk"),
                (lambda: lib.tta_gather_rotate_bw_tgtwalk(None, None, None, None, None, None, None,
                                                          None, None, None, None, 1, 1, C, None),
                 b"tgtwalk"),
                (lambda: lib.tta_gather_rotate_bw_dst(None, None, None, None, None, None, None,
                                                      None, None, None, 1, 1, C, None), b"bw_dst")):
            st = call()   # one call at a time: the error text is the last call's
            assert st != 0
            err = lib.tta_last_error()
            assert who in err
            ok.append(b"null pointer" in err)
            assert ok[-1] or b"channel count" in err
        assert ok[0] == ok[1] == ok[2] == _native.bw_walk_width_ok(C), C
        if ok[0]:
            accepted.append(C)
    assert accepted == list(range(4, 65, 4)) + [128, 256]
