"""Host logic of the functional APIs' engine cache (tt_atom/engine_cache.py): an engine is reused
while every topology input compares equal and rebuilt otherwise, including after the caller edits
its own array in place."""
import torch

from tt_atom import engine_cache


class _Owner:
    pass


def test_reuse_and_rebuild():
    owner, built = _Owner(), []

    def build():
        built.append(object())
        return built[-1]

    ei = torch.tensor([[0, 1, 2], [1, 2, 0]])
    Z = torch.tensor([1, 6, 8])
    key = lambda: (ei, Z, None, (3,), 1.5)
    e1 = engine_cache.cached_engine(owner, "s", key(), build)
    assert engine_cache.cached_engine(owner, "s", key(), build) is e1
    # equal values in new tensors: still a hit
    assert engine_cache.cached_engine(owner, "s", (ei.clone(), Z.clone(), None, [3], 1.5),
                                      build) is e1
    assert len(built) == 1
    # another slot of the same owner is independent
    e2 = engine_cache.cached_engine(owner, "t", key(), build)
    assert e2 is not e1 and engine_cache.cached_engine(owner, "s", key(), build) is e1
    # the caller edits its edge list in place: the key kept a copy, so this is a miss
    ei[0, 0] = 2
    e3 = engine_cache.cached_engine(owner, "s", key(), build)
    assert e3 is not e1 and len(built) == 3
    # dtype, shape, None-ness and scalar changes are misses
    for k in ((ei.int(), Z, None, (3,), 1.5), (ei[:, :2], Z, None, (3,), 1.5),
              (ei, Z, torch.zeros(3, 3), (3,), 1.5), (ei, Z, None, (2, 1), 1.5),
              (ei, Z, None, (3,), 2.0)):
        e = engine_cache.cached_engine(owner, "s", k, build)
        assert engine_cache.cached_engine(owner, "s", k, build) is e
    assert len(built) == 8
    engine_cache.release(owner)
    assert engine_cache.cached_engine(owner, "s", key(), build) is built[-1] and len(built) == 9
