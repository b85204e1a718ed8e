"""``Calculator(atoms, model=...)``: the name-dispatching front door (reference auto.py:1-89).

``"uma-..."`` names give a ``TTAtomCalculator`` over the composition-keyed bundle cache,
``"orb-..."`` names (the four checkpoints of ``orb_weight_cache.CHECKPOINTS``) an
``OrbCalculator`` over the per-checkpoint weight cache.  Both load cached files only (see
``bundle_cache`` / ``orb_weight_cache``).
"""
from __future__ import annotations


def _family(model):
    """'uma' or 'orb' from the model name (auto.py:19-37)."""
    m = str(model).lower()
    if m.startswith("uma"):
        return "uma"
    if m.startswith("orb"):
        return "orb"
    from . import orb_weight_cache
    raise ValueError(f"unknown model {model!r}: expected a UMA model (e.g. 'uma-s-1') or an Orb "
                     f"checkpoint (one of {', '.join(orb_weight_cache.CHECKPOINTS)})")


def Calculator(atoms=None, model="uma-s-1", *, task=None, charge=0, spin=1, refenv=None,
               checkpoint=None, cache_dir=None, device=None, device_id=0, fast=False,
               trace=False, **kwargs):
    """A ready ASE calculator for ``model`` (auto.py:40-89).  UMA needs ``atoms`` (its
    composition picks the bundle) and infers the task from the cell when ``task`` is None; Orb
    takes no task or checkpoint override (the name is the checkpoint) and only stamps charge /
    spin defaults onto ``atoms``."""
    if _family(model) == "uma":
        from . import bundle_cache
        from .calculator import TTAtomCalculator
        if atoms is None:
            raise ValueError("a UMA model needs `atoms`: the merged bundle is chosen by the "
                             "reduced composition, charge, spin and task")
        if task is None:
            task = bundle_cache.infer_task(atoms)
        return TTAtomCalculator.from_uma(model=model, task_name=task, atoms=atoms, charge=charge,
                                         spin=spin, refenv=refenv, checkpoint=checkpoint,
                                         cache_dir=cache_dir, device=device, device_id=device_id,
                                         fast=fast, trace=trace, **kwargs)
    from .orb_calculator import OrbCalculator
    if task is not None:
        raise ValueError(f"`task` applies only to UMA models; the Orb checkpoint {model!r} fixes "
                         "omat vs omol itself")
    if checkpoint is not None:
        raise ValueError(f"for Orb the model name is the checkpoint (model={model!r}); drop "
                         "checkpoint=")
    if trace:
        raise ValueError("trace= is not an Orb calculator option: OrbEngine replays its step "
                         "graph by itself")
    if atoms is not None:
        atoms.info.setdefault("charge", charge)
        atoms.info.setdefault("spin", spin)
    return OrbCalculator.from_checkpoint(checkpoint=model, refenv=refenv, cache_dir=cache_dir,
                                         device=device, device_id=device_id, fast=fast, **kwargs)
