"""tt_atom -- MI355X (gfx950) build of the eSCN-MD (UMA) and Orb-v3 edgewise hot paths.

Same module and class names as the reference package for the path it covers
(``geometry.HostGeometry``, ``geometry.radius_graph``, ``geometry.csd_embedding``,
``model.Backbone``, ``model.GraphContext``, ``forces.energy_and_forces``,
``trace.TracedEngine``, ``weights.WeightBundle``, ``calculator.TTAtomCalculator``,
``orb.OrbWeights`` / ``orb.energy_and_forces(_batch)``, ``orb_calculator.OrbCalculator``,
``bundle_cache`` / ``orb_weight_cache``, the per-op ``rotation`` / ``scatter`` entry points and the
``Calculator`` front door); the compute runs in
hand-written HIP kernels behind the C ABI of ``include/tt_atom_hip.h``.
"""
__all__ = ["geometry", "model", "forces", "trace", "weights", "synthetic", "calculator", "orb",
           "orb_calculator", "bundle_cache", "orb_weight_cache", "auto", "rotation", "scatter",
           "Calculator"]
__version__ = "0.1.0"


def __getattr__(name):
    # ``from tt_atom import Calculator`` (reference __init__), imported on first use
    if name == "Calculator":
        from .auto import Calculator
        return Calculator
    raise AttributeError(f"module 'tt_atom' has no attribute {name!r}")
