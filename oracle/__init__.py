"""CPU oracle for the eSCN-MD (UMA) and Orb-v3 edgewise hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this directory; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it, and
only as the checker (or the timed CPU baseline), never as the thing that is measured or shipped.

It is a plain PyTorch-CPU restatement of the reference's CPU path (``tt_atom/geometry.py`` plus
the ``tests/mirror.py`` forward semantics, the spectral feed-forward, the edge-degree node init,
autograd forces and the strain-leaf stress).  Every function cites the reference file:line it
follows.  Parity pins (see tests/test_oracle_*.py):

* geometry + backbone + energy + forces: the committed fairchem fp32 goldens
  (``tests/golden/golden_tiny.npz``, ``golden_bulk_tiny.npz``), gauge-free quantities only;
* Wigner blocks: orthogonality, the fixture's ``Jd`` / ``to_m``, closed-form l=1 rotation;
* neighbour list: brute-force triple loop on tiny inputs with the same fp32 comparisons;
* forces / stress: fp64 finite differences and rotation/translation invariance;
* system embedding: the goldens' ``host@sys_node_embedding`` and known rand_emb / pos_emb rows;
* spectral feed-forward: constant-gate closed form and loop known answers (planted mistakes fail);
* Orb: reference-written geometry vectors, closed-form-vs-autograd geometry VJP, finite
  differences, and known answers of every layer and head from selection-matrix weights (no
  committed Orb vector of a full model exists in the reference).
"""
