#!/usr/bin/env python
"""Headline benchmark: energy + conservative forces of the uma-s-1-architecture eSCN-MD model
(random-init weights) on the 2,048-atom C3 cluster, one MI355X, fp32.

``--workload c4`` runs the same model on the periodic FCC Cu supercell with stress and
``--workload c5`` the Orb-v3 architecture on the 256-molecule batch; the default line (C3) is the
headline metric, the others are secondary measurements.

A step is positions -> (energy, forces) with a fixed topology (the neighbour list is built once,
as in the reference's traced-MD convention): Wigner/edge geometry, edge-degree init, 4 eSCN-MD
blocks, energy head, the full reverse pass and the geometric VJP, all in HIP kernels.
``value`` = atoms * steps / wall time of the timed steps (atom-steps/s).

Also reported on the same JSON line:
  roofline      the dominant kernel (the split MFMA GEMM that runs the edge-level
                contractions at fp32 accuracy): algorithmic FLOPs (2MNK) of its launches / their
                HIP-event durations (recorded on the launch stream during a second pass of the
                same K steps, so that the timed pass carries no instrumentation), against
                the ceiling of its arithmetic (fp16 dense MFMA peak 2.5 PFLOP/s / 3 plane
                products); ``traffic`` = HBM bytes per launch from rocprofv3 FETCH_SIZE +
                WRITE_SIZE when profiles/uma_c3_step_counters.txt holds them, else null.  The
                other GEMM kernel family (fp32 MFMA, node-level and short-K products) is listed
                under ``gemm_families``; ``hbm_kernels`` gives the same for the HBM-bound edge
                kernels (rotation, segment sums) against the 8 TB/s HBM peak.
  cpu_baseline  the CPU oracle (PyTorch-CPU restatement of the reference path) on a bounded sample
                of the same workload: the full 2048-atom C3 step (a 512-atom cluster of the same
                density on a slow host), one warm-up step then the median of 3, in atom-steps/s,
                with the CPU model, core counts and threads in ``sample``.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (ROOT, ROOT / "tt-atom_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "atom-steps/s (energy+forces), uma-s-1 arch 2,048 atoms; % HBM/MFMA roofline"
# MI355X published dense peaks (TFLOP/s).  The split GEMM computes an fp32-accurate product with
# 3 fp16 plane products (mode 16, the default) or 6 bf16 plane products (mode 6): its
# fp32-equivalent ceiling is the fp16 / bf16 dense peak (both 2.5 PFLOP/s) / number of products.
PEAK_FP32_MFMA = 157.3
PEAK_HBM_GBPS = 8000.0
PEAK_BF16_MFMA = 2500.0
PEAKS = {"f32": PEAK_FP32_MFMA, "f16x3": PEAK_BF16_MFMA / 3, "f16x3-panel": PEAK_BF16_MFMA / 3,
         "bf16x6": PEAK_BF16_MFMA / 6, "bf16x3": PEAK_BF16_MFMA / 3, "bf16x1": PEAK_BF16_MFMA}
KERNELS = {"f32": "gemm_f32_kernel (fp32 MFMA 16x16x4)",
           "f16x3": "gemm_bf16x_kernel<2,16> (split-fp16, 2x2 power-of-two-scaled planes / 3 "
                    "products, fp32-accurate)",
           "f16x3-panel": "gemm_f16x3_panel<KT,2> (the same split-fp16 arithmetic for K <= 128: "
                          "the radial output layer)",
           "bf16x6": "gemm_bf16x_kernel<2,6> (split-bf16, 3x3 planes / 6 products, fp32-accurate)",
           "bf16x3": "gemm_bf16x_kernel<2,3> (split-bf16, 2x2 planes / 3 products)",
           "bf16x1": "gemm_bf16x_kernel<2,1> (bf16 operands)"}
# rocprofv3 counter summary of the C3 step (per-kernel HBM bytes and MFMA counters), written by
# ``bench.py --summarize-counters`` from the profiler's CSV output; read to report counter-measured
# HBM bytes next to the algorithmic ones.
TRAFFIC_FILE = ROOT / "profiles" / "uma_c3_step_counters.txt"
# per workload: the counter summary and the profiled step's title and command
COUNTER_FILES = {"c3": TRAFFIC_FILE, "c5": ROOT / "profiles" / "orb_c5_step_counters.txt"}
COUNTER_TITLES = {
    "c3": "C3 step (uma-s-1 architecture, 2048 atoms, E = 61440)",
    "c5": "C5 step (Orb-v3 conservative architecture, 256 molecules, 10,150 atoms, E = 196,555)"}


class GemmEvents:
    """HIP events around every GEMM launch (same stream as the launch), per kernel family, and
    within a family per launch class (``part``: e.g. the gate epilogues; None = the rest)."""

    def __init__(self, torch):
        self.torch = torch
        self.kinds = {}
        self.parts = {}
        self._cur = None

    def before(self, flops, nbytes, kind="f32", part=None):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self._cur = (e, kind, part)
        for key, table in ((kind, self.kinds), ((kind, part), self.parts)):
            k = table.setdefault(key, {"pairs": [], "flops": 0.0, "nbytes": 0.0})
            k["flops"] += flops
            k["nbytes"] += nbytes

    def after(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        start, kind, part = self._cur
        self.kinds[kind]["pairs"].append((start, e))
        self.parts[(kind, part)]["pairs"].append((start, e))

    @staticmethod
    def _sum(table):
        out = {}
        for key, k in table.items():
            ms = sum(a.elapsed_time(b) for a, b in k["pairs"])
            out[key] = dict(n=len(k["pairs"]), flops=k["flops"], nbytes=k["nbytes"], ms=ms)
        return out

    def summary(self):
        return self._sum(self.kinds)

    def parts_of(self, kind):
        """{part: stats} of one family, the launches of no named class under "other"."""
        return {("other" if part is None else part): v
                for (k, part), v in self._sum(self.parts).items() if k == kind}


class HbmEvents:
    """HIP events around every HBM-bound edge kernel launch (rotation / segment kernels)."""

    def __init__(self, torch):
        self.torch = torch
        self.k = {}
        self._cur = None

    def before(self, kernel, nbytes, compulsory=None):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        self._cur = (e, kernel)
        d = self.k.setdefault(kernel, {"pairs": [], "nbytes": 0.0, "compulsory": 0.0})
        d["nbytes"] += nbytes
        d["compulsory"] += nbytes if compulsory is None else compulsory

    def after(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record()
        start, kernel = self._cur
        self.k[kernel]["pairs"].append((start, e))

    def summary(self, traffic=None):
        """Per kernel: launches, average HIP-event duration, and GB/s from (i) the compulsory
        bytes (every distinct operand byte once: the least HBM traffic the launch can have;
        ``frac`` is this one), (ii) the algorithmic per-use bytes (gathered node rows once per
        edge) and, when ``traffic`` holds the kernel, (iii) the rocprofv3 FETCH_SIZE +
        WRITE_SIZE bytes per launch of the same workload."""
        out = {}
        for name, d in self.k.items():
            ms = sum(a.elapsed_time(b) for a, b in d["pairs"])
            n = max(1, len(d["pairs"]))
            sec = ms * 1e-3 / n
            rate = (lambda b: b / sec / 1e9 if sec > 0 else 0.0)
            comp, per_use = d["compulsory"] / n, d["nbytes"] / n
            e = {"launches": len(d["pairs"]), "avg_launch_us": round(sec * 1e6, 2),
                 "compulsory_bytes_per_launch": round(comp),
                 "achieved_GBps": round(rate(comp), 1), "peak_GBps": PEAK_HBM_GBPS,
                 "frac": round(rate(comp) / PEAK_HBM_GBPS, 4),
                 "algorithmic_bytes_per_launch": round(per_use),
                 "algorithmic_GBps": round(rate(per_use), 1)}
            if traffic and name in traffic:
                e["counter_bytes_per_launch"] = round(traffic[name])
                e["counter_GBps"] = round(rate(traffic[name]), 1)
                e["counter_frac"] = round(rate(traffic[name]) / PEAK_HBM_GBPS, 4)
            out[name] = e
        return out


def build_c2(torch, N=8192):
    from tt_atom import synthetic
    ei, vec, x, g = synthetic.c2_tensors(N=N)
    return ei, vec, x, g, synthetic.c2_weights(), synthetic.jd_matrices()


def _cpu_info():
    """CPU model, physical cores and logical CPUs of this host (from /proc/cpuinfo)."""
    model, phys, logical = "unknown", set(), 0
    try:
        cur = {}
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if cur:
                    phys.add((cur.get("physical id"), cur.get("core id")))
                cur = {}
                continue
            k, v = (t.strip() for t in line.split(":", 1))
            cur[k] = v
            if k == "processor":
                logical += 1
            elif k == "model name" and model == "unknown":
                model = v
        if cur:
            phys.add((cur.get("physical id"), cur.get("core id")))
    except OSError:
        pass
    return model, len(phys) if phys and None not in next(iter(phys)) else None, logical


def _median_of_3(run):
    """One untimed warm-up call at the measured size, then the median of three timed calls (the
    CPU-baseline procedure of the reference's CPU-vs-device comparison)."""
    run()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[1], ts


def _cpu_threads(torch):
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    return threads


def _cpu_sample_note(what, dt, ts, threads):
    model, phys, logical = _cpu_info()
    return (f"{what}; one warm-up step, then the median of 3 steps ({', '.join(f'{t:.2f}' for t in ts)}"
            f" s -> {dt:.2f} s); {threads} threads on {model} ({phys} physical cores, {logical} "
            f"logical CPUs visible)")


def cpu_baseline_c2(torch):
    """Oracle on a bounded sample of C2: the same pipeline on N = 2048 nodes (E = 51,200)."""
    from oracle import uma as U
    threads = _cpu_threads(torch)
    ei, vec, x, g, w, jd = build_c2(torch, N=2048)

    def run():
        ev = torch.from_numpy(vec).requires_grad_(True)
        out = U.isolated_edgewise(torch.from_numpy(x), ev, torch.from_numpy(ei[0]),
                                  torch.from_numpy(ei[1]), w, "c2", jd, 2048)
        torch.autograd.grad((out * torch.from_numpy(g)).sum(), ev)
    dt, ts = _median_of_3(run)
    E = int(ei.shape[1])
    return {"value": round(E / dt, 1), "unit": "edge-steps/s", "cores": threads, "kind": "port",
            "sample": _cpu_sample_note(f"CPU oracle (torch-CPU fp32) of the C2 pipeline on "
                                       f"N=2048 nodes (E={E})", dt, ts, threads)}


def build_c3(torch, n_atoms=2048, seed=None):
    from tt_atom import geometry, synthetic
    cfg = dict(synthetic.CFG_UMA_S)
    w, host = synthetic.random_uma_bundle(cfg, synthetic.SEEDS["C3"] + synthetic.WEIGHT_SEED_OFFSET)
    radius = 17.0 * (n_atoms / 2048.0) ** (1.0 / 3.0)
    pos, Z = synthetic.c3_system(seed=synthetic.SEEDS["C3"] if seed is None else seed,
                                 n=n_atoms, radius=radius)
    pos, Z = torch.from_numpy(pos), torch.from_numpy(Z)
    t0 = time.perf_counter()
    ei, shift = geometry.radius_graph(pos, cfg["cutoff"], max_neighbors=cfg["max_neighbors"])
    nl_ms = (time.perf_counter() - t0) * 1e3
    se = geometry.csd_embedding(w, torch.tensor([0.0]), torch.tensor([1.0]), dataset=cfg["task"])
    se = se.expand(len(Z), -1).contiguous()
    return cfg, w, host, pos, Z, ei, se, nl_ms


def build_c4(torch):
    from tt_atom import geometry, synthetic
    cfg = dict(synthetic.CFG_UMA_S, task="omat")
    w, host = synthetic.random_uma_bundle(cfg, synthetic.SEEDS["C3"] + synthetic.WEIGHT_SEED_OFFSET)
    pos, Z, cell = synthetic.c4_system()
    pos, Z = torch.from_numpy(pos), torch.from_numpy(Z)
    t0 = time.perf_counter()
    ei, shift = geometry.radius_graph(pos, cfg["cutoff"], cell, [True] * 3,
                                      max_neighbors=cfg["max_neighbors"])
    nl_ms = (time.perf_counter() - t0) * 1e3
    se = geometry.csd_embedding(w, torch.tensor([0.0]), torch.tensor([0.0]), dataset=cfg["task"])
    se = se.expand(len(Z), -1).contiguous()
    return cfg, w, host, pos, Z, ei, shift, se, cell, nl_ms


def build_c5(torch, K=256):
    from tt_atom import orb, synthetic
    cfg = dict(synthetic.CFG_ORB_C5)
    w = synthetic.random_orb_weights(cfg, synthetic.SEEDS["C5"] + synthetic.WEIGHT_SEED_OFFSET)
    systems = synthetic.c5_systems(K=K)
    t0 = time.perf_counter()
    bg = orb.assemble_orb(systems, cfg["cutoff"], cfg["max_num_neighbors"], truncate=True)
    nl_ms = (time.perf_counter() - t0) * 1e3
    return cfg, w, bg, nl_ms


def c5_cap_report(torch, cfg, bg, K=256):
    """How the C5 graph relates to the reference's rule, which refuses a system with an atom of
    sender or receiver degree above max_num_neighbors (disjoint.py:188-197): the degrees of the
    uncapped graph and the edges the per-sender cap (assemble_orb(truncate=True)) dropped."""
    from tt_atom import orb, synthetic
    full = orb.assemble_orb(synthetic.c5_systems(K=K), cfg["cutoff"], 1 << 30, truncate=True)
    n = int(full.pos.shape[0])
    deg = max(int(torch.bincount(full.senders, minlength=n).max()),
              int(torch.bincount(full.receivers, minlength=n).max()))
    kept, total = int(bg.senders.numel()), int(full.senders.numel())
    return {"max_num_neighbors": int(cfg["max_num_neighbors"]), "max_degree_uncapped": deg,
            "edges_uncapped": total, "edges_kept": kept, "edges_dropped_by_cap": total - kept,
            "reference_would_refuse": deg > int(cfg["max_num_neighbors"])}


# Published small-batch throughputs of the reference (p150a card, bf16; docs/perf_baselines.json,
# CHANGELOG.md:79-85): evaluate_batch end to end, systems per second.
PUBLISHED_BATCH = {"uma-s-1 omol K=8 ethanol": 111.06617871436099,
                   "orb-v3-conservative-omol K=8 ethanol": 463.91522419389514,
                   "orb-v3-conservative-inf-omat K=8 Si 2x1x1": 374.4622548238998,
                   "orb-v3-conservative-omol K=128 ethanol": 1338.0,
                   "orb-v3-direct-omol K=128 ethanol": 2056.0}
# covalent radii (A) of the elements in these inputs, for the Orb ZBL term (ASE's table has the
# same values; ase is not installed here)
_RADII = {1: 0.31, 6: 0.76, 7: 0.71, 8: 0.66, 14: 1.11}


def run_batch_workload(args, torch):
    """Small-system throughput, as the reference's release gate measures it: K systems per
    evaluate_batch call (host neighbour lists and assembly, the device step, the host readout
    with normalisers and ZBL), median of 5 calls after 2 warm-up calls."""
    import tempfile
    import numpy as np
    from tt_atom import calculator, orb, orb_calculator, synthetic, weights
    td = pathlib.Path(tempfile.mkdtemp())
    radii = np.ones(120)
    for z, r in _RADII.items():
        radii[z] = r

    def timed(fn):
        for _ in range(2):
            fn()
        ts = []
        for _ in range(5):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2]

    res = {}
    cfg = dict(synthetic.CFG_UMA_S)
    w, host = synthetic.random_uma_bundle(cfg, synthetic.SEEDS["C3"] + synthetic.WEIGHT_SEED_OFFSET)
    weights.save_bundle(td / "uma.npz", cfg, w, host)
    uma = calculator.Session(str(td / "uma.npz"), precision=args.precision)
    eth8 = synthetic.ethanol_batch(8)
    t = timed(lambda: uma.evaluate_batch(eth8))
    res["uma-s-1 omol K=8 ethanol"] = (8 / t, t * 1e3)

    def orb_session(name, direct, cond, cap):
        c = dict(synthetic.CFG_ORB_C5, has_charge_spin_cond=cond, max_num_neighbors=cap,
                 task="omol" if cond else "omat")
        ow = synthetic.random_orb_weights(c, synthetic.SEEDS["C5"] + synthetic.WEIGHT_SEED_OFFSET,
                                          direct=direct)
        orb.save_orb_bundle(td / f"{name}.npz", c, ow)
        return orb_calculator.OrbSession(str(td / f"{name}.npz"), precision=args.precision,
                                         covalent_radii=radii)

    cons_omol = orb_session("cons_omol", False, True, 120)
    t = timed(lambda: cons_omol.evaluate_batch(eth8))
    res["orb-v3-conservative-omol K=8 ethanol"] = (8 / t, t * 1e3)
    si8 = synthetic.si_batch(8)
    cons_omat = orb_session("cons_omat", False, False, 1 << 20)
    t = timed(lambda: cons_omat.evaluate_batch(si8))
    res["orb-v3-conservative-inf-omat K=8 Si 2x1x1"] = (8 / t, t * 1e3)
    eth128 = synthetic.ethanol_batch(128)
    t = timed(lambda: cons_omol.evaluate_batch(eth128))
    res["orb-v3-conservative-omol K=128 ethanol"] = (128 / t, t * 1e3)
    dir_omol = orb_session("dir_omol", True, True, 120)
    t = timed(lambda: dir_omol.evaluate_batch(eth128))
    res["orb-v3-direct-omol K=128 ethanol"] = (128 / t, t * 1e3)

    head = "uma-s-1 omol K=8 ethanol"
    out = {
        "metric": "systems/s, evaluate_batch end to end (K=8 rattled ethanol, uma-s-1 "
                  "architecture, energy + forces)",
        "value": round(res[head][0], 2),
        "unit": "systems/s",
        "n_gpus": 1,
        "steps": 5,
        "warmup": 2,
        "ms_per_step": round(res[head][1], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(res[head][0] / PUBLISHED_BATCH[head], 2),
        "dtype": "bf16" if args.precision == "bf16" else "f32",
        "data": "synthetic: random-init weights of the named architectures; rattled CH3CH2OH "
                "(G2) and diamond Si 2x1x1 as the reference's release gate builds them",
        "config": {"workload": "small-system batches (reference docs/perf_baselines.json)",
                   "precision": args.precision,
                   "batches": {k: {"systems_per_s": round(v[0], 1),
                                   "ms_per_call": round(v[1], 3),
                                   "published_systems_per_s_p150a": PUBLISHED_BATCH[k],
                                   "ratio": round(v[0] / PUBLISHED_BATCH[k], 2)}
                               for k, v in res.items()}},
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def direct_c5_ms(torch, cfg, bg, precision, steps):
    """ms per step of a direct Orb checkpoint of the C5 architecture (same random draw plus the
    force and stress heads) on the C5 batch: forward, ForceHead and StressHead, replayed graph."""
    from tt_atom import orb, synthetic
    w = synthetic.random_orb_weights(cfg, synthetic.SEEDS["C5"] + synthetic.WEIGHT_SEED_OFFSET,
                                     direct=True)
    mdl = orb.OrbModel(w, cfg, precision=precision)
    graph = orb.OrbGraph(mdl.device, senders=bg.senders, receivers=bg.receivers,
                         num_nodes=bg.pos.shape[0], atomic_numbers=bg.Z,
                         cell_shift=bg.cell_shift, natoms=bg.natoms)
    eng = orb.OrbEngine(mdl, graph)
    p = bg.pos.to(mdl.device)
    for _ in range(4):
        eng.step(p, compute_stress=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.step(p, compute_stress=True)
    torch.cuda.synchronize()
    return round((time.perf_counter() - t0) * 1e3 / steps, 3)


def device_nl_ms(torch, fn, ref):
    """Median wall time of the device neighbour list (after one warm-up call), and whether it
    reproduced the host graph ``ref`` = (edge_index, shift) exactly."""
    out = fn()
    same = torch.equal(out[0].cpu(), ref[0]) and torch.equal(out[1].cpu().float(),
                                                               ref[1].float())
    ts = []
    for _ in range(5):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    return round(sorted(ts)[2], 3), same


def run_neighbor_workload(args, torch):
    """Device neighbour list, row scan against cell list (same graph, checked edge for edge): one
    JSON line per system and cap with the median wall time of a whole radius_graph_device call
    (host grid set-up, passes, edge-count read-back) over --steps calls after one warm-up."""
    from tt_atom import geometry, synthetic
    cases = [("cluster", synthetic.lattice_cluster(n, 2.2, 2), None, None)
             for n in (2048, 8192, 16384, 52000, 200000)]
    cases += [(name, *synthetic.shuffled_fcc(reps, 7), pbc)
              for name, pbc in (("crystal", [True] * 3), ("slab", [True, True, False]))
              for reps in (8, 24)]
    for name, pos, cell, pbc in cases:
        pos = torch.from_numpy(pos)
        cell = None if cell is None else torch.from_numpy(cell)
        for cap in (None, 30):
            row = {"metric": "neighbor_list_ms", "system": name, "atoms": int(pos.shape[0]),
                   "pbc": pbc, "cutoff": 6.0, "cap": cap, "data": "synthetic"}
            out = {}
            for method in ("rows", "cells"):
                if method == "rows" and pos.shape[0] > 60000:
                    continue                      # O(N^2): skipped at 200k atoms
                fn = lambda: geometry.radius_graph_device(pos, 6.0, cell, pbc,
                                                          max_neighbors=cap, method=method)
                out[method] = fn()
                ts = []
                for _ in range(max(1, args.steps)):
                    torch.cuda.synchronize()
                    t0 = time.perf_counter()
                    fn()
                    torch.cuda.synchronize()
                    ts.append((time.perf_counter() - t0) * 1e3)
                row[f"{method}_ms"] = round(sorted(ts)[len(ts) // 2], 3)
            row["edges"] = int(out["cells"][0].shape[1])
            if "rows" in out:
                row["same"] = bool(torch.equal(out["rows"][0], out["cells"][0])
                                   and torch.equal(out["rows"][1], out["cells"][1]))
            print(json.dumps(row), flush=True)


def cpu_baseline_c5(torch):
    """Orb CPU oracle on a bounded sample of C5: the first 32 molecules of the batch."""
    from oracle import orb as O
    threads = _cpu_threads(torch)
    cfg, w, bg, _ = build_c5(torch, K=32)
    args = (w, cfg, bg.pos, bg.Z, bg.senders, bg.receivers, bg.cell_shift, bg.batch, bg.natoms)
    dt, ts = _median_of_3(lambda: O.energy_and_forces(*args))
    n = int(bg.pos.shape[0])
    return {"value": round(n / dt, 3), "unit": "atom-steps/s", "cores": threads, "kind": "port",
            "sample": _cpu_sample_note(f"Orb CPU oracle (torch-CPU fp32), first 32 C5 molecules "
                                       f"({n} atoms, E={int(bg.senders.numel())})", dt, ts,
                                       threads)}


def cpu_baseline(torch):
    """CPU oracle on a bounded sample of the C3 workload: the full 2048-atom step when the host
    runs it in under 12 s (the warm-up step measures that), else a 512-atom cluster of the same
    density, so that the four steps stay within about half a minute."""
    from oracle import forces as OF
    threads = _cpu_threads(torch)
    for n_atoms in (2048, 512):
        cfg, w, host, pos, Z, ei, se, _ = build_c3(torch, n_atoms=n_atoms)
        m = OF.Model(w, cfg, host)
        run = lambda: OF.energy_and_forces(m, pos, Z, ei, se)
        t0 = time.perf_counter()
        run()                                                # warm-up at the measured size
        if time.perf_counter() - t0 < 12.0 or n_atoms == 512:
            break
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    dt = sorted(ts)[1]
    return {"value": round(len(Z) / dt, 3), "unit": "atom-steps/s", "cores": threads,
            "kind": "port",
            "sample": _cpu_sample_note(f"CPU oracle (torch-CPU restatement of the reference "
                                       f"path), C3 model on a {len(Z)}-atom same-density cluster "
                                       f"(E={ei.shape[1]})", dt, ts, threads)}


def read_traffic(path=TRAFFIC_FILE):
    """{kernel: HBM bytes per launch} and {kernel: MFMA counter figures} from the ``traffic`` and
    ``mfma`` lines of a counter summary written by ``--summarize-counters``."""
    traffic, mfma = {}, {}
    if not path.exists():
        return traffic, mfma
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == "traffic":
            traffic[parts[1]] = float(parts[2])
        elif len(parts) >= 3 and parts[0] == "mfma":
            mfma[parts[1]] = {k: float(v) for k, v in (t.split("=") for t in parts[2:])}
    return traffic, mfma


def _kernel_names(full):
    """(variant, base) of a profiler kernel name: 'void (anonymous namespace)::k<2, 9>(float..)'
    -> ('k<2,9>', 'k')."""
    n = full.replace("(anonymous namespace)::", "")
    if n.startswith("void "):
        n = n[5:]
    depth, end = 0, len(n)
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            end = i
            break
    variant = n[:end].replace(" ", "")
    return variant, variant.split("<", 1)[0]


def _read_pmc(d):
    """rocprofv3 --pmc CSV rows under directory d -> {dispatch: {kernel, counters{}, ns}}."""
    import csv
    rows = {}
    for f in sorted(pathlib.Path(d).rglob("*counter_collection.csv")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                key = (str(f), r["Dispatch_Id"])
                e = rows.setdefault(key, {"kernel": r["Kernel_Name"], "c": {},
                                          "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
                e["c"][r["Counter_Name"]] = e["c"].get(r["Counter_Name"], 0.0) + float(
                    r["Counter_Value"])
    return rows


def summarize_counters(root, out_path, workload="c3"):
    """Per-kernel HBM bytes and MFMA counters of a profiled step (C3 or C5).

    ``root`` holds the rocprofv3 --pmc output of five runs: step_FETCH_SIZE, step_WRITE_SIZE and
    step_MFMA (the step under ``--pmc FETCH_SIZE``, ``WRITE_SIZE`` and ``MfmaUtil MfmaFlopsF16
    MfmaFlopsF32``)
    and copy_FETCH_SIZE, copy_WRITE_SIZE (``--calibrate-copy``: a 256 MiB read + 256 MiB write
    copy kernel).  Bytes = counter KiB x 1024 x (the copy's known bytes / what the same counter
    reads for it)."""
    root = pathlib.Path(root)
    copy_bytes = 256 * 1024 * 1024
    scale = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = [e["c"].get(c, 0.0) for e in _read_pmc(root / f"copy_{c}").values()]
        scale[c] = copy_bytes / (max(vals) * 1024.0)
    per = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        for e in _read_pmc(root / f"step_{c}").values():
            v, b = _kernel_names(e["kernel"])
            for k in {v, b}:
                d = per.setdefault(k, {"FETCH_SIZE": [], "WRITE_SIZE": [], "variant": k == v})
                d[c].append(e["c"].get(c, 0.0))
    mf = {}
    mdir = root / "step_MFMA"
    if mdir.exists():
        for e in _read_pmc(mdir).values():
            v, _ = _kernel_names(e["kernel"])
            d = mf.setdefault(v, {"util": [], "flops": [], "ns": []})
            d["util"].append(e["c"].get("MfmaUtil", 0.0))
            d["flops"].append(sum(e["c"].get(c, 0.0) for c in
                                  ("MfmaFlopsF16", "MfmaFlopsBF16", "MfmaFlopsF32")))
            d["ns"].append(e["ns"])
    lines = [f"# rocprofv3 counters of the {COUNTER_TITLES[workload]}, MI355X",
             "# Commands (repository root $REPO on the GPU box; one pass per counter group):",
             "#   cd /tmp && export TMPDIR=/tmp"]
    wl_arg = "" if workload == "c3" else f" --workload {workload}"
    step = (f"python3 $REPO/bench.py{wl_arg} --steps 1 --warmup 1 --no-cpu-baseline --no-secondary "
            "--eager")
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        lines.append(f"#   rocprofv3 --pmc {c} --output-format csv -d $REPO/gpurun_out/{root.name}/"
                     f"step_{c} -o s -- {step}")
    lines.append("#   rocprofv3 --pmc MfmaUtil MfmaFlopsF16 MfmaFlopsF32 --output-format csv -d "
                 f"$REPO/gpurun_out/{root.name}/step_MFMA -o s -- {step}")
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        lines.append(f"#   rocprofv3 --pmc {c} --output-format csv -d $REPO/gpurun_out/{root.name}/"
                     f"copy_{c} -o c -- python3 $REPO/bench.py --calibrate-copy")
    lines.append(f"#   python3 $REPO/bench.py{wl_arg} --summarize-counters $REPO/gpurun_out/"
                 f"{root.name} {pathlib.Path(out_path).as_posix()}")
    lines.append(f"# Calibration (256 MiB copy): FETCH_SIZE x {scale['FETCH_SIZE']:.4f}, "
                 f"WRITE_SIZE x {scale['WRITE_SIZE']:.4f}")
    lines.append("# Three steps are profiled (warm-up, timed, probed); figures are means per launch.")
    lines.append("#")
    lines.append("# kernel | launches | FETCH KiB raw | WRITE KiB raw | HBM MB per launch "
                 "(scaled read + write)")
    traffic = []
    for k, d in sorted(per.items(), key=lambda kv: -sum(kv[1]["FETCH_SIZE"])):
        n = len(d["FETCH_SIZE"])
        if n == 0 or len(d["WRITE_SIZE"]) != n or "::" in k or k.startswith("__"):
            continue                       # library kernels only (torch / rocprim / runtime copies)
        fk, wk = sum(d["FETCH_SIZE"]) / n, sum(d["WRITE_SIZE"]) / n
        nbytes = 1024.0 * (fk * scale["FETCH_SIZE"] + wk * scale["WRITE_SIZE"])
        if d["variant"]:
            lines.append(f"#   {k} | {n} | {fk:.1f} | {wk:.1f} | {nbytes / 1e6:.1f}")
        traffic.append(f"traffic {k} {nbytes:.0f}")
    if mf:
        lines.append("#")
        lines.append("# MFMA counters (MfmaUtil = matrix-core busy cycles / (GUI-active cycles x "
                     "SIMDs); MfmaFlopsF16 / F32 = 512 x MOPS, the matrix work actually issued)")
        for k, d in sorted(mf.items(), key=lambda kv: -sum(kv[1]["ns"])):
            if max(d["flops"]) <= 0 or "::" in k:
                continue
            n = len(d["util"])
            util = sum(d["util"]) / n
            fl = sum(d["flops"]) / n
            us = sum(d["ns"]) / n / 1e3
            lines.append(f"#   {k} | {n} launches | MfmaUtil {util:.1f} % | {fl / 1e9:.1f} GFLOP "
                         f"issued per launch | {us:.1f} us under counters | "
                         f"{fl / (us * 1e-6) / 1e12:.0f} TFLOP/s issued")
            traffic.append(f"mfma {k} util_pct={util:.2f} issued_flops={fl:.0f} us={us:.2f}")
    pathlib.Path(out_path).write_text("\n".join(lines + traffic) + "\n")


def summarize_stats(stats_csv, out_path, workload="c3", steps=5, warmup=2):
    """Markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv of the eager step:
    the top 30 kernels by total time, with the command that produced the CSV."""
    import csv
    rows = list(csv.DictReader(open(stats_csv, newline="")))
    tot = sum(float(r["TotalDurationNs"]) for r in rows)
    nsteps = warmup + 2 * steps          # warm-up, timed pass, probed pass
    wl_arg = "" if workload == "c3" else f" --workload {workload}"
    cmd = (f"rocprofv3 --kernel-trace --stats --output-format csv -d $REPO/gpurun_out/kt_{workload} "
           f"-o {workload} -- python3 $REPO/bench.py{wl_arg} --steps {steps} --warmup {warmup} "
           "--no-cpu-baseline --no-secondary --eager")
    lines = [f"# {COUNTER_TITLES[workload]}: rocprofv3 kernel statistics, MI355X", "",
             "Command (repository root $REPO on the GPU box):", "", "```",
             "cd /tmp && export TMPDIR=/tmp", cmd,
             f"python3 $REPO/bench.py{wl_arg} --summarize-stats $REPO/gpurun_out/kt_{workload}/"
             f"{workload}_kernel_stats.csv {pathlib.Path(out_path).as_posix()}", "```", "",
             f"{nsteps} steps profiled (warm-up, timed and the probed pass, all launched kernel by "
             f"kernel); total kernel time {tot / 1e6:.2f} ms = {tot / 1e6 / nsteps:.2f} ms per step.",
             "", "| share | calls | avg us | kernel |", "|---:|---:|---:|---|"]
    for r in rows[:30]:
        name = r["Name"].replace("(anonymous namespace)::", "")
        if len(name) > 70:
            name = name[:70] + "..."
        lines.append(f"| {float(r['Percentage']):.2f}% | {r['Calls']} | "
                     f"{float(r['AverageNs']) / 1000:.1f} | `{name}` |")
    pathlib.Path(out_path).write_text("\n".join(lines) + "\n")


def summarize_trace(trace_csv, out_path, pattern):
    """Per-kernel, per-grid median durations of a rocprofv3 --kernel-trace CSV for the kernels
    whose name matches ``pattern`` (rows: kernel, workgroups, dispatches, median us)."""
    import csv
    import re
    groups = {}
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "")
            name = re.sub(r"\(.*", "", name)
            if not re.search(pattern, name):
                continue
            wgs = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            groups.setdefault((name, wgs), []).append(us)
    lines = [f"{'kernel':28s} {'workgroups':>10s} {'dispatches':>10s} {'median_us':>10s}"]
    for (name, wgs), v in groups.items():
        v.sort()
        lines.append(f"{name:28s} {wgs:10d} {len(v):10d} {v[len(v) // 2]:10.2f}")
    pathlib.Path(out_path).write_text("\n".join(lines) + "\n")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("c2", "c3", "c4", "c5", "batch", "neighbors"),
                    default="c3",
                    help="c3 (headline), c2 (isolated edgewise kernel), c4 (periodic + stress), "
                         "c5 (Orb-v3 batch), batch (small-system evaluate_batch throughput "
                         "against the reference's published numbers) or neighbors (device "
                         "neighbour list: row scan against cell list, up to 200k atoms)")
    ap.add_argument("--precision", choices=("f32", "f32-bf16x6", "f32-mfma", "bf16"), default="f32",
                    help="GEMM arithmetic: f32 (scaled split-fp16, fp32-accurate), f32-bf16x6 "
                         "(split-bf16, fp32-accurate), f32-mfma, or bf16 operands (the bf16 "
                         "variants of C2 / C5)")
    ap.add_argument("--eager", action="store_true",
                    help="launch the step kernel by kernel instead of replaying its HIP graph "
                         "(for profilers)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the secondary measurements (device neighbour list, the step with the "
                         "neighbour search, the step after a topology change, the direct Orb "
                         "checkpoint), so that a profiler sees only the warm-up, timed and probed "
                         "steps")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device copy (y = -x) for the HBM counter scale")
    ap.add_argument("--summarize-counters", nargs=2, metavar=("PMC_ROOT", "OUT"),
                    help="write the per-kernel counter summary of rocprofv3 --pmc runs (no GPU)")
    ap.add_argument("--summarize-stats", nargs=2, metavar=("STATS_CSV", "OUT"),
                    help="write the markdown kernel table of a rocprofv3 --stats run of the eager "
                         "step (--steps 5 --warmup 2) (no GPU)")
    ap.add_argument("--summarize-trace", nargs=3, metavar=("TRACE_CSV", "OUT", "REGEX"),
                    help="write per-kernel, per-grid median durations of a rocprofv3 kernel "
                         "trace for kernels matching REGEX (no GPU)")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
        return
    if args.summarize_stats:
        summarize_stats(*args.summarize_stats, workload=args.workload or "c3")
        return
    if args.summarize_counters:
        summarize_counters(*args.summarize_counters, workload=args.workload or "c3")
        return
    if args.calibrate_copy:
        import torch
        x = torch.randn(64 * 1024 * 1024, device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        torch.neg(x, out=y)                       # reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": x.numel() * 4, "copy_bytes_written": y.numel() * 4}))
        return
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU; --gpus must be 1 (multi-GPU sharding is a "
              "design note only)", file=sys.stderr)
        sys.exit(2)

    import torch
    from tt_atom import _native

    wl = args.workload
    if wl == "batch":
        run_batch_workload(args, torch)
        return
    if wl == "neighbors":
        run_neighbor_workload(args, torch)
        return
    if wl == "c2":
        from tt_atom.edgewise import EdgewiseStep
        ei, vec, x, g, w, jd = build_c2(torch)
        nl_ms = 0.0
        nl_dev = None
        st = EdgewiseStep(w, "c2", jd, ei[0], ei[1], 8192, precision=args.precision)
        x_d = torch.from_numpy(x).cuda()
        ev_d = torch.from_numpy(vec).cuda()[st.order].contiguous()
        g_d = torch.from_numpy(g).cuda()

        def step():
            st.forward(x_d, ev_d)
            st.backward(x_d, g_d)
        step_eager = step
        n_atoms, n_edges = 8192, int(ei.shape[1])
        energy_of = lambda: float(st.out.abs().sum())
        forces_of = lambda: st.g_ev
    elif wl in ("c3", "c4"):
        from tt_atom import geometry, model, trace
        if wl == "c3":
            cfg, w, host, pos, Z, ei, se, nl_ms = build_c3(torch)
            shift, cell = None, None
        else:
            cfg, w, host, pos, Z, ei, shift, se, cell, nl_ms = build_c4(torch)
        dev = torch.device("cuda:0")
        bb = model.Backbone(w, dev, cfg, precision=args.precision)
        geo = geometry.HostGeometry(w, cfg, host["to_m"], host["gauss_offset"],
                                    host["gauss_coeff"], device=dev)
        eng = trace.TracedEngine(bb, geo, Z, ei, se, edge_cell_shift=shift)
        nl_dev = None if args.no_secondary else device_nl_ms(
            torch, lambda: geometry.radius_graph_device(
                pos, cfg["cutoff"], cell, None if cell is None else [True] * 3,
                max_neighbors=cfg["max_neighbors"]),
            (ei, shift if shift is not None else torch.zeros(ei.shape[1], 3)))
        pos_d = pos.to(dev)
        stress = wl == "c4"
        step = lambda: eng.run(pos_d, compute_stress=stress, eager=args.eager)
        step_eager = lambda: eng.run(pos_d, compute_stress=stress, eager=True)
        n_atoms, n_edges = len(Z), int(ei.shape[1])
        energy_of = lambda: float(eng.energy_buf)
        forces_of = lambda: eng.forces
    else:
        from tt_atom import orb
        cfg, w, bg, nl_ms = build_c5(torch)
        mdl = orb.OrbModel(w, cfg, precision=args.precision)
        graph = orb.OrbGraph(mdl.device, senders=bg.senders, receivers=bg.receivers,
                             num_nodes=bg.pos.shape[0], atomic_numbers=bg.Z,
                             cell_shift=bg.cell_shift, natoms=bg.natoms)
        eng = orb.OrbEngine(mdl, graph)
        from tt_atom import synthetic as syn
        systems = syn.c5_systems(K=256)
        ref_bg = bg
        nl_dev = None if args.no_secondary else device_nl_ms(
            torch, lambda: (lambda g: (torch.stack([g.receivers, g.senders]), g.cell_shift))(
                orb.assemble_orb(systems, cfg["cutoff"], cfg["max_num_neighbors"], "device",
                                 truncate=True)),
            (torch.stack([ref_bg.receivers, ref_bg.senders]), ref_bg.cell_shift))
        pos_d = bg.pos.to(mdl.device)

        step = lambda: eng.step(pos_d, eager=args.eager)
        step_eager = lambda: eng.step(pos_d, eager=True)
        n_atoms, n_edges = int(bg.pos.shape[0]), int(bg.senders.numel())
        energy_of = lambda: float(eng.raw.sum())
        forces_of = lambda: eng.forces
    # a graph-replayed step runs eagerly on its first call and is captured on its second: two
    # preparation calls, so that the W warm-up steps and the timed steps are all replays
    if not args.eager and wl != "c2":
        step()
        step()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print(f"[bench] {wl} warm-up done: N={n_atoms} E={n_edges} energy={energy_of():.6f}",
          file=sys.stderr, flush=True)

    # timed region: K steps between two device synchronisations, no instrumentation
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    # the same K steps again, launched kernel by kernel (not through the step graph) with HIP
    # events recorded around every GEMM and HBM-bound edge-kernel launch on the launch stream
    # (kernel durations for the roofline; the extra host calls of the events would otherwise
    # inflate the timed step)
    probe = GemmEvents(torch)
    hbm = HbmEvents(torch)
    _native.set_gemm_probe(probe)
    _native.set_hbm_probe(hbm)
    for _ in range(args.steps):
        step_eager()
    torch.cuda.synchronize()
    _native.set_gemm_probe(None)
    _native.set_hbm_probe(None)
    # secondary (C3 / C4): the step with the neighbour search in it -- device radius graph and a
    # topology comparison every step, then the replay (the topology does not change here) -- and
    # the cost of a step whose topology did change (new engine, first call launched eagerly)
    nl_step_ms = topo_step_ms = direct_ms = cap_report = None
    if wl == "c5":
        cap_report = c5_cap_report(torch, cfg, bg)
    if wl == "c5" and not args.no_secondary:
        direct_ms = direct_c5_ms(torch, cfg, bg, args.precision, min(args.steps, 10))
    if wl in ("c3", "c4") and not args.no_secondary:
        ei_dev = ei.to(dev)

        def nl_step():
            ei_new, _ = geometry.radius_graph_device(
                pos_d, cfg["cutoff"], cell, None if cell is None else [True] * 3,
                max_neighbors=cfg["max_neighbors"])
            if not torch.equal(ei_new, ei_dev):
                raise RuntimeError("topology changed between identical steps")
            step()
        nl_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(min(args.steps, 10)):
            nl_step()
        torch.cuda.synchronize()
        nl_step_ms = round((time.perf_counter() - t0) * 1e3 / min(args.steps, 10), 3)
        ts = []
        for _ in range(2):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            e2 = trace.TracedEngine(bb, geo, Z, ei, se, edge_cell_shift=shift)
            e2.run(pos_d, compute_stress=stress)
            torch.cuda.synchronize()
            ts.append((time.perf_counter() - t0) * 1e3)
            del e2
        topo_step_ms = round(min(ts), 3)
    energy = energy_of()
    if not (energy == energy) or not bool(torch.isfinite(forces_of()).all()):
        raise RuntimeError("non-finite energy or forces")
    fam = probe.summary()
    gemm_ms = sum(v["ms"] for v in fam.values())
    dom = max(fam, key=lambda k: fam[k]["ms"])
    d = fam[dom]
    achieved = d["flops"] / (d["ms"] * 1e-3) / 1e12 if d["ms"] > 0 else 0.0
    counted = wl in COUNTER_FILES and args.precision == "f32"
    kernel_traffic, kernel_mfma = read_traffic(COUNTER_FILES[wl]) if counted else ({}, {})
    dom_kernel = {"f16x3": "gemm_bf16x_kernel<2,16>"}.get(dom)
    traffic = kernel_traffic.get(dom_kernel) if dom_kernel else None
    mfma_counters = kernel_mfma.get(dom_kernel) if dom_kernel else None
    ms_step = dt / args.steps * 1e3
    others = {k: {"launches": v["n"], "avg_launch_us": round(v["ms"] * 1e3 / max(1, v["n"]), 2),
                  "achieved_tflops": round(v["flops"] / max(1e-12, v["ms"] * 1e-3) / 1e12, 2),
                  "peak_tflops": round(PEAKS[k], 1), "share_of_step": round(v["ms"] / (dt * 1e3), 4)}
              for k, v in fam.items()}
    classes = {p: {"launches": v["n"], "avg_launch_us": round(v["ms"] * 1e3 / max(1, v["n"]), 2),
                   "achieved_tflops": round(v["flops"] / max(1e-12, v["ms"] * 1e-3) / 1e12, 2),
                   "frac": round(v["flops"] / max(1e-12, v["ms"] * 1e-3) / 1e12 / PEAKS[dom], 4)}
               for p, v in probe.parts_of(dom).items()}
    unit = "atom-steps/s"
    if wl == "c2":
        metric = "edge-steps/s (forward + edge-vector VJP), isolated edgewise kernel (C2)"
        unit = "edge-steps/s"
        workload = ("C2: isolated edgewise step, N=8192 nodes, E=204800 (in-degree 25, dst-sorted, "
                    "src uniform), lmax=2, 128 channels: gather(src) -> rotate -> SO(2) conv -> "
                    "rotate back -> scatter-add, plus the VJP w.r.t. edge vectors")
        data = "synthetic (seeded C2 graph, N(0,1) features / adjoint, N(0,1/sqrt(fan_in)) weights)"
    elif wl == "c5":
        metric = "atom-steps/s (energy+forces), Orb-v3-conservative arch, 256 molecules (C5)"
        workload = ("C5: Orb-v3-conservative arch (5 layers, latent 256, MLP hidden 1024, 8 "
                    "Bessel x SH l<=3), 256 H/C/N/O molecules of 20-60 atoms in 7 A cubes, "
                    "cutoff 6 A, cap 20, energy+forces, fixed topology")
        data = "synthetic (random-init Orb-v3-conservative-architecture weights, seeded C5 batch)"
    else:
        metric = METRIC
        workload = ("C3: uma-s-1 arch (4 eSCN-MD layers, C=H=128, lmax=mmax=2, 512 gaussians, "
                    "spectral FF), 2048-atom H/C/N/O cluster in a 17 A ball, cutoff 6 A, cap 30, "
                    "energy+forces, fixed topology") if wl == "c3" else (
                    "C4: C3 weights (task omat) on FCC Cu 8x8x8 (a=3.61 A, N(0,0.05) noise), "
                    "PBC, cutoff 6 A, cap 30, energy+forces+stress, fixed topology")
        data = ("synthetic (random-init uma-s-1-architecture weights, seeded "
                f"{wl.upper()} system)")
    out = {
        "metric": metric,
        "value": round((n_edges if wl == "c2" else n_atoms) * args.steps / dt, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.precision == "bf16" else "f32",
        "data": data,
        "config": {"workload": workload, "precision": args.precision,
                   "step_launch": ("kernel sequence" if wl == "c2" or args.eager
                                   else "HIP graph replay"),
                   "atoms" if wl != "c2" else "nodes": n_atoms, "edges": n_edges,
                   "neighbor_list_host_ms": round(nl_ms, 1),
                   "neighbor_list_device_ms": None if nl_dev is None else nl_dev[0],
                   "neighbor_list_device_equals_host": None if nl_dev is None else nl_dev[1],
                   "ms_per_step_with_neighbor_search": nl_step_ms,
                   "ms_per_step_after_topology_change": topo_step_ms,
                   "direct_checkpoint_ms_per_step": direct_ms,
                   "graph_cap": cap_report,
                   "energy": energy},
        "roofline": {"bound": "mfma", "kernel": KERNELS[dom],
                     "achieved": round(achieved, 3), "peak": round(PEAKS[dom], 2),
                     "unit": "TFLOP/s", "frac": round(achieved / PEAKS[dom], 4),
                     "traffic": traffic, "launches": d["n"],
                     "mfma_counters": mfma_counters,
                     "algorithmic_bytes_per_launch": round(d["nbytes"] / max(1, d["n"])),
                     "algorithmic_flops_per_launch": round(d["flops"] / max(1, d["n"])),
                     "avg_launch_us": round(d["ms"] * 1e3 / max(1, d["n"]), 2),
                     "peak_note": ("algorithmic fp32 GEMM flops (2MNK) against the ceiling of "
                                   "the kernel's arithmetic: fp32 MFMA 157.3, or the fp16 / bf16 "
                                   "dense MFMA 2500 / number of plane products"),
                     "frac_note": ("the default split (f16x3: 3 fp16 products per fp32 "
                                   "product); the peak assumes the 2.4 GHz clock, which the part "
                                   "does not hold under this load, and each 128 x 128 tile ends "
                                   "in an epilogue that writes 64 KB (13-35 % of a tile's time "
                                   "on these shapes); the fp32-accurate bf16x6 mode reads a "
                                   "higher frac (0.43-0.44 of its /6 ceiling) at a lower rate "
                                   "(178-184 TF/s on this step, --precision f32-bf16x6)"),
                     "gemm_share_of_step": round(gemm_ms / (dt * 1e3), 4),
                     "measured": ("HIP events around each launch, on the launch stream, over a "
                                  "second pass of the same steps"),
                     "gemm_families": others,
                     "launch_classes": classes,
                     "launch_classes_note": ("the dominant family's launches split by epilogue: "
                                             "'gate' = the SO(2) conv-1 products with the gate "
                                             "applied as they are written and the conv-2 adjoint "
                                             "products with its input adjoint (the gate's "
                                             "elementwise work, which no separate pass does any "
                                             "more, counts in their time but not in their "
                                             "flops)")},
        "hbm_kernels": hbm.summary(kernel_traffic),
        "hbm_kernels_note": ("frac = compulsory bytes (every distinct operand byte once) / HIP-event "
                             "time / 8 TB/s; algorithmic_GBps counts gathered node rows once per "
                             "edge; counter_GBps uses rocprofv3 FETCH_SIZE + WRITE_SIZE bytes per "
                             "launch of the same workload ("
                             + (COUNTER_FILES[wl].relative_to(ROOT).as_posix() if counted
                                else "no counter summary for this workload") + ")"),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = (cpu_baseline_c5(torch) if wl == "c5" else
                               cpu_baseline_c2(torch) if wl == "c2" else cpu_baseline(torch))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
