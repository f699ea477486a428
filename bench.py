"""Benchmark of the MI355X MTP E/F/S path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-train]

Workload (the metric's configuration): level-16 two-species MTP (radial
basis size 8, min_dist 1.9 A, cutoff 5.0 A, coefficients U[-0.05, 0.05],
scaling 0.01) on a 32,000-atom FCC supercell (20x20x20 conventional,
a = 3.56 A), 75/25 species, symmetric strain +-2 %, Gaussian displacements
sigma = 0.12 A; synthetic, seeded.

A step is one E/F/S evaluation (energy, forces, stress, site energies) of the
whole cell with the neighbour lists resident in HBM (the reference fastfit
"kernel" time).  `value` = atoms * K / wall time of the K timed steps.  The
roofline entry prices the dominant kernel's algorithmic fp64 flops per launch
(n_i (8R + 4MR + 4 nu_max + 38B + 24) + 9T + 2S + 2 per atom) against the
MI355X fp64 peak, over the kernel's mean duration measured with HIP events on
the library's stream.  The CPU baseline is the oracle's getEFSOMP restatement
on the host cores.  Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "imr-mlp_amd"))

from mtpx import capi  # noqa: E402
from mtpx import synth as S  # noqa: E402

METRIC = "MTP E/F/S atom-evals/s (lvl16, 32k atoms); train loss+grad configs/s"
FP64_PEAK_TFLOPS = 78.6
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "efs_kernel_lvl16_32k_traffic.json")


def efs_flops(model_text: str, n: int, P: int) -> float:
    t = S.template_topology(model_text)
    hdr = {k: int(v) for k, v in
           (l.strip().split(" = ") for l in model_text.splitlines()
            if l.strip().startswith(("radial_basis_size", "radial_funcs_count")))}
    R, M = hdr["radial_basis_size"], hdr["radial_funcs_count"]
    B, T, Sn = len(t["basic"]), len(t["times"]), len(t["map"])
    nu = int(t["basic"][:, 1:].sum(axis=1).max())
    per_pair = 8 * R + 4 * M * R + 4 * nu + 32 * B + 6 * B + 24
    per_site = 9 * T + 2 * Sn + 2
    return float(P) * per_pair + float(n) * per_site


def train_flops(model_text: str, n: int, P: int) -> float:
    """Loss+gradient per atom: E/F/S + n_i (30B + 4MR + 24) + 18T + 4S."""
    t = S.template_topology(model_text)
    hdr = {k: int(v) for k, v in
           (l.strip().split(" = ") for l in model_text.splitlines()
            if l.strip().startswith(("radial_basis_size", "radial_funcs_count")))}
    R, M = hdr["radial_basis_size"], hdr["radial_funcs_count"]
    B, T, Sn = len(t["basic"]), len(t["times"]), len(t["map"])
    return efs_flops(model_text, n, P) + float(P) * (30 * B + 4 * M * R + 24) + \
        float(n) * (18 * T + 4 * Sn)


def training_set(nconf: int):
    """Workload: level-20 three-species model (radial basis 10, cutoff 6.0),
    nconf liquid configurations of 108-216 atoms at 0.06 atoms/A^3 (minimum
    distance 1.5 A); labels are a seeded reference model's E/F/S (computed
    by this library) plus Gaussian noise (1 meV/atom, 0.05 eV/A)."""
    ref_text, start_text = S.training_models(5)
    structs = S.training_structures(5, nconf)
    for st in structs:
        st.pos = capi.wrap(st.cell, st.pbc, st.pos)
    return ref_text, start_text, structs


def train_bench(ctx, steps: int, warmup: int, nconf: int):
    ref_text, start_text, structs = training_set(nconf)
    cutoff = 6.0
    ctx.load_model_text(ref_text)
    t0 = time.perf_counter()
    off = ctx.set_structures(structs, cutoff)  # neighbour lists of every structure, once
    build_ms = 1e3 * (time.perf_counter() - t0)
    E, F, St, _ = ctx.compute_batch()
    rng = S.rng_for(5, 3)
    tE, tF, tS = [], [], []
    for c, st in enumerate(structs):
        e, f, sv = S.noisy_labels(rng, st.n, E[c], F[off[c]:off[c + 1]], St[c])
        tE.append(e)
        tF.append(f)
        tS.append(sv)
    tE, tF, tS = np.array(tE), np.concatenate(tF), np.array(tS)
    ctx.load_model_text(start_text)
    has = np.ones((nconf, 3), np.int32)
    active, wE, wF, wS = capi.loss_weights(capi.LossSettings.make(), off, has, tF)
    ctx.set_labels(active, tE, wE, tF, wF, tS, wS)
    for _ in range(warmup):
        ctx.loss_grad(penalty_weight=1e-6, reg_l2=1e-10)
    tims = []
    t0 = time.perf_counter()
    for _ in range(steps):
        f, g, met = ctx.loss_grad(penalty_weight=1e-6, reg_l2=1e-10)
        tims.append(ctx.last_train_timings())
    wall = time.perf_counter() - t0
    tims = np.array(tims)
    n, P = ctx.neighbor_count()
    flops = train_flops(start_text, n, P)
    dev_ms = float(np.mean(tims[:, 0]))
    grad_ms = float(np.mean(tims[:, 3]))
    return {
        "metric": "train loss+grad configs/s (lvl20, 3 species, %d liquid configs)" % nconf,
        "value": nconf * steps / wall, "unit": "configs/s", "steps": steps, "warmup": warmup,
        "ms_per_step": 1e3 * wall / steps,
        "config": {"workload": "loss+gradient, level-20 MTP, 3 species, R=10, cutoff 6.0, "
                               "%d liquid configs of 108-216 atoms, rho 0.06, d_min 1.5" % nconf,
                   "atoms": n, "neighbor_entries": P},
        "roofline": {"bound": "mfma", "achieved": flops / (dev_ms * 1e-3) / 1e12,
                     "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": flops / (dev_ms * 1e-3) / 1e12 / FP64_PEAK_TFLOPS, "traffic": None,
                     "kernel": "loss+grad step (efs_kernel, loss_kernel, grad_kernel)",
                     "device_ms": dev_ms, "efs_ms": float(np.mean(tims[:, 1])),
                     "loss_ms": float(np.mean(tims[:, 2])), "grad_ms": grad_ms,
                     "algorithmic_flops_per_step": flops},
        "loss": f,
        "list_build_ms": build_ms,
    }, (start_text, structs, off, tE, tF, tS, cutoff)


def linear_flops(model_text: str, n: int, P: int, rows: int) -> float:
    """Linear step: sum_i [n_i (8R + 4MR + 4nu + 32B + 12T + 24S) + 3T + 2S]
    + rows p (p + 1) + 2 rows p, p = Z + S."""
    t = S.template_topology(model_text)
    hdr = {k: int(v) for k, v in
           (l.strip().split(" = ") for l in model_text.splitlines()
            if l.strip().startswith(("radial_basis_size", "radial_funcs_count",
                                     "species_count")))}
    R, M, Z = hdr["radial_basis_size"], hdr["radial_funcs_count"], hdr["species_count"]
    B, T, Sn = len(t["basic"]), len(t["times"]), len(t["map"])
    nu = int(t["basic"][:, 1:].sum(axis=1).max())
    p = Z + Sn
    per_pair = 8 * R + 4 * M * R + 4 * nu + 32 * B + 12 * T + 24 * Sn
    return float(P) * per_pair + float(n) * (3 * T + 2 * Sn) + rows * p * (p + 1) + 2.0 * rows * p


def linear_bench(ctx, steps: int, nconf: int):
    """Workload: level-16 two-species model (radial basis 8, cutoff 5.0),
    nconf FCC/BCC structures of 64-256 atoms (strain 3 %, displacements
    0.1-0.3 A); labels from a seeded reference model (this library) plus
    noise; weights energy/force/stress 1/0.01/0.001.  A step is
    TrainLinearFast's assembly: design rows, AddLinearFast rows, Gram."""
    ref_text, start_text = S.training_models(4)
    structs = S.training_structures(4, nconf)
    for st in structs:
        st.pos = capi.wrap(st.cell, st.pbc, st.pos)
    ctx.load_model_text(ref_text)
    t0 = time.perf_counter()
    off = ctx.set_structures(structs, 5.0)  # neighbour lists of every structure, once
    build_ms = 1e3 * (time.perf_counter() - t0)
    E, F, St, _ = ctx.compute_batch()
    rng = S.rng_for(4, 3)
    tE, tF, tS = [], [], []
    for c, st in enumerate(structs):
        e, f, sv = S.noisy_labels(rng, st.n, E[c], F[off[c]:off[c + 1]], St[c])
        tE.append(e)
        tF.append(f)
        tS.append(sv)
    tE, tF, tS = np.array(tE), np.concatenate(tF), np.array(tS)
    ctx.load_model_text(start_text)
    has = np.ones((nconf, 3), np.int32)
    sets = capi.LossSettings.make(weight_energy=1.0, weight_forces=0.01, weight_stress=0.001)
    active, wE, wF, wS = capi.loss_weights(sets, off, has, tF)
    ctx.set_labels(active, tE, wE, tF, wF, tS, wS)
    ctx.linear_system()  # warm-up
    tims = []
    t0 = time.perf_counter()
    for _ in range(steps):
        G, b = ctx.linear_system()
        tims.append(ctx.last_linear_timings())
    wall = time.perf_counter() - t0
    tims = np.array(tims)
    n, P = ctx.neighbor_count()
    rows = int(tims[0, 3])
    flops = linear_flops(start_text, n, P, rows)
    dev_ms = float(np.mean(tims[:, 0]))
    return {
        "metric": "linear-fit assembly configs/s (lvl16, 2 species, %d FCC/BCC configs)" % nconf,
        "value": nconf * steps / wall, "unit": "configs/s", "steps": steps,
        "ms_per_step": 1e3 * wall / steps,
        "config": {"workload": "linear fit, level-16 MTP, 2 species, R=8, cutoff 5.0, %d FCC/BCC "
                               "configs of 64-256 atoms, weights 1/0.01/0.001" % nconf,
                   "atoms": n, "neighbor_entries": P, "rows": rows, "p": int(G.shape[0])},
        "roofline": {"bound": "mfma", "achieved": flops / (dev_ms * 1e-3) / 1e12,
                     "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": flops / (dev_ms * 1e-3) / 1e12 / FP64_PEAK_TFLOPS, "traffic": None,
                     "kernel": "lin_site_kernel + gram_kernel (MFMA)", "device_ms": dev_ms,
                     "components_ms": float(np.mean(tims[:, 1])),
                     "gram_ms": float(np.mean(tims[:, 2])),
                     "algorithmic_flops_per_step": flops},
        "list_build_ms": build_ms,
    }, (start_text, structs, off, tE, tF, tS)


def linear_cpu_baseline(data, budget_s: float = 12.0):
    """The oracle's CalcEFSCmpt_R + AddLinearFast + Gram on the host cores,
    on the first structures of the same batch (bounded sample)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    text, structs, off, tE, tF, tS = data
    threads = max(1, min(16, os.cpu_count() or 1))
    m = O.Model(text)
    sample = min(32, len(structs))
    nbs, labels = [], []
    for k in range(sample):
        st = structs[k]
        nbs.append(O.Neighbors.build(st.cell, st.pbc, st.pos, st.types, 5.0))
        labels.append(O.Labels(st.n, energy=tE[k], forces=tF[off[k]:off[k + 1]], stress=tS[k]))
    sets = O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=0.001)
    O.linear_system_batch(m, nbs, labels, sets, threads)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        O.linear_system_batch(m, nbs, labels, sets, threads)
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= 1000:
            break
    return {"value": reps * len(nbs) / el, "unit": "configs/s", "cores": threads, "kind": "port",
            "sample": "%d assemblies over the first %d structures of the batch (oracle "
                      "CalcEFSCmpt_R + AddLinearFast + Gram, %d OpenMP threads, %.1f s)"
                      % (reps, len(nbs), threads, el)}


def train_cpu_baseline(data, budget_s: float = 12.0):
    """The oracle's AccumulateGard restatement on the host cores, on the
    first structures of the same batch (bounded sample)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    text, structs, off, tE, tF, tS, cutoff = data
    threads = max(1, min(16, os.cpu_count() or 1))
    m = O.Model(text)
    sample = min(16, len(structs))
    nbs, labels = [], []
    for k in range(sample):
        st = structs[k]
        nbs.append(O.Neighbors.build(st.cell, st.pbc, st.pos, st.types, cutoff))
        labels.append(O.Labels(st.n, energy=tE[k], forces=tF[off[k]:off[k + 1]], stress=tS[k]))
    st = O.LossSettings.make()
    O.loss_grad_batch(m, nbs, labels, st, 1e-6, 1e-10, 0.0, threads)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        O.loss_grad_batch(m, nbs, labels, st, 1e-6, 1e-10, 0.0, threads)
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= 1000:
            break
    return {"value": reps * len(nbs) / el, "unit": "configs/s", "cores": threads, "kind": "port",
            "sample": "%d loss+gradient passes over the first %d structures of the batch "
                      "(oracle AccumulateGard, %d OpenMP threads, %.1f s)"
                      % (reps, len(nbs), threads, el)}


def cpu_baseline(model_text, cell, pbc, pos, types, budget_s: float = 12.0):
    """The oracle's getEFSOMP restatement timed on the host cores (bounded sample)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    threads = max(1, min(16, os.cpu_count() or 1))
    m = O.Model(model_text)
    nb = O.Neighbors.build(cell, pbc, pos, types, m.cutoff)
    O.efs(m, nb, threads=threads)  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        O.efs(m, nb, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= 2000:
            break
    return {"value": reps * nb.n / el, "unit": "atom-evals/s", "cores": threads, "kind": "port",
            "sample": "%d full E/F/S evaluations of the 32,000-atom cell (oracle getEFSOMP, "
                      "prebuilt lists, %d OpenMP threads, %.1f s)" % (reps, threads, el)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--deterministic", action="store_true")
    ap.add_argument("--no-train", action="store_true")
    ap.add_argument("--train-steps", type=int, default=5)
    ap.add_argument("--train-configs", type=int, default=1000)
    ap.add_argument("--no-linear", action="store_true")
    ap.add_argument("--linear-steps", type=int, default=3)
    ap.add_argument("--linear-configs", type=int, default=2000)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only copy a MIB-MiB device buffer 3 times (calibrates the HBM "
                         "byte counters against a plain copy of known size)")
    args = ap.parse_args()
    if args.copy_probe:
        import torch
        nbytes = args.copy_probe << 20
        a = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": nbytes, "copies": 3}))
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)

    model_text, s = S.workload_inference(2)
    pos = capi.wrap(s.cell, s.pbc, s.pos)  # Atoms::wrap, as CalcEFS does before building lists
    ctx = capi.Context(0)
    ctx.load_model_text(model_text)
    cutoff = 5.0

    t0 = time.perf_counter()
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, cutoff)
    nbuild_first = time.perf_counter() - t0
    n, P = ctx.neighbor_count()
    det = bool(args.deterministic)

    for _ in range(args.warmup):
        ctx.efs_device(det)
    kernel_ms = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.efs_device(det)
        kernel_ms.append(ctx.last_timings()[1])
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps

    # "total": neighbour build from host positions + E/F/S (fastfit total_ns_atom)
    tot = []
    for _ in range(3):
        t1 = time.perf_counter()
        ctx.build_neighbors(s.cell, s.pbc, pos, s.types, cutoff)
        ctx.efs_device(det)
        tot.append(time.perf_counter() - t1)
    E, F, St, _ = ctx.efs(det)
    train = None
    if not args.no_train:
        train, tdata = train_bench(ctx, args.train_steps, 1, args.train_configs)
    linear = None
    if not args.no_linear:
        linear, ldata = linear_bench(ctx, args.linear_steps, args.linear_configs)
    ctx.close()

    flops = efs_flops(model_text, n, P)
    k_ms = float(np.mean(kernel_ms))
    achieved = flops / (k_ms * 1e-3) / 1e12
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        traffic = json.load(open(TRAFFIC_FILE)).get("hbm_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": n * args.steps / wall,
        "unit": "atom-evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic (seeded FCC supercell and random-coefficient model)",
        "config": {"workload": "E/F/S, level-16 MTP, 2 species, 32,000-atom FCC 20x20x20 a=3.56, "
                               "cutoff 5.0, 75/25, strain 2%, sigma 0.12",
                   "atoms": n, "neighbor_entries": P, "mean_neighbors": P / n,
                   "deterministic": det},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": FP64_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / FP64_PEAK_TFLOPS, "traffic": traffic,
                     "kernel": "efs_kernel<4,6,8>", "kernel_ms": k_ms,
                     "kernel_ms_min": float(np.min(kernel_ms)),
                     "algorithmic_flops_per_launch": flops,
                     "note": "fp64 VALU-bound; the MI355X fp64 vector and matrix peaks are both "
                             "78.6 TFLOP/s"},
        "extra": {"total_ms_build_plus_efs": 1e3 * float(np.median(tot)),
                  "neighbor_build_first_ms": 1e3 * nbuild_first,
                  "energy": E, "max_abs_force": float(np.abs(F).max())},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(model_text, s.cell, s.pbc, pos, s.types)
    if train is not None:
        if not args.no_cpu:
            train["cpu_baseline"] = train_cpu_baseline(tdata)
        out["train"] = train
    if linear is not None:
        if not args.no_cpu:
            linear["cpu_baseline"] = linear_cpu_baseline(ldata)
        out["linear"] = linear
    print(json.dumps(out))


if __name__ == "__main__":
    main()
