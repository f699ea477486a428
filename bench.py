"""Benchmark of the MI355X MTP E/F/S path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-train]
                    [--no-linear] [--no-large]

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
the library's stream.  Further legs (same JSON line): the 256,000-atom
level-20 four-species cell ("large"), the nonlinear training loss+gradient
("train") and the linear-fit assembly ("linear").

The CPU baselines time the oracle's restatement of the reference CPU path
(getEFSOMP, AccumulateGard, CalcEFSCmpt_R + AddLinearFast + Gram) built
with the reference's release flags (-O3 -march=native -fopenmp) on the host
that runs the benchmark, on the cores allotted to the job (OMP_NUM_THREADS)
and on one core; medians of timed rounds with their interquartile range.
Prints one JSON line.
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


def traffic_of(*keys: str):
    """HBM bytes of one launch of a kernel (or, for several keys, of one step
    that launches each of those kernels as often as its summary's
    dispatches_per_step says), from the calibrated FETCH_SIZE / WRITE_SIZE
    summaries under profiles/ (None if one is absent)."""
    total = 0.0
    for key in keys:
        path = os.path.join(ROOT, "profiles", key + "_traffic.json")
        if not os.path.exists(path):
            return None
        js = json.load(open(path))
        total += js["hbm_bytes_per_launch"] * (js.get("dispatches_per_step", 1) if len(keys) > 1
                                               else 1)
    return total


def compute_roofline(flops: float, ms: float, kernel: str, traffic_keys, pipe="fp64 VALU",
                     **extra):
    """Roofline of an fp64 compute-bound kernel (or step): algorithmic flops
    per launch over its mean duration against the MI355X fp64 peak
    (78.6 TFLOP/s for the vector and the matrix pipe alike; `bound` names the
    pipe whose roof applies), and its HBM bytes over the same duration
    against the 8 TB/s HBM peak."""
    achieved = flops / (ms * 1e-3) / 1e12
    keys = (traffic_keys,) if isinstance(traffic_keys, str) else tuple(traffic_keys)
    traffic = traffic_of(*keys)
    hbm = None if traffic is None else traffic / (ms * 1e-3) / 1e9
    r = {"bound": "mfma" if pipe == "fp64 MFMA" else "fp64 VALU", "achieved": achieved,
         "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": achieved / FP64_PEAK_TFLOPS,
         "traffic": traffic, "hbm_gbs": hbm, "hbm_peak_gbs": HBM_PEAK_GBS,
         "hbm_frac": None if hbm is None else hbm / HBM_PEAK_GBS,
         "kernel": kernel, "pipe": pipe, "kernel_ms": ms, "algorithmic_flops_per_launch": flops,
         "traffic_keys": list(keys)}
    r.update(extra)
    return r


def copy_probe(mib: int):
    """A plain device-to-device copy of MIB MiB, three times (calibrates the
    HBM byte counters against traffic of known size); HIP runtime only."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
    hip.hipFree.argtypes = [C.c_void_p]
    nbytes = mib << 20
    a, b = C.c_void_p(), C.c_void_p()
    assert hip.hipMalloc(C.byref(a), nbytes) == 0 and hip.hipMalloc(C.byref(b), nbytes) == 0
    assert hip.hipMemset(a, 1, nbytes) == 0
    for _ in range(3):
        assert hip.hipMemcpy(b, a, nbytes, 3) == 0  # device to device
    assert hip.hipDeviceSynchronize() == 0
    hip.hipFree(a)
    hip.hipFree(b)
    print(json.dumps({"copy_probe_bytes": nbytes, "copies": 3}))


def pmc_summary(dirs, delete_raw: bool):
    """Per-kernel means of rocprofv3 csv output (counter collection and
    kernel statistics) under each directory, as one JSON object keyed by the
    directory name; with delete_raw the per-dispatch csv files are removed."""
    import csv
    import glob
    import re
    from collections import defaultdict

    def short(name):
        name = name.replace("(anonymous namespace)::", "").replace("mtpx::", "")
        return re.sub(r"\(.*", "", name)[:160]

    out = {}
    for d in dirs:
        res = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            acc = defaultdict(lambda: defaultdict(float))
            disp = defaultdict(set)
            with open(f) as fh:
                for row in csv.DictReader(fh):
                    k = short(row["Kernel_Name"])
                    acc[k][row["Counter_Name"]] += float(row["Counter_Value"])
                    disp[k].add(row["Dispatch_Id"])
            for k in acc:
                n = len(disp[k])
                res[k] = {"dispatches": n, **{c: v / n for c, v in acc[k].items()}}
            if delete_raw:
                os.remove(f)
        for f in glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True):
            with open(f) as fh:
                res["_stats"] = [{"name": short(r["Name"]), "calls": int(r["Calls"]),
                                  "avg_us": float(r["AverageNs"]) / 1e3,
                                  "min_us": float(r["MinNs"]) / 1e3,
                                  "max_us": float(r["MaxNs"]) / 1e3,
                                  "percent": float(r["Percentage"])}
                                 for r in csv.DictReader(fh)][:40]
        if delete_raw:
            for f in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
                os.remove(f)
        out[os.path.basename(d.rstrip("/"))] = res
    print(json.dumps(out, indent=1))


def large_bench(ctx, steps: int, warmup: int):
    """The 256,000-atom level-20 four-species cell (40x40x40 FCC, a = 3.6 A,
    equiatomic, sigma 0.15 A, radial basis 10, cutoff 5.5 A): E/F/S with the
    lists resident, and list build + E/F/S from host positions."""
    model_text, s = S.workload_inference(3)
    pos = capi.wrap(s.cell, s.pbc, s.pos)
    ctx.load_model_text(model_text)
    cutoff = 5.5
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, cutoff)
    n, P = ctx.neighbor_count()
    for _ in range(warmup):
        ctx.efs_device(False)
    kms = []
    t0 = time.perf_counter()
    for _ in range(steps):
        ctx.efs_device(False)
        kms.append(ctx.last_timings()[1])
    wall = time.perf_counter() - t0
    tot = []
    for _ in range(3):
        t1 = time.perf_counter()
        ctx.build_neighbors(s.cell, s.pbc, pos, s.types, cutoff)
        ctx.efs_device(False)
        tot.append(time.perf_counter() - t1)
    flops = efs_flops(model_text, n, P)
    k_ms = float(np.mean(kms))
    return {
        "metric": "MTP E/F/S atom-evals/s (lvl20, 4 species, 256k atoms)",
        "value": n * steps / wall, "unit": "atom-evals/s", "steps": steps,
        "ms_per_step": 1e3 * wall / steps,
        "config": {"workload": "E/F/S, level-20 MTP, 4 species, R=10, cutoff 5.5, 256,000-atom "
                               "FCC 40x40x40 a=3.6, equiatomic, sigma 0.15",
                   "atoms": n, "neighbor_entries": P, "mean_neighbors": P / n},
        "roofline": compute_roofline(flops, k_ms, "efs_kernel<level 20>", "efs_lvl20_256k"),
        "total_ms_build_plus_efs": 1e3 * float(np.median(tot)),
    }, (model_text, s.cell, s.pbc, pos, s.types)


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
        "roofline": compute_roofline(
            flops, dev_ms, "loss+grad step (efs_kernel, loss_kernel, grad_kernel)",
            ("efs_lvl20_1000", "grad_lvl20_1000"), efs_ms=float(np.mean(tims[:, 1])),
            loss_ms=float(np.mean(tims[:, 2])), grad_ms=grad_ms,
            traffic_scope="one step: the E/F/S and gradient kernels (loss and reductions "
                          "move under 0.1 % of it)"),
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
        "roofline": compute_roofline(
            flops, dev_ms, "linear-fit step (lin_jac_kernel, lin_tile_kernel, gram_kernel)",
            ("lin_jac_lvl16_2000", "lin_tile_lvl16_2000", "gram_lvl16_2000"),
            pipe="fp64 VALU (design rows) + fp64 MFMA (Gram)",
            components_ms=float(np.mean(tims[:, 1])), gram_ms=float(np.mean(tims[:, 2])),
            traffic_scope="one step: every kernel of the assembly"),
        "list_build_ms": build_ms,
    }, (start_text, structs, off, tE, tF, tS)


# ------------------------------------------------------------ CPU baselines --

_ORACLE = None


def oracle_module():
    """The oracle's timing build (make -C oracle fast: -O3 -march=native
    -fopenmp, compiled here, on the host that runs the baseline); the parity
    build if that compile fails."""
    global _ORACLE
    if _ORACLE is None:
        import subprocess
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        fast = os.path.join(ROOT, "oracle", "_fast", "liboracle_fast.so")
        r = subprocess.run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle"), "fast"],
                           capture_output=True, text=True)
        if r.returncode == 0 and os.path.exists(fast):
            O.use_library(fast)
            O.BUILD_FLAGS = "-O3 -march=native -fopenmp (oracle/Makefile fast)"
        else:
            O.BUILD_FLAGS = "-O2 -ffp-contract=off -fopenmp (parity build; fast build failed)"
        _ORACLE = O
    return _ORACLE


def host_info():
    """Host of the CPU baseline: the CPU model as lscpu names it (else
    /proc/cpuinfo's model name), core counts, OMP_NUM_THREADS."""
    import subprocess
    model = "unknown"
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10)
        for line in r.stdout.splitlines():
            if line.strip().startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if model == "unknown":
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"nproc": os.cpu_count(), "affinity_cpus": affinity, "cpu_model": model,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def job_threads() -> int:
    """The cores allotted to this job: OMP_NUM_THREADS where the scheduler
    sets it (16 per GPU on the MI355X pool), else the affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return host_info()["affinity_cpus"] or 1


def timed(fn, budget_s: float, min_reps: int = 5, max_reps: int = 1000, warmup: int = 1):
    """Median and interquartile range of per-round wall times (warm-up
    rounds first; at least min_reps rounds, then until the budget is used)."""
    for _ in range(warmup):
        fn()
    t = []
    t0 = time.perf_counter()
    while len(t) < max_reps and (len(t) < min_reps or time.perf_counter() - t0 < budget_s):
        t1 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t1)
    q1, med, q3 = np.percentile(t, [25, 50, 75])
    return float(med), float(q3 - q1), len(t)


def _leg(units: float, unit: str, med: float, iqr: float, reps: int, cores: int, what: str):
    return {"value": units / med, "unit": unit, "cores": cores, "kind": "port",
            "median_s": med, "iqr_s": iqr, "rounds": reps,
            "sample": "%s; median of %d rounds (IQR %.3g s), %d thread%s"
                      % (what, reps, iqr, cores, "" if cores == 1 else "s")}


def efs_cpu_baseline(model_text, cell, pbc, pos, types, label: str, budget_s: float = 6.0,
                     single: bool = True, total: bool = True):
    """The oracle's getEFSOMP (atom-parallel, per-thread buffers, serial
    merge; potential_mtp.cpp:2416-2486) on the job's cores and on one core,
    lists prebuilt ("kernel"); plus list build + E/F/S ("total", the BOXED
    build is serial in the reference)."""
    O = oracle_module()
    t = job_threads()
    m = O.Model(model_text)
    nb = O.Neighbors.build(cell, pbc, pos, types, m.cutoff)
    n = nb.n
    med, iqr, reps = timed(lambda: O.efs(m, nb, threads=t), budget_s, min_reps=3)
    out = _leg(n, "atom-evals/s", med, iqr, reps, t, "E/F/S of the %s, prebuilt lists" % label)
    if single:
        med1, iqr1, reps1 = timed(lambda: O.efs(m, nb, threads=1), budget_s, min_reps=3)
        out["single_core"] = _leg(n, "atom-evals/s", med1, iqr1, reps1, 1,
                                  "E/F/S of the %s, prebuilt lists" % label)
    if total:
        def build_and_efs():
            b = O.Neighbors.build(cell, pbc, pos, types, m.cutoff)
            O.efs(m, b, threads=t)
        medt, iqrt, repst = timed(build_and_efs, budget_s / 2, min_reps=3)
        out["total"] = _leg(n, "atom-evals/s", medt, iqrt, repst, t,
                            "BOXED list build (serial) + E/F/S of the %s" % label)
    out["host"] = host_info()
    out["build"] = O.BUILD_FLAGS
    return out


def train_cpu_baseline(data, budget_s: float = 6.0):
    """The oracle's AccumulateGard (per-thread loss/gradient accumulators
    merged in thread order) on the job's cores and on one core."""
    O = oracle_module()
    text, structs, off, tE, tF, tS, cutoff = data
    t = job_threads()
    m = O.Model(text)

    def sample(k):
        nbs, labels = [], []
        for c in range(min(k, len(structs))):
            st = structs[c]
            nbs.append(O.Neighbors.build(st.cell, st.pbc, st.pos, st.types, cutoff))
            labels.append(O.Labels(st.n, energy=tE[c], forces=tF[off[c]:off[c + 1]],
                                   stress=tS[c]))
        return nbs, labels

    st = O.LossSettings.make()
    nbs, labels = sample(250)
    med, iqr, reps = timed(lambda: O.loss_grad_batch(m, nbs, labels, st, 1e-6, 1e-10, 0.0, t),
                           budget_s, min_reps=3)
    out = _leg(len(nbs), "configs/s", med, iqr, reps, t,
               "loss+gradient pass over the first %d structures of the batch" % len(nbs))
    nb1, lb1 = nbs[:24], labels[:24]
    med1, iqr1, reps1 = timed(lambda: O.loss_grad_batch(m, nb1, lb1, st, 1e-6, 1e-10, 0.0, 1),
                              budget_s, min_reps=3)
    out["single_core"] = _leg(len(nb1), "configs/s", med1, iqr1, reps1, 1,
                              "loss+gradient pass over the first %d structures" % len(nb1))
    out["host"] = host_info()
    out["build"] = O.BUILD_FLAGS
    return out


def linear_cpu_baseline(data, budget_s: float = 6.0):
    """The oracle's CalcEFSCmpt_R + AddLinearFast + Gram (per-thread normal
    equations merged in thread order) on the job's cores and on one core."""
    O = oracle_module()
    text, structs, off, tE, tF, tS = data
    t = job_threads()
    m = O.Model(text)
    nbs, labels = [], []
    for c in range(min(1000, len(structs))):
        st = structs[c]
        nbs.append(O.Neighbors.build(st.cell, st.pbc, st.pos, st.types, 5.0))
        labels.append(O.Labels(st.n, energy=tE[c], forces=tF[off[c]:off[c + 1]], stress=tS[c]))
    sets = O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=0.001)
    med, iqr, reps = timed(lambda: O.linear_system_batch(m, nbs, labels, sets, t), budget_s,
                           min_reps=3)
    out = _leg(len(nbs), "configs/s", med, iqr, reps, t,
               "normal-equation assembly over the first %d structures of the batch" % len(nbs))
    nb1, lb1 = nbs[:64], labels[:64]
    med1, iqr1, reps1 = timed(lambda: O.linear_system_batch(m, nb1, lb1, sets, 1), budget_s,
                              min_reps=3)
    out["single_core"] = _leg(len(nb1), "configs/s", med1, iqr1, reps1, 1,
                              "normal-equation assembly over the first %d structures" % len(nb1))
    out["host"] = host_info()
    out["build"] = O.BUILD_FLAGS
    return out


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
    ap.add_argument("--no-large", action="store_true")
    ap.add_argument("--large-steps", type=int, default=20)
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="only print per-kernel means of rocprofv3 csv output in DIR...")
    ap.add_argument("--delete-raw", action="store_true",
                    help="with --pmc-summary: remove the per-dispatch csv files")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary, args.delete_raw)
        return
    if args.copy_probe:
        copy_probe(args.copy_probe)
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

    # the timed calls record no HIP events (mtpx_set_timings); the kernel's
    # own duration comes from an untimed pass of the same calls with them
    ctx.set_timings(False)
    for _ in range(args.warmup):
        ctx.efs_device(det)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ctx.efs_device(det)
    wall = time.perf_counter() - t0
    ms_per_step = 1e3 * wall / args.steps
    ctx.set_timings(True)
    kernel_ms = []
    for _ in range(args.steps):
        ctx.efs_device(det)
        kernel_ms.append(ctx.last_timings()[1])

    # "total": neighbour build from host positions + E/F/S (fastfit total_ns_atom)
    ctx.set_timings(False)
    tot = []
    for _ in range(20):
        t1 = time.perf_counter()
        ctx.build_neighbors(s.cell, s.pbc, pos, s.types, cutoff)
        ctx.efs_device(det)
        tot.append(time.perf_counter() - t1)
    ctx.set_timings(True)
    E, F, St, _ = ctx.efs(det)
    large = None
    if not args.no_large:
        large, large_data = large_bench(ctx, args.large_steps, 3)
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
        "roofline": compute_roofline(flops, k_ms, "efs_kernel<level 16>", "efs_lvl16_32k",
                                     kernel_ms_min=float(np.min(kernel_ms))),
        "extra": {"total_ms_build_plus_efs": 1e3 * float(np.median(tot)),
                  "neighbor_build_first_ms": 1e3 * nbuild_first,
                  "energy": E, "max_abs_force": float(np.abs(F).max())},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = efs_cpu_baseline(model_text, s.cell, s.pbc, pos, s.types,
                                               "32,000-atom level-16 cell")
    if large is not None:
        if not args.no_cpu:
            large["cpu_baseline"] = efs_cpu_baseline(*large_data, "256,000-atom level-20 cell",
                                                     single=False, total=False)
        out["large"] = large
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
