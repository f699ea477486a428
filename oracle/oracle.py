"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, where it is the checker or the timed CPU
baseline -- never the thing measured or shipped.  Each wrapper names the
reference function the C code restates (see mtp_oracle.c for file:line).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

_dp = C.POINTER(C.c_double)
_ip = C.POINTER(C.c_int)
_lib = None


def build(force: bool = False) -> None:
    """Compile liboracle.so (and the reference binaries when the IMR-MLP
    sources are present) with oracle/Makefile."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-C", HERE, "-B" if force else "-s", "liboracle.so"], check=True)


def use_library(path: str) -> None:
    """Load the oracle from another build of the same source (the timing
    build of the CPU baseline, `make -C oracle fast`); call before any other
    oracle function."""
    global LIB_PATH, _lib
    if _lib is not None and LIB_PATH != path:
        raise RuntimeError("oracle library already loaded from " + LIB_PATH)
    LIB_PATH = path


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.orc_model_load_text.restype = C.c_void_p
        L.orc_model_load_text.argtypes = [C.c_char_p, C.c_char_p, C.c_int]
        L.orc_model_free.argtypes = [C.c_void_p]
        L.orc_model_info.argtypes = [C.c_void_p, _ip]
        L.orc_model_head.argtypes = [C.c_void_p, _ip]
        L.orc_model_get_coeffs.argtypes = [C.c_void_p, _dp]
        L.orc_model_set_coeffs.argtypes = [C.c_void_p, _dp]
        L.orc_model_tables.argtypes = [C.c_void_p, _ip, _ip, _ip, _dp]
        L.orc_model_save_text.restype = C.c_int
        L.orc_model_save_text.argtypes = [C.c_void_p, C.c_char_p, C.c_int]
        L.orc_orthogonalize.argtypes = [C.c_void_p]
        L.orc_rb_calc_der.argtypes = [C.c_void_p, C.c_double, _dp, _dp]
        L.orc_rb_calc_der_pair.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_double, _dp, _dp]
        L.orc_wrap.argtypes = [_dp, _ip, C.c_int, _dp]
        L.orc_cell_inverse.argtypes = [_dp, _dp]
        L.orc_build_neighbors.restype = C.c_void_p
        L.orc_build_neighbors.argtypes = [_dp, _ip, C.c_int, _dp, _ip, C.c_double, C.c_char_p,
                                          C.c_int]
        L.orc_nbh_from_csr.restype = C.c_void_p
        L.orc_nbh_from_csr.argtypes = [C.c_int, _ip, _ip, _ip, _dp, _dp, _ip]
        L.orc_nbh_free.argtypes = [C.c_void_p]
        L.orc_nbh_size.restype = C.c_int64
        L.orc_nbh_size.argtypes = [C.c_void_p, _ip, _ip, _ip]
        L.orc_nbh_export.argtypes = [C.c_void_p, _ip, _ip, _ip, _dp, _dp, _ip, _ip]
        L.orc_nbh_export_points.argtypes = [C.c_void_p, _dp, _ip]
        L.orc_site_efs.argtypes = [C.c_void_p, C.c_void_p, C.c_int, _dp, _dp]
        L.orc_efs.argtypes = [C.c_void_p, C.c_void_p, _dp, _dp, _dp, _dp]
        L.orc_efs_omp.argtypes = [C.c_void_p, C.c_void_p, C.c_int, _dp, _dp, _dp, _dp]
        L.orc_energy.argtypes = [C.c_void_p, C.c_void_p, _dp, _dp]
        L.orc_site_moments.argtypes = [C.c_void_p, C.c_void_p, C.c_int, _dp]
        L.orc_accumulate_fp_grad.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_double, _dp,
                                             _dp]
        L.orc_accumulate_efs_combination_grad.argtypes = [C.c_void_p, C.c_void_p, C.c_double,
                                                          _dp, _dp, _dp]
        L.orc_add_loss_grad.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, _dp,
                                        _dp, _dp]
        L.orc_add_penalty_grad.argtypes = [C.c_void_p, C.c_double, C.c_double, C.c_double, _dp,
                                           _dp]
        L.orc_loss_grad_batch.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_void_p), C.c_void_p,
                                          C.c_void_p, C.c_double, C.c_double, C.c_double,
                                          C.c_int, _dp, _dp]
        L.orc_efs_components.argtypes = [C.c_void_p, C.c_void_p, _dp, _dp, _dp]
        L.orc_linear_rows.restype = C.c_int64
        L.orc_linear_rows.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, _dp, _dp]
        L.orc_linear_rows_ex.restype = C.c_int64
        L.orc_linear_rows_ex.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                         _dp, _dp]
        L.orc_linear_system_batch_ex.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_void_p),
                                                 C.c_void_p, C.c_void_p, C.c_int, C.c_int, _dp,
                                                 _dp]
        L.orc_linear_row_count.restype = C.c_int64
        L.orc_linear_row_count.argtypes = [C.c_void_p, C.c_void_p]
        L.orc_gram.argtypes = [C.c_int64, C.c_int, _dp, _dp, _dp, _dp]
        L.orc_linear_system_batch.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_void_p),
                                              C.c_void_p, C.c_void_p, C.c_int, _dp, _dp]
        L.orc_efs_flops.restype = C.c_double
        L.orc_efs_flops.argtypes = [C.c_void_p, C.c_void_p]
        _lib = L
    return _lib


def _d(a):
    return a.ctypes.data_as(_dp)


def _i(a):
    return a.ctypes.data_as(_ip)


def _f64(a, shape=None):
    a = np.ascontiguousarray(a, dtype=np.float64)
    return a if shape is None else a.reshape(shape)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


class LossSettings(C.Structure):
    """Trainer_MTP weights (train/train_mtp.h:206-217 defaults)."""
    _fields_ = [("weight_eng", C.c_double), ("weight_force", C.c_double),
                ("weight_stress", C.c_double), ("eng_pow", C.c_double),
                ("force_pow", C.c_double), ("stress_pow", C.c_double),
                ("force_norm_d", C.c_double), ("force_norm_f", C.c_double),
                ("force_norm_p", C.c_double)]

    @classmethod
    def make(cls, weight_eng=1.0, weight_force=0.01, weight_stress=1e-4, eng_pow=1.0,
             force_pow=0.0, stress_pow=1.0, force_norm_d=0.1, force_norm_f=0.0,
             force_norm_p=1.0):
        return cls(weight_eng, weight_force, weight_stress, eng_pow, force_pow, stress_pow,
                   force_norm_d, force_norm_f, force_norm_p)


class _Config(C.Structure):
    _fields_ = [("n", C.c_int), ("has_energy", C.c_int), ("has_forces", C.c_int),
                ("has_stress", C.c_int), ("energy", C.c_double), ("forces", _dp),
                ("stress", _dp), ("fitness", C.c_double), ("atomic_fitness", _dp)]


@dataclass
class Labels:
    """Training labels of one configuration (Atoms energy_/forces_/stress_)."""
    n: int
    energy: float | None = None
    forces: np.ndarray | None = None
    stress: np.ndarray | None = None
    fitness: float = 1.0
    atomic_fitness: np.ndarray | None = None
    _keep: list = field(default_factory=list, repr=False)

    def cstruct(self):
        f = None if self.forces is None else _f64(self.forces, (-1,))
        s = None if self.stress is None else _f64(self.stress, (-1,))
        af = None if self.atomic_fitness is None else _f64(self.atomic_fitness)
        self._keep = [f, s, af]
        return _Config(self.n, int(self.energy is not None), int(f is not None),
                       int(s is not None), 0.0 if self.energy is None else float(self.energy),
                       _d(f) if f is not None else None, _d(s) if s is not None else None,
                       float(self.fitness), _d(af) if af is not None else None)


class Model:
    """PotMTP restated (potentials/potential_mtp.cpp:119-571 loader)."""

    def __init__(self, text: str):
        err = C.create_string_buffer(512)
        self.h = lib().orc_model_load_text(text.encode(), err, 512)
        if not self.h:
            raise ValueError(err.value.decode())
        info = np.zeros(11, np.int32)
        lib().orc_model_info(self.h, _i(info))
        (self.Z, self.M, self.R, self.K, self.B, self.T, self.S, self.max_nu1, self.max_mu,
         self.nradial, self.ncoef) = [int(v) for v in info]
        hd = np.zeros(6, np.int32)
        lib().orc_model_head(self.h, _i(hd))
        # MTP-M head (runtime/mtp/mlip.cpp:70-296): 0 none, 1 li, 2 q2, 3 fs,
        # 4 nn1, 5 nn2; descriptors P, hidden sizes, activation (0 tanh,
        # 1 relu, 2 sigmoid, 3 linear), head coefficient count
        self.head, self.P, self.h1, self.h2, self.act, self.Mc = [int(v) for v in hd]

    def linear_only(self, what):
        """The training and linear-fit restatements cover the linear MTP only."""
        if self.head:
            raise ValueError("%s: the oracle restates the linear MTP only" % what)

    @classmethod
    def from_file(cls, path):
        with open(path) as f:
            return cls(f.read())

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_model_free(self.h)
            self.h = None

    @property
    def coeffs(self) -> np.ndarray:
        x = np.zeros(self.ncoef)
        lib().orc_model_get_coeffs(self.h, _d(x))
        return x

    @coeffs.setter
    def coeffs(self, x):
        x = _f64(x)
        assert x.size == self.ncoef
        lib().orc_model_set_coeffs(self.h, _d(x))

    def tables(self):
        basic = np.zeros((max(self.B, 1), 4), np.int32)
        times = np.zeros((max(self.T, 1), 4), np.int32)
        mp = np.zeros(max(self.S, 1), np.int32)
        rb = np.zeros(3)
        lib().orc_model_tables(self.h, _i(basic), _i(times), _i(mp), _d(rb))
        return basic[:self.B], times[:self.T], mp[:self.S], rb

    def save_text(self) -> str:
        """PotMTP::Save text (a JSON potential_tag is not restated: ValueError)."""
        n = lib().orc_model_save_text(self.h, None, 0)
        if n < 0:
            raise ValueError("the oracle does not restate JSON potential tags")
        buf = C.create_string_buffer(n + 1)
        lib().orc_model_save_text(self.h, buf, n + 1)
        return buf.value.decode()

    def orthogonalize(self):
        lib().orc_orthogonalize(self.h)

    def rb_calc_der(self, r: float, ti: int | None = None, tj: int | None = None):
        """Radial basis values and derivatives at r: the shared basis, or the
        basis of the ordered species pair (ti, tj)."""
        v = np.zeros(self.R)
        d = np.zeros(self.R)
        if ti is None:
            lib().orc_rb_calc_der(self.h, float(r), _d(v), _d(d))
        else:
            lib().orc_rb_calc_der_pair(self.h, int(ti), int(tj), float(r), _d(v), _d(d))
        return v, d

    @property
    def cutoff(self):
        return float(self.tables()[3][1])


def wrap(cell, pbc, pos) -> np.ndarray:
    """Atoms::wrap (base/structures.cpp:1282-1305)."""
    cell = _f64(cell, (9,))
    pbc = _i32(pbc)
    out = _f64(pos, (-1, 3)).copy()
    lib().orc_wrap(_d(cell), _i(pbc), out.shape[0], _d(out))
    return out


class Neighbors:
    """Neighborhoods (BOXED) restated, CSR form."""

    def __init__(self, handle):
        self.h = handle
        n = C.c_int()
        npts = C.c_int()
        bl = np.zeros(3, np.int32)
        self.P = int(lib().orc_nbh_size(self.h, C.byref(n), C.byref(npts), _i(bl)))
        self.n = n.value
        self.npts = npts.value
        self.boxle = bl
        P = max(self.P, 1)
        self.offsets = np.zeros(self.n + 1, np.int32)
        self.idx = np.zeros(P, np.int32)
        self.types = np.zeros(P, np.int32)
        self.vec = np.zeros((P, 3))
        self.dist = np.zeros(P)
        self.pt = np.zeros(P, np.int32)
        self.center_types = np.zeros(max(self.n, 1), np.int32)
        lib().orc_nbh_export(self.h, _i(self.offsets), _i(self.idx), _i(self.types),
                             _d(self.vec), _d(self.dist), _i(self.pt), _i(self.center_types))
        self.idx, self.types, self.vec = self.idx[:self.P], self.types[:self.P], self.vec[:self.P]
        self.dist, self.pt = self.dist[:self.P], self.pt[:self.P]
        self.center_types = self.center_types[:self.n]

    @classmethod
    def build(cls, cell, pbc, pos, types, cutoff):
        """Neighborhoods(atom, cutoff) (base/neighborhood.cpp:77-146)."""
        cell = _f64(cell, (9,))
        pbc = _i32(pbc)
        pos = _f64(pos, (-1, 3))
        types = _i32(types)
        err = C.create_string_buffer(256)
        h = lib().orc_build_neighbors(_d(cell), _i(pbc), pos.shape[0], _d(pos), _i(types),
                                      float(cutoff), err, 256)
        if not h:
            raise ValueError(err.value.decode())
        return cls(h)

    @classmethod
    def from_csr(cls, offsets, idx, types, vec, dist, center_types):
        offsets, idx, types, ct = _i32(offsets), _i32(idx), _i32(types), _i32(center_types)
        vec, dist = _f64(vec, (-1,)), _f64(dist)
        h = lib().orc_nbh_from_csr(len(offsets) - 1, _i(offsets), _i(idx), _i(types), _d(vec),
                                   _d(dist), _i(ct))
        return cls(h)

    def points(self):
        pts = np.zeros((max(self.npts, 1), 3))
        orig = np.zeros(max(self.npts, 1), np.int32)
        lib().orc_nbh_export_points(self.h, _d(pts), _i(orig))
        return pts[:self.npts], orig[:self.npts]

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_nbh_free(self.h)
            self.h = None


def efs(model: Model, nb: Neighbors, threads: int = 0):
    """getEFS (threads == 0: serial, potential_mtp.cpp:1899-1933) or getEFSOMP
    (threads > 0: :2416-2486).  Returns E, F[n,3], S[3,3], site energies."""
    E = C.c_double()
    F = np.zeros((max(nb.n, 1), 3))
    S = np.zeros((3, 3))
    se = np.zeros(max(nb.n, 1))
    if threads > 0:
        lib().orc_efs_omp(model.h, nb.h, threads, C.byref(E), _d(F), _d(S), _d(se))
    else:
        lib().orc_efs(model.h, nb.h, C.byref(E), _d(F), _d(S), _d(se))
    return E.value, F[:nb.n], S, se[:nb.n]


def energy(model: Model, nb: Neighbors):
    E = C.c_double()
    se = np.zeros(max(nb.n, 1))
    lib().orc_energy(model.h, nb.h, C.byref(E), _d(se))
    return E.value, se[:nb.n]


def site_efs(model: Model, nb: Neighbors, i: int):
    n = int(nb.offsets[i + 1] - nb.offsets[i])
    e = C.c_double()
    d = np.zeros((max(n, 1), 3))
    lib().orc_site_efs(model.h, nb.h, i, C.byref(e), _d(d))
    return e.value, d[:n]


def site_moments(model: Model, nb: Neighbors, i: int):
    m = np.zeros(model.K)
    lib().orc_site_moments(model.h, nb.h, i, _d(m))
    return m


def accumulate_fp_grad(model, nb, i, se_weight, f_weight=None, grad=None):
    model.linear_only("accumulate_fp_grad")
    g = np.zeros(model.ncoef) if grad is None else grad
    fw = None if f_weight is None else _f64(f_weight, (-1,))
    lib().orc_accumulate_fp_grad(model.h, nb.h, i, float(se_weight),
                                 _d(fw) if fw is not None else None, _d(g))
    return g


def accumulate_efs_combination_grad(model, nb, dLdE, dLdF, dLdS, grad=None):
    model.linear_only("accumulate_efs_combination_grad")
    g = np.zeros(model.ncoef) if grad is None else grad
    dLdF = _f64(dLdF, (-1,))
    dLdS = _f64(dLdS, (-1,))
    lib().orc_accumulate_efs_combination_grad(model.h, nb.h, float(dLdE), _d(dLdF), _d(dLdS),
                                              _d(g))
    return g


def add_loss_grad(model, nb, settings: LossSettings, labels: Labels, grad=None):
    """Trainer_MTP::AddLossGard for one configuration.  Returns (loss, grad,
    metrics[loss_e, loss_f, loss_s, sq_e_at, sq_f, sq_s])."""
    model.linear_only("add_loss_grad")
    g = np.zeros(model.ncoef) if grad is None else grad
    loss = C.c_double(0.0)
    met = np.zeros(6)
    cfg = labels.cstruct()
    lib().orc_add_loss_grad(model.h, nb.h, C.byref(settings), C.byref(cfg), C.byref(loss), _d(g),
                            _d(met))
    return loss.value, g, met


def penalty_grad(model, weight=1e-6, reg_l2=1e-10, reg_l1=0.0):
    loss = C.c_double(0.0)
    g = np.zeros(model.ncoef)
    lib().orc_add_penalty_grad(model.h, float(weight), float(reg_l2), float(reg_l1),
                               C.byref(loss), _d(g))
    return loss.value, g


def loss_grad_batch(model, nbs, labels, settings, penalty_weight=1e-6, reg_l2=1e-10,
                    reg_l1=0.0, threads=0):
    """Trainer_MTP::AccumulateGard: f, g over a batch of configurations."""
    model.linear_only("loss_grad_batch")
    arr = (C.c_void_p * len(nbs))(*[nb.h for nb in nbs])
    cfgs = (_Config * len(labels))(*[lb.cstruct() for lb in labels])
    f = C.c_double()
    g = np.zeros(model.ncoef)
    lib().orc_loss_grad_batch(model.h, len(nbs), arr, C.cast(cfgs, C.c_void_p),
                              C.byref(settings), float(penalty_weight), float(reg_l2),
                              float(reg_l1), int(threads), C.byref(f), _d(g))
    return f.value, g


def efs_components(model, nb):
    """CalcEFSCmpt_R (potential_mtp.cpp:2675-2707): energy[p], force[n,3,p],
    stress[3,3,p] with p = species + scalar moments."""
    model.linear_only("efs_components")
    p = model.Z + model.S
    ec = np.zeros(p)
    fc = np.zeros((max(nb.n, 1), 3, p))
    sc = np.zeros((3, 3, p))
    lib().orc_efs_components(model.h, nb.h, _d(ec), _d(fc), _d(sc))
    return ec, fc[:nb.n], sc


def linear_rows(model, nb, settings, labels: Labels, fix_species=False):
    """AddLinearFast rows (train/train_mtp.cpp:1289-1395): F, S, E, scaled by
    sqrt(w); fix_species drops the species columns (fix_species_coeffs)."""
    model.linear_only("linear_rows")
    cfg = labels.cstruct()
    rows = int(lib().orc_linear_row_count(C.byref(settings), C.byref(cfg)))
    p = model.S if fix_species else model.Z + model.S
    A = np.zeros((max(rows, 1), p))
    y = np.zeros(max(rows, 1))
    got = lib().orc_linear_rows_ex(model.h, nb.h, C.byref(settings), C.byref(cfg),
                                   int(bool(fix_species)), _d(A), _d(y))
    assert got == rows
    return A[:rows], y[:rows]


def gram(A, y):
    A = _f64(A)
    y = _f64(y)
    p = A.shape[1]
    G = np.zeros((p, p))
    b = np.zeros(p)
    lib().orc_gram(A.shape[0], p, _d(A), _d(y), _d(G), _d(b))
    return G, b


def linear_system_batch(model, nbs, labels, settings, threads=0, fix_species=False):
    model.linear_only("linear_system_batch")
    arr = (C.c_void_p * len(nbs))(*[nb.h for nb in nbs])
    cfgs = (_Config * len(labels))(*[lb.cstruct() for lb in labels])
    p = model.S if fix_species else model.Z + model.S
    G = np.zeros((p, p))
    b = np.zeros(p)
    lib().orc_linear_system_batch_ex(model.h, len(nbs), arr, C.cast(cfgs, C.c_void_p),
                                     C.byref(settings), int(bool(fix_species)), int(threads),
                                     _d(G), _d(b))
    return G, b


def efs_flops(model, nb) -> float:
    return float(lib().orc_efs_flops(model.h, nb.h))


# ---- reference binaries (oracle/_ref, built from the IMR-MLP sources) ----

def ref_available(name: str) -> bool:
    return os.path.exists(os.path.join(REF_DIR, name))


def ref_neighbors(cell, pbc, pos, types, cutoff, workdir):
    """Run oracle/_ref/nbh_ref (base/neighborhood.cpp).  Returns CSR arrays."""
    pos = _f64(pos, (-1, 3))
    n = pos.shape[0]
    fin = os.path.join(workdir, "nbh_in.bin")
    fout = os.path.join(workdir, "nbh_out.bin")
    with open(fin, "wb") as f:
        f.write(np.int32(n).tobytes())
        f.write(_f64(cell, (9,)).tobytes())
        f.write(_i32(pbc).tobytes())
        f.write(np.float64(cutoff).tobytes())
        f.write(pos.tobytes())
        f.write(_i32(types).tobytes())
    subprocess.run([os.path.join(REF_DIR, "nbh_ref"), fin, fout], check=True)
    raw = open(fout, "rb").read()
    o = 0
    nn = int(np.frombuffer(raw, np.int32, 1, o)[0]); o += 4
    P = int(np.frombuffer(raw, np.int64, 1, o)[0]); o += 8
    offsets = np.frombuffer(raw, np.int32, nn + 1, o); o += 4 * (nn + 1)
    idx = np.frombuffer(raw, np.int32, P, o); o += 4 * P
    typ = np.frombuffer(raw, np.int32, P, o); o += 4 * P
    vec = np.frombuffer(raw, np.float64, 3 * P, o).reshape(P, 3); o += 24 * P
    dist = np.frombuffer(raw, np.float64, P, o); o += 8 * P
    ct = np.frombuffer(raw, np.int32, nn, o)
    return dict(offsets=offsets, idx=idx, types=typ, vec=vec, dist=dist, center_types=ct)


def ref_mlip_efs(model_text, nb: Neighbors, point_types, cutoff, workdir, Z, binary="mlip_ref"):
    """Run oracle/_ref/mlip_ref (runtime/mtp/mlip.cpp) -- or, with binary
    "mtpm_ref", the MTP-M site executor (runtime/mtp/cpu/mtp_cpu.cpp) -- over
    the oracle's periodic images as ghost atoms.  Returns E, site E[n],
    F[n,3], virial6."""
    pts, orig = nb.points()
    if isinstance(model_text, bytes):  # a GPM bundle, read by the same core
        mpath = os.path.join(workdir, "model.gpm")
        with open(mpath, "wb") as f:
            f.write(model_text)
    else:
        mpath = os.path.join(workdir, "model.mtp")
        with open(mpath, "w") as f:
            f.write(model_text)
    fin = os.path.join(workdir, "mlip_in.bin")
    fout = os.path.join(workdir, "mlip_out.bin")
    with open(fin, "wb") as f:
        f.write(np.int32(Z).tobytes())
        f.write(np.int32(len(pts)).tobytes())
        f.write(np.int32(nb.n).tobytes())
        f.write(np.float64(cutoff).tobytes())
        f.write(_f64(pts).tobytes())
        f.write(_i32(np.asarray(point_types)[orig]).tobytes())
        f.write(_i32(orig).tobytes())
    subprocess.run([os.path.join(REF_DIR, binary), mpath, fin, fout], check=True)
    raw = np.frombuffer(open(fout, "rb").read(), np.float64)
    n = nb.n
    return raw[0], raw[1:1 + n], raw[1 + n:1 + 4 * n].reshape(n, 3), raw[1 + 4 * n:7 + 4 * n]


class RefLbfgsParams(C.Structure):
    """The parameter block of oracle/_ref/liblbfgs_ref.so (LBFGSpp::LBFGSParam
    fields of the Lewis-Overton solver)."""
    _fields_ = [("m", C.c_int), ("epsilon", C.c_double), ("epsilon_rel", C.c_double),
                ("epsgmax", C.c_double), ("past", C.c_int), ("delta", C.c_double),
                ("max_iterations", C.c_int), ("max_linesearch", C.c_int),
                ("min_step", C.c_double), ("max_step", C.c_double), ("f_dec_coeff", C.c_double),
                ("s_curv_coeff", C.c_double), ("max_step_move", C.c_double),
                ("machine_prec", C.c_double), ("initial_step", C.c_double),
                ("first_initial_step", C.c_double), ("unscale_iterate", C.c_int)]

    @classmethod
    def default(cls, **kw):
        """LBFGSParam() defaults (deplibs/LBFGSpp/include/LBFGSpp/Param.h:224-243)
        with the trainer's epsgmax = 0 (train/train_mtp.cpp:59)."""
        p = cls(m=6, epsilon=1e-5, epsilon_rel=1e-5, epsgmax=0.0, past=0, delta=0.0,
                max_iterations=0, max_linesearch=20, min_step=1e-20, max_step=1e20,
                f_dec_coeff=1e-4, s_curv_coeff=0.9, max_step_move=1e20, machine_prec=1e-16,
                initial_step=-1.0, first_initial_step=-1.0, unscale_iterate=1)
        for k, v in kw.items():
            setattr(p, k, v)
        return p


_REF_OBJECTIVE = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_double),
                             C.POINTER(C.c_double), C.c_int, C.POINTER(C.c_double))
_ref_lbfgs_lib = None


def ref_lbfgs(fg, x0, params=None):
    """LBFGSSolver<double, LineSearchLewisOverton>::minimize of the reference's
    vendored LBFGSpp (oracle/_ref/liblbfgs_ref.so) over fg(x) -> (f, grad[,
    point to leave in the solver's iterate]).  Returns (ok, x, iterations, f,
    evaluations, message)."""
    global _ref_lbfgs_lib
    if _ref_lbfgs_lib is None:
        L = C.CDLL(os.path.join(REF_DIR, "liblbfgs_ref.so"))
        L.ref_lbfgs_minimize.argtypes = [C.POINTER(RefLbfgsParams), C.c_int,
                                         C.POINTER(C.c_double), _REF_OBJECTIVE, C.c_void_p,
                                         C.POINTER(C.c_int), C.POINTER(C.c_double), C.c_char_p,
                                         C.c_int]
        L.ref_lbfgs_minimize.restype = C.c_int
        _ref_lbfgs_lib = L
    p = params if params is not None else RefLbfgsParams.default()
    x = np.array(x0, dtype=np.float64)
    n = x.size
    count = [0]

    def cb(_user, xp, gp, nn, fp):
        try:
            xa = np.ctypeslib.as_array(xp, shape=(nn,))
            res = fg(xa.copy())
            np.ctypeslib.as_array(gp, shape=(nn,))[:] = res[1]
            if len(res) > 2:
                xa[:] = res[2]
            fp[0] = res[0]
            count[0] += 1
            return 0
        except Exception:  # noqa: BLE001 -- reported to the solver as a failure
            return 1

    cfn = _REF_OBJECTIVE(cb)
    it = C.c_int()
    fx = C.c_double()
    msg = C.create_string_buffer(256)
    rc = _ref_lbfgs_lib.ref_lbfgs_minimize(C.byref(p), n, x.ctypes.data_as(C.POINTER(C.c_double)),
                                           cfn, None, C.byref(it), C.byref(fx), msg, 256)
    return rc == 0, x, it.value, fx.value, count[0], msg.value.decode()
