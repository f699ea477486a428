"""ctypes binding of libmtpx.so (include/mtpx.h).

The library is loaded from imr-mlp_amd/lib/libmtpx.so (built in-tree by
imr-mlp_amd/build.py).  There is no fallback: if the HIP library is missing
or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "lib", "libmtpx.so")
HEADER = os.path.join(ROOT, "include", "mtpx.h")

OK = 0
ERRORS = {-1: "MTPX_E_INVALID", -2: "MTPX_E_MODEL", -3: "MTPX_E_NO_MODEL",
          -4: "MTPX_E_NO_TOPOLOGY", -5: "MTPX_E_DEVICE", -6: "MTPX_E_ALLOC",
          -7: "MTPX_E_CAPACITY", -8: "MTPX_E_RANGE", -9: "MTPX_E_SOLVER"}
ERRORS_BY_NAME = {v: k for k, v in ERRORS.items()}

_dp = C.POINTER(C.c_double)
_ip = C.POINTER(C.c_int)
_lib = None


class MtpxError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("%s (%d): %s" % (ERRORS.get(code, "error"), code, msg))
        self.code = code


def declared_symbols() -> list[str]:
    """Entry points declared in include/mtpx.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mtpx_\w+)\s*\(", text, re.M)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libmtpx.so is not built (run imr-mlp_amd/build.py): " + LIB_PATH)
        L = C.CDLL(LIB_PATH)
        L.mtpx_version.restype = C.c_char_p
        L.mtpx_create.argtypes = [C.c_int, C.POINTER(C.c_void_p)]
        L.mtpx_destroy.argtypes = [C.c_void_p]
        L.mtpx_last_error.restype = C.c_char_p
        L.mtpx_last_error.argtypes = [C.c_void_p]
        L.mtpx_load_model_text.argtypes = [C.c_void_p, C.c_char_p]
        L.mtpx_parse_model_text.argtypes = [C.c_char_p, _ip, _dp, C.c_char_p, C.c_int]
        L.mtpx_model_info.argtypes = [C.c_void_p, _ip]
        L.mtpx_model_head.argtypes = [C.c_void_p, _ip]
        L.mtpx_load_model_gpm.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t]
        L.mtpx_save_model_gpm.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t,
                                          C.POINTER(C.c_size_t)]
        L.mtpx_gpm_to_text.argtypes = [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t,
                                       C.POINTER(C.c_size_t), C.c_char_p, C.c_int]
        L.mtpx_gpm_from_text.argtypes = [C.c_char_p, C.c_int, C.c_void_p, C.c_size_t,
                                         C.POINTER(C.c_size_t), C.c_char_p, C.c_int]
        L.mtpx_parse_model_gpm.argtypes = [C.c_char_p, C.c_size_t, _ip, _dp, C.c_char_p, C.c_int]
        L.mtpx_parse_model_head.argtypes = [C.c_char_p, _ip, C.c_char_p, C.c_int]
        L.mtpx_get_coeffs.argtypes = [C.c_void_p, _dp]
        L.mtpx_set_coeffs.argtypes = [C.c_void_p, _dp]
        L.mtpx_wrap.argtypes = [_dp, _ip, C.c_int, _dp]
        L.mtpx_build_neighbors.argtypes = [C.c_void_p, _dp, _ip, C.c_int, _dp, _ip, C.c_double]
        L.mtpx_neighbor_count.argtypes = [C.c_void_p, C.POINTER(C.c_int64), _ip]
        L.mtpx_get_neighbors.argtypes = [C.c_void_p, _ip, _ip, _ip, _dp, _dp, _ip]
        L.mtpx_set_neighbors.argtypes = [C.c_void_p, C.c_int, _ip, _ip, _ip, _dp, _dp, _ip]
        L.mtpx_efs.argtypes = [C.c_void_p, C.c_int, _dp, _dp, _dp, _dp]
        L.mtpx_efs_device.argtypes = [C.c_void_p, C.c_int]
        L.mtpx_energy.argtypes = [C.c_void_p, _dp, _dp]
        L.mtpx_last_timings.argtypes = [C.c_void_p, _dp]
        L.mtpx_set_timings.argtypes = [C.c_void_p, C.c_int]
        L.mtpx_set_structures.argtypes = [C.c_void_p, C.c_int, _ip, _dp, _ip, _dp, _ip,
                                          C.c_double]
        L.mtpx_structure_count.argtypes = [C.c_void_p, _ip]
        L.mtpx_compute_batch.argtypes = [C.c_void_p, C.c_int, _dp, _dp, _dp, _dp]
        L.mtpx_loss_weights.argtypes = [C.POINTER(LossSettings), C.c_int, _ip, _ip, _dp, _dp,
                                        _dp, _ip, _dp, _dp, _dp]
        L.mtpx_set_labels.argtypes = [C.c_void_p, _ip, _dp, _dp, _dp, _dp, _dp, _dp]
        L.mtpx_prepare_loss.argtypes = [C.c_void_p, _dp]
        L.mtpx_accumulate_gradient.argtypes = [C.c_void_p, _dp, _dp, _dp, C.c_int, _dp]
        L.mtpx_penalty.argtypes = [C.c_void_p, C.c_double, C.c_double, C.c_double, _dp, _dp]
        L.mtpx_loss_grad.argtypes = [C.c_void_p, C.c_int, C.c_double, C.c_double, C.c_double,
                                     _dp, _dp, _dp]
        L.mtpx_last_train_timings.argtypes = [C.c_void_p, _dp]
        L.mtpx_efs_components.argtypes = [C.c_void_p, _dp, _dp, _dp]
        L.mtpx_linear_rows.argtypes = [C.c_void_p, C.POINTER(C.c_int64), _dp, _dp]
        L.mtpx_linear_system.argtypes = [C.c_void_p, _dp, _dp]
        L.mtpx_orthogonalize.argtypes = [C.c_void_p]
        L.mtpx_last_linear_timings.argtypes = [C.c_void_p, _dp]
        L.mtpx_set_add_efs.argtypes = [C.c_void_p, C.c_int]
        L.mtpx_set_fix_species_coeffs.argtypes = [C.c_void_p, C.c_int]
        L.mtpx_lbfgs_default_params.argtypes = [C.POINTER(LbfgsParams)]
        L.mtpx_lbfgs_default_params.restype = None
        L.mtpx_train_lbfgs.argtypes = [C.c_void_p, C.POINTER(LbfgsParams), _dp, _dp, C.c_int,
                                       C.c_double, C.c_double, C.c_double, _ip, _dp, _dp,
                                       C.c_int, _ip]
        L.mtpx_lbfgs_minimize.argtypes = [C.POINTER(LbfgsParams), C.c_int, _dp, LBFGS_OBJECTIVE,
                                          C.c_void_p, _ip, _dp, _ip, C.c_char_p, C.c_int]
        L.mtpx_save_model_text.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t,
                                           C.POINTER(C.c_size_t)]
        L.mtpx_format_model_text.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t,
                                             C.POINTER(C.c_size_t), C.c_char_p, C.c_int]
        L.mtpx_efs_noalloc.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.mtpx_compute_sites.argtypes = [C.c_void_p, C.POINTER(SiteRequest)]
        L.mtpx_load_model.argtypes = [C.c_void_p, C.POINTER(ModelView)]
        L.mtpx_format_model_view.argtypes = [C.POINTER(ModelView), C.c_char_p, C.c_size_t,
                                             C.POINTER(C.c_size_t), C.c_char_p, C.c_int]
        L.mtpx_set_species_map.argtypes = [C.c_void_p, C.c_int, _ip]
        _lib = L
    return _lib


# Enum values of a model view: RadialBasis, RadialCutoff, RadialTransform,
# MTPGpuModel and MTPGpuActivation of the reference's GPU runtime
# (runtime/mtp/gpu-direct/mtp_gpu_direct.h:152-213).
RB_KINDS = {"RBChebyshev": 0, "RBChebyCos": 1, "RBChebyshevPoly5": 2,
            "RBChebyshevConfigurable": 3, "RBChebyshevPoly4": 4, "RBPolyB": 5, "RBPolyBCos": 6}
CUTOFFS = {"quadratic": 0, "cosine": 1, "poly5": 2, "normalized_quadratic": 3,
           "cosine_left": 4, "cosine_unscaled": 5, "cosine_squared": 6, "sine_squared": 7,
           "poly3": 8, "poly4": 9, "smoothstep5": 10, "smoothstep7": 11}
SHIFTS = {"linear": 0, "exponential": 1, "exponential_left": 2, "i2": 3, "exponential_tanh": 4}
VIEW_MODELS = {"linear": 0, "mtp_m_q2": 1, "mtp_m_fs": 2, "mtp_m_n1": 3, "mtp_m_n2": 4,
               "mtp_m_li": 5}
VIEW_ACTIVATIONS = {"TANH": 0, "RELU": 1, "SIGMOID": 2, "LINEAR": 3}


class RadialBasisView(C.Structure):
    """mtpx_radial_basis_view (MTPGpuRadialBasisView)."""
    _fields_ = [("radial_basis", C.c_int), ("min_dist", C.c_double), ("max_dist", C.c_double),
                ("scaling", C.c_double), ("cutoff", C.c_int), ("transform", C.c_int),
                ("cutoff_parameter", C.c_double), ("transform_parameter", C.c_double),
                ("one_minus_chebyshev", C.c_int), ("cutoff_r1", C.c_double),
                ("cutoff_r2", C.c_double), ("transform_scale_parameter", C.c_double),
                ("polynomial_matrix", _dp), ("polynomial_normalizations", _dp)]


class ModelView(C.Structure):
    """mtpx_model_view (MTPGpuPotentialView), field for field."""
    _fields_ = [("species_count", C.c_int), ("max_type", C.c_int), ("spmap", _ip),
                ("alpha_moments_count", C.c_int), ("alpha_index_basic_count", C.c_int),
                ("alpha_index_times_count", C.c_int), ("alpha_scalar_moments", C.c_int),
                ("radial_func_count", C.c_int), ("rb_size", C.c_int), ("max_mu", C.c_int),
                ("max_alpha_index_basic", C.c_int), ("min_dist", C.c_double),
                ("max_dist", C.c_double), ("cutoff", C.c_double), ("scaling", C.c_double),
                ("radial_basis", C.c_int),
                ("pair_radial_bases", C.POINTER(RadialBasisView)),
                ("pair_radial_basis_count", C.c_int), ("radial_coeffs", _dp),
                ("radial_coeffs_count", C.c_int), ("species_coeffs", _dp),
                ("moment_coeffs", _dp), ("model", C.c_int), ("descriptor_count", C.c_int),
                ("scalar_gather", C.c_int), ("input_mean", _dp), ("input_inverse_std", _dp),
                ("input_species", _dp), ("descriptor_species_coeffs", _dp),
                ("descriptor_moment_coeffs", _dp), ("model_coeffs", _dp),
                ("model_coeffs_count", C.c_int), ("model_activation", C.c_int),
                ("model_hidden1", C.c_int), ("model_hidden2", C.c_int),
                ("alpha_index_basic", _ip), ("alpha_index_times", _ip),
                ("alpha_moment_mapping", _ip), ("nu_arr_list", _ip)]


def make_view(fields: dict, pair_bases=None):
    """A ModelView from plain values and numpy arrays (kept alive on the
    returned object as `_keep`).  Array fields are converted to contiguous
    int32 / float64; pair_bases is a list of dicts of RadialBasisView
    fields (or None)."""
    keep = []
    v = ModelView()
    for name, ctype in ModelView._fields_:
        if name not in fields or fields[name] is None or name == "pair_radial_bases":
            continue
        val = fields[name]
        if ctype is _ip:
            a = np.ascontiguousarray(val, np.int32)
            keep.append(a)
            setattr(v, name, a.ctypes.data_as(_ip))
        elif ctype is _dp:
            a = np.ascontiguousarray(val, np.float64)
            keep.append(a)
            setattr(v, name, a.ctypes.data_as(_dp))
        else:
            setattr(v, name, val)
    if pair_bases:
        arr = (RadialBasisView * len(pair_bases))()
        for k, b in enumerate(pair_bases):
            for name, val in b.items():
                setattr(arr[k], name, val)
        keep.append(arr)
        v.pair_radial_bases = C.cast(arr, C.POINTER(RadialBasisView))
        v.pair_radial_basis_count = len(pair_bases)
    v._keep = keep
    return v


def format_model_view(view: ModelView) -> str:
    """mtpx_format_model_view: the .mtp text of the model a view describes
    (host only)."""
    n = C.c_size_t()
    err = C.create_string_buffer(512)
    rc = lib().mtpx_format_model_view(C.byref(view), None, 0, C.byref(n), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    buf = C.create_string_buffer(n.value + 1)
    rc = lib().mtpx_format_model_view(C.byref(view), buf, n.value + 1, C.byref(n), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    return buf.value.decode()


class SiteRequest(C.Structure):
    """mtpx_site_request (MTPGpuBatchRequest / MTPGpuComputeRequest)."""
    _fields_ = [("center_count", C.c_int), ("nlocal", C.c_int), ("ntotal", C.c_int),
                ("centers", _ip), ("offsets", _ip), ("neighbors", _ip),
                ("neighbor_index_mask", C.c_int), ("neighbor_vectors", _dp), ("type", _ip),
                ("x", _dp), ("force", _dp), ("total_energy", _dp), ("global_virial", _dp),
                ("site_energy", _dp), ("site_virial", _dp), ("accumulate_force", C.c_int),
                ("reuse_topology", C.c_int), ("deterministic", C.c_int)]


class LbfgsParams(C.Structure):
    """mtpx_lbfgs_params (LBFGSpp::LBFGSParam)."""
    _fields_ = [("m", C.c_int), ("epsilon", C.c_double), ("epsilon_rel", C.c_double),
                ("epsgmax", C.c_double), ("past", C.c_int), ("delta", C.c_double),
                ("max_iterations", C.c_int), ("max_linesearch", C.c_int),
                ("min_step", C.c_double), ("max_step", C.c_double), ("f_dec_coeff", C.c_double),
                ("s_curv_coeff", C.c_double), ("max_step_move", C.c_double),
                ("machine_prec", C.c_double), ("initial_step", C.c_double),
                ("first_initial_step", C.c_double), ("unscale_iterate", C.c_int)]

    @classmethod
    def default(cls, **kw):
        p = cls()
        lib().mtpx_lbfgs_default_params(C.byref(p))
        for k, v in kw.items():
            setattr(p, k, v)
        return p


LBFGS_OBJECTIVE = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_double),
                              C.POINTER(C.c_double), C.c_int, C.POINTER(C.c_double))


def lbfgs_minimize(fg, x0, params=None):
    """mtpx_lbfgs_minimize over a Python objective fg(x) -> (f, grad); fg may
    return a third value, the point to leave in the solver's iterate.
    Returns (status, x, iterations, f, evaluations, message)."""
    p = params if params is not None else LbfgsParams.default()
    x = f64(x0).copy()
    n = x.size

    def cb(_user, xp, gp, nn, fp):
        try:
            xa = np.ctypeslib.as_array(xp, shape=(nn,))
            res = fg(xa.copy())
            f, g = res[0], res[1]
            np.ctypeslib.as_array(gp, shape=(nn,))[:] = g
            if len(res) > 2:
                xa[:] = res[2]
            fp[0] = f
            return 0
        except Exception:  # noqa: BLE001 -- reported to the solver as a status
            return 1

    cfn = LBFGS_OBJECTIVE(cb)
    it = C.c_int()
    ev = C.c_int()
    fx = C.c_double()
    msg = C.create_string_buffer(256)
    rc = lib().mtpx_lbfgs_minimize(C.byref(p), n, _d(x), cfn, None, C.byref(it), C.byref(fx),
                                   C.byref(ev), msg, 256)
    return rc, x, it.value, fx.value, ev.value, msg.value.decode()


class LossSettings(C.Structure):
    """mtpx_loss_settings; defaults are Trainer_MTP's (train_mtp.cpp:2552-2568)."""
    _fields_ = [(k, C.c_double) for k in
                ("weight_energy", "weight_forces", "weight_stress", "energy_pow", "force_pow",
                 "stress_pow", "force_norm_d", "force_norm_f", "force_norm_p")]

    @classmethod
    def make(cls, weight_energy=1.0, weight_forces=0.01, weight_stress=1e-4, energy_pow=1.0,
             force_pow=0.0, stress_pow=1.0, force_norm_d=0.1, force_norm_f=0.0,
             force_norm_p=1.0):
        return cls(weight_energy, weight_forces, weight_stress, energy_pow, force_pow,
                   stress_pow, force_norm_d, force_norm_f, force_norm_p)


def _d(a):
    return None if a is None else a.ctypes.data_as(_dp)


def _i(a):
    return None if a is None else a.ctypes.data_as(_ip)


def f64(a, shape=None):
    a = np.ascontiguousarray(a, dtype=np.float64)
    return a if shape is None else a.reshape(shape)


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def gpm_to_text(data: bytes) -> str:
    """The .mtp text of a GPM bundle's root model (mtpx_gpm_to_text)."""
    n = C.c_size_t()
    err = C.create_string_buffer(512)
    rc = lib().mtpx_gpm_to_text(data, len(data), None, 0, C.byref(n), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    buf = C.create_string_buffer(n.value + 1)
    rc = lib().mtpx_gpm_to_text(data, len(data), buf, n.value + 1, C.byref(n), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    return buf.value.decode()


def gpm_from_text(text: str, zstd_level: int = 0) -> bytes:
    """The GPM bundle of .mtp text (mtpx_gpm_from_text)."""
    n = C.c_size_t()
    err = C.create_string_buffer(512)
    rc = lib().mtpx_gpm_from_text(text.encode(), int(zstd_level), None, 0, C.byref(n), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    buf = C.create_string_buffer(max(n.value, 1))
    rc = lib().mtpx_gpm_from_text(text.encode(), int(zstd_level), buf, n.value, C.byref(n), err,
                                  512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    return buf.raw[:n.value]


def parse_model_gpm(data: bytes):
    """Host-only parse of a GPM bundle: (sizes dict, coefficients)."""
    info = np.zeros(8, np.int32)
    err = C.create_string_buffer(512)
    rc = lib().mtpx_parse_model_gpm(data, len(data), _i(info), None, err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    coef = np.zeros(int(info[7]))
    lib().mtpx_parse_model_gpm(data, len(data), _i(info), _d(coef), err, 512)
    keys = ["Z", "M", "R", "K", "B", "T", "S", "ncoef"]
    return dict(zip(keys, [int(v) for v in info])), coef


def format_model_text(text: str) -> str:
    """PotMTP::Load then PotMTP::Save on the host (mtpx_format_model_text)."""
    n = C.c_size_t()
    err = C.create_string_buffer(512)
    rc = lib().mtpx_format_model_text(text.encode(), None, 0, C.byref(n), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    buf = C.create_string_buffer(n.value + 1)
    rc = lib().mtpx_format_model_text(text.encode(), buf, n.value + 1, C.byref(n), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    return buf.value.decode()


def version() -> str:
    return lib().mtpx_version().decode()


def wrap(cell, pbc, pos) -> np.ndarray:
    """Atoms::wrap on host arrays (returns a wrapped copy)."""
    out = f64(pos, (-1, 3)).copy()
    cell = f64(cell, (9,))
    pbc = i32(pbc)
    rc = lib().mtpx_wrap(_d(cell), _i(pbc), out.shape[0], _d(out))
    if rc != OK:
        raise MtpxError(rc, "mtpx_wrap")
    return out


def loss_weights(settings: LossSettings, atom_offsets, has, target_forces=None, fitness=None,
                 atomic_fitness=None):
    """Per-structure loss weights (host): (active [nconf][3], wE, wF, wS)."""
    off = i32(atom_offsets)
    nconf = len(off) - 1
    N = int(off[-1])
    has = i32(has).reshape(-1)
    active = np.zeros(3 * max(nconf, 1), np.int32)
    wE, wS, wF = np.zeros(max(nconf, 1)), np.zeros(max(nconf, 1)), np.zeros(max(N, 1))
    tf = None if target_forces is None else f64(target_forces, (-1,))
    fit = None if fitness is None else f64(fitness)
    af = None if atomic_fitness is None else f64(atomic_fitness)
    rc = lib().mtpx_loss_weights(C.byref(settings), nconf, _i(off), _i(has), _d(tf), _d(fit),
                                 _d(af), _i(active), _d(wE), _d(wF), _d(wS))
    if rc != OK:
        raise MtpxError(rc, "mtpx_loss_weights")
    return active[:3 * nconf].reshape(nconf, 3), wE[:nconf], wF[:N], wS[:nconf]


def parse_model_text(text: str):
    """Host-only .mtp parse: (sizes dict, coefficients)."""
    info = np.zeros(8, np.int32)
    err = C.create_string_buffer(512)
    rc = lib().mtpx_parse_model_text(text.encode(), _i(info), None, err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    coef = np.zeros(int(info[7]))
    lib().mtpx_parse_model_text(text.encode(), _i(info), _d(coef), err, 512)
    keys = ["Z", "M", "R", "K", "B", "T", "S", "ncoef"]
    return dict(zip(keys, [int(v) for v in info])), coef


HEADS = ("linear", "mtp_m_li", "mtp_m_q2", "mtp_m_fs", "mtp_m_n1", "mtp_m_n2")
ACTIVATIONS = ("TANH", "RELU", "SIGMOID", "LINEAR")


def _head_dict(v):
    return dict(head=HEADS[v[0]], q=int(v[1]), hidden1=int(v[2]), hidden2=int(v[3]),
                activation=ACTIVATIONS[v[4]], model_coeffs_count=int(v[5]))


def parse_model_head(text: str) -> dict:
    """Host-only: the site-energy head .mtp text declares (mtpx_parse_model_head)."""
    v = np.zeros(6, np.int32)
    err = C.create_string_buffer(512)
    rc = lib().mtpx_parse_model_head(text.encode(), _i(v), err, 512)
    if rc != OK:
        raise MtpxError(rc, err.value.decode())
    return _head_dict(v)


class Context:
    """One mtpx_context on one device."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        rc = lib().mtpx_create(device, C.byref(h))
        if rc != OK:
            raise MtpxError(rc, "mtpx_create(%d)" % device)
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().mtpx_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _check(self, rc, what):
        if rc != OK:
            raise MtpxError(rc, "%s: %s" % (what, lib().mtpx_last_error(self.h).decode()))

    # ---- model ----
    def load_model_text(self, text: str):
        self._check(lib().mtpx_load_model_text(self.h, text.encode()), "load_model_text")
        info = np.zeros(8, np.int32)
        self._check(lib().mtpx_model_info(self.h, _i(info)), "model_info")
        self.info = dict(zip(["Z", "M", "R", "K", "B", "T", "S", "ncoef"], [int(v) for v in info]))
        return self.info

    def load_model_view(self, view: ModelView):
        """mtpx_load_model (MTPGpuDirect::initialize over a view)."""
        self._check(lib().mtpx_load_model(self.h, C.byref(view)), "load_model")
        info = np.zeros(8, np.int32)
        self._check(lib().mtpx_model_info(self.h, _i(info)), "model_info")
        self.info = dict(zip(["Z", "M", "R", "K", "B", "T", "S", "ncoef"], [int(v) for v in info]))
        return self.info

    def set_species_map(self, spmap=None):
        """mtpx_set_species_map: caller types -> species (None: identity)."""
        if spmap is None:
            self._check(lib().mtpx_set_species_map(self.h, 0, None), "set_species_map")
            return
        a = np.ascontiguousarray(spmap, np.int32)
        self._check(lib().mtpx_set_species_map(self.h, a.size, _i(a)), "set_species_map")

    def load_model_gpm(self, data: bytes):
        self._check(lib().mtpx_load_model_gpm(self.h, data, len(data)), "load_model_gpm")
        info = np.zeros(8, np.int32)
        self._check(lib().mtpx_model_info(self.h, _i(info)), "model_info")
        self.info = dict(zip(["Z", "M", "R", "K", "B", "T", "S", "ncoef"], [int(v) for v in info]))
        return self.info

    def save_model_gpm(self, zstd_level: int = 0) -> bytes:
        n = C.c_size_t()
        self._check(lib().mtpx_save_model_gpm(self.h, int(zstd_level), None, 0, C.byref(n)),
                    "save_model_gpm")
        buf = C.create_string_buffer(max(n.value, 1))
        self._check(lib().mtpx_save_model_gpm(self.h, int(zstd_level), buf, n.value, C.byref(n)),
                    "save_model_gpm")
        return buf.raw[:n.value]

    def model_head(self) -> dict:
        """The loaded potential's head (mtpx_model_head)."""
        v = np.zeros(6, np.int32)
        self._check(lib().mtpx_model_head(self.h, _i(v)), "model_head")
        return _head_dict(v)

    def save_model_text(self) -> str:
        n = C.c_size_t()
        self._check(lib().mtpx_save_model_text(self.h, None, 0, C.byref(n)), "save_model_text")
        buf = C.create_string_buffer(n.value + 1)
        self._check(lib().mtpx_save_model_text(self.h, buf, n.value + 1, C.byref(n)),
                    "save_model_text")
        return buf.value.decode()

    def get_coeffs(self) -> np.ndarray:
        x = np.zeros(self.info["ncoef"])
        self._check(lib().mtpx_get_coeffs(self.h, _d(x)), "get_coeffs")
        return x

    def set_coeffs(self, x):
        x = f64(x)
        assert x.size == self.info["ncoef"]
        self._check(lib().mtpx_set_coeffs(self.h, _d(x)), "set_coeffs")

    # ---- neighbours ----
    def build_neighbors(self, cell, pbc, pos, types, cutoff):
        cell = f64(cell, (9,))
        pbc = i32(pbc)
        pos = f64(pos, (-1, 3))
        types = i32(types)
        self._check(lib().mtpx_build_neighbors(self.h, _d(cell), _i(pbc), pos.shape[0], _d(pos),
                                               _i(types), float(cutoff)), "build_neighbors")

    def set_neighbors(self, offsets, idx, types, vec, dist, center_types):
        offsets, idx, types, ct = i32(offsets), i32(idx), i32(types), i32(center_types)
        vec, dist = f64(vec, (-1,)), f64(dist)
        self._check(lib().mtpx_set_neighbors(self.h, len(offsets) - 1, _i(offsets), _i(idx),
                                             _i(types), _d(vec), _d(dist), _i(ct)),
                    "set_neighbors")

    def neighbor_count(self):
        P = C.c_int64()
        n = C.c_int()
        self._check(lib().mtpx_neighbor_count(self.h, C.byref(P), C.byref(n)), "neighbor_count")
        return n.value, P.value

    def get_neighbors(self):
        n, P = self.neighbor_count()
        Pz = max(P, 1)
        offsets = np.zeros(n + 1, np.int32)
        idx = np.zeros(Pz, np.int32)
        types = np.zeros(Pz, np.int32)
        vec = np.zeros((Pz, 3))
        dist = np.zeros(Pz)
        ct = np.zeros(max(n, 1), np.int32)
        self._check(lib().mtpx_get_neighbors(self.h, _i(offsets), _i(idx), _i(types), _d(vec),
                                             _d(dist), _i(ct)), "get_neighbors")
        return dict(offsets=offsets, idx=idx[:P], types=types[:P], vec=vec[:P], dist=dist[:P],
                    center_types=ct[:n])

    # ---- E/F/S ----
    def efs(self, deterministic: bool = False, init=None):
        """getEFS; init = (E, F, S, site energies) start values, which the
        outputs are added onto when add_efs is set."""
        n, _ = self.neighbor_count()
        E = C.c_double()
        F = np.zeros((max(n, 1), 3))
        S = np.zeros((3, 3))
        se = np.zeros(max(n, 1))
        if init is not None:
            E.value = float(init[0])
            F[:n] = init[1]
            S[:] = init[2]
            se[:n] = init[3]
        self._check(lib().mtpx_efs(self.h, int(deterministic), C.byref(E), _d(F), _d(S), _d(se)),
                    "efs")
        return E.value, F[:n], S, se[:n]

    def efs_noalloc(self, forces_ptr: int, site_energies_ptr: int, energy_stress_ptr: int):
        """mtpx_efs_noalloc on caller-owned device buffers (raw addresses)."""
        self._check(lib().mtpx_efs_noalloc(self.h, C.c_void_p(forces_ptr),
                                           C.c_void_p(site_energies_ptr),
                                           C.c_void_p(energy_stress_ptr)), "efs_noalloc")

    def set_add_efs(self, flag: bool):
        self._check(lib().mtpx_set_add_efs(self.h, int(bool(flag))), "set_add_efs")

    def compute_sites(self, offsets, neighbors, types, x=None, vectors=None, centers=None,
                      nlocal=None, mask=-1, force=None, accumulate=True, reuse=False,
                      deterministic=False, site_virial=True):
        """mtpx_compute_sites over a CSR with ghost atoms.  types [ntotal];
        force (optional start values, [ntotal][3]) is added onto when
        accumulate.  Returns dict(energy, virial6, force, site_energy,
        site_virial)."""
        offsets, neighbors, types = i32(offsets), i32(neighbors), i32(types)
        ntotal = int(types.size)
        nc = len(offsets) - 1
        nlocal = ntotal if nlocal is None else int(nlocal)
        cen = None if centers is None else i32(centers)
        xs = None if x is None else f64(x, (-1,))
        vs = None if vectors is None else f64(vectors, (-1,))
        F = np.zeros((max(ntotal, 1), 3))
        if force is not None:
            F[:ntotal] = force
        E = np.zeros(1)
        V6 = np.zeros(6)
        se = np.zeros(max(nlocal, 1))
        sv = np.zeros((max(ntotal, 1), 6)) if site_virial else None
        r = SiteRequest(nc, nlocal, ntotal, None if cen is None else _i(cen), _i(offsets),
                        _i(neighbors), int(mask), None if vs is None else _d(vs), _i(types),
                        None if xs is None else _d(xs), _d(F), _d(E), _d(V6), _d(se),
                        None if sv is None else _d(sv), int(bool(accumulate)), int(bool(reuse)),
                        int(bool(deterministic)))
        self._check(lib().mtpx_compute_sites(self.h, C.byref(r)), "compute_sites")
        return dict(energy=float(E[0]), virial6=V6, force=F[:ntotal], site_energy=se[:nlocal],
                    site_virial=None if sv is None else sv[:ntotal])

    def energy(self):
        """getE: per-structure energies and site energies."""
        n, _ = self.neighbor_count()
        try:
            nc = self.structure_count()
        except MtpxError:
            nc = 1
        E = np.zeros(max(nc, 1))
        se = np.zeros(max(n, 1))
        self._check(lib().mtpx_energy(self.h, _d(E), _d(se)), "energy")
        return E[:nc], se[:n]

    def efs_device(self, deterministic: bool = False):
        self._check(lib().mtpx_efs_device(self.h, int(deterministic)), "efs_device")

    def last_timings(self):
        t = np.zeros(4)
        self._check(lib().mtpx_last_timings(self.h, _d(t)), "last_timings")
        return t

    def set_timings(self, enabled: bool):
        self._check(lib().mtpx_set_timings(self.h, int(bool(enabled))), "set_timings")

    # ---- training batches ----
    def set_structures(self, structures, cutoff):
        """structures: objects with cell (3x3), pbc (3), pos (n x 3), types (n)."""
        off = np.zeros(len(structures) + 1, np.int32)
        for c, st in enumerate(structures):
            off[c + 1] = off[c] + len(st.types)
        cells = f64(np.array([f64(st.cell, (9,)) for st in structures]).reshape(-1))
        pbc = i32(np.array([i32(st.pbc) for st in structures]).reshape(-1))
        pos = f64(np.concatenate([f64(st.pos, (-1, 3)) for st in structures]) if len(structures)
                  else np.zeros((0, 3)), (-1,))
        types = i32(np.concatenate([i32(st.types) for st in structures]) if len(structures)
                    else np.zeros(0))
        self._check(lib().mtpx_set_structures(self.h, len(structures), _i(off), _d(cells),
                                              _i(pbc), _d(pos), _i(types), float(cutoff)),
                    "set_structures")
        self.atom_offsets = off
        return off

    def structure_count(self):
        n = C.c_int()
        self._check(lib().mtpx_structure_count(self.h, C.byref(n)), "structure_count")
        return n.value

    def compute_batch(self, deterministic: bool = False):
        n, _ = self.neighbor_count()
        nc = self.structure_count()
        E, S = np.zeros(max(nc, 1)), np.zeros((max(nc, 1), 3, 3))
        F, se = np.zeros((max(n, 1), 3)), np.zeros(max(n, 1))
        self._check(lib().mtpx_compute_batch(self.h, int(deterministic), _d(E), _d(F), _d(S),
                                             _d(se)), "compute_batch")
        return E[:nc], F[:n], S[:nc], se[:n]

    def set_labels(self, active, tE=None, wE=None, tF=None, wF=None, tS=None, wS=None):
        conv = lambda a, shape=None: None if a is None else f64(a, shape)
        self._labels = [i32(active).reshape(-1), conv(tE), conv(wE), conv(tF, (-1,)), conv(wF),
                        conv(tS, (-1,)), conv(wS)]
        a = self._labels
        self._check(lib().mtpx_set_labels(self.h, _i(a[0]), _d(a[1]), _d(a[2]), _d(a[3]),
                                          _d(a[4]), _d(a[5]), _d(a[6])), "set_labels")

    def prepare_loss(self):
        m = np.zeros(7)
        self._check(lib().mtpx_prepare_loss(self.h, _d(m)), "prepare_loss")
        return m

    def accumulate_gradient(self, dLdE=None, dLdF=None, dLdS=None, gradient=None):
        g = np.zeros(self.info["ncoef"]) if gradient is None else f64(gradient).copy()
        conv = lambda a: None if a is None else f64(a, (-1,))
        a = [conv(dLdE), conv(dLdF), conv(dLdS)]
        self._check(lib().mtpx_accumulate_gradient(self.h, _d(a[0]), _d(a[1]), _d(a[2]),
                                                   int(gradient is not None), _d(g)),
                    "accumulate_gradient")
        return g

    def penalty(self, weight, reg_l2, reg_l1):
        loss = C.c_double(0.0)
        g = np.zeros(self.info["ncoef"])
        self._check(lib().mtpx_penalty(self.h, weight, reg_l2, reg_l1, C.byref(loss), _d(g)),
                    "penalty")
        return loss.value, g

    def loss_grad(self, penalty_weight=0.0, reg_l2=0.0, reg_l1=0.0, deterministic=False):
        loss = C.c_double()
        g = np.zeros(self.info["ncoef"])
        m = np.zeros(7)
        self._check(lib().mtpx_loss_grad(self.h, int(deterministic), penalty_weight, reg_l2,
                                         reg_l1, C.byref(loss), _d(g), _d(m)), "loss_grad")
        return loss.value, g, m

    def train_lbfgs(self, params=None, scaling=None, x=None, deterministic=True,
                    penalty_weight=0.0, reg_l2=0.0, reg_l1=0.0, history_cap=256,
                    raise_on_error=True):
        """Trainer_MTP::TrainNonLinearLBFGS: returns (iterations, loss,
        objective values of the evaluations, evaluations, final iterate); with
        raise_on_error False, (status, message) come first and a solver
        failure returns what the run reached."""
        p = params if params is not None else LbfgsParams.default()
        sc = None if scaling is None else f64(scaling)
        xv = f64(x).copy() if x is not None else np.zeros(self.info["ncoef"])
        it = C.c_int()
        ev = C.c_int()
        loss = C.c_double()
        hist = np.zeros(history_cap)
        if x is None:
            xv[:] = self.get_coeffs() * (1.0 if sc is None else sc)
        rc = lib().mtpx_train_lbfgs(self.h, C.byref(p), _d(sc), _d(xv), int(bool(deterministic)),
                                    penalty_weight, reg_l2, reg_l1, C.byref(it), C.byref(loss),
                                    _d(hist), history_cap, C.byref(ev))
        out = (it.value, loss.value, hist[:min(ev.value, history_cap)], ev.value, xv)
        if raise_on_error:
            self._check(rc, "train_lbfgs")
            return out
        msg = lib().mtpx_last_error(self.h).decode() if rc != OK else ""
        return (rc, msg) + out

    def last_train_timings(self):
        t = np.zeros(4)
        self._check(lib().mtpx_last_train_timings(self.h, _d(t)), "last_train_timings")
        return t

    # ---- linear fit ----
    def efs_components(self):
        n, _ = self.neighbor_count()
        nc = self.structure_count()
        p = self.info["Z"] + self.info["S"]
        ec = np.zeros((max(nc, 1), p))
        fc = np.zeros((max(n, 1), 3, p))
        sc = np.zeros((max(nc, 1), 9, p))
        self._check(lib().mtpx_efs_components(self.h, _d(ec), _d(fc), _d(sc)), "efs_components")
        return ec[:nc], fc[:n], sc[:nc].reshape(nc, 3, 3, p)

    def set_fix_species_coeffs(self, fix: bool):
        self._check(lib().mtpx_set_fix_species_coeffs(self.h, int(bool(fix))),
                    "set_fix_species_coeffs")
        self.fix_species = bool(fix)

    def _row_width(self):
        return self.info["S"] + (0 if getattr(self, "fix_species", False) else self.info["Z"])

    def linear_rows(self):
        R = C.c_int64(0)
        self._check(lib().mtpx_linear_rows(self.h, C.byref(R), None, None), "linear_rows")
        p = self._row_width()
        A = np.zeros((max(R.value, 1), p))
        y = np.zeros(max(R.value, 1))
        self._check(lib().mtpx_linear_rows(self.h, C.byref(R), _d(A), _d(y)), "linear_rows")
        return A[:R.value], y[:R.value]

    def linear_system(self):
        p = self._row_width()
        G = np.zeros((p, p))
        b = np.zeros(p)
        self._check(lib().mtpx_linear_system(self.h, _d(G), _d(b)), "linear_system")
        return G, b

    def orthogonalize(self):
        self._check(lib().mtpx_orthogonalize(self.h), "orthogonalize")

    def last_linear_timings(self):
        t = np.zeros(4)
        self._check(lib().mtpx_last_linear_timings(self.h, _d(t)), "last_linear_timings")
        return t
