"""Deterministic synthetic workloads: structures, MTP models and labels.

Everything is drawn from numpy's PCG64 bit generator seeded with
``20261201 + workload_id``.  Uniform doubles are ``Generator.random()``
((next_uint64 >> 11) * 2**-53); Gaussians use Box-Muller on two uniforms:
``sqrt(-2 ln(1 - u1)) * cos(2 pi u2)``.

Structures are returned unwrapped (cell rows are lattice vectors); callers
wrap them with ``Atoms::wrap`` semantics before building neighbour lists, as
the reference's CalcEFS front end does (apps/calc_efs.cpp:360).

Models are written as complete ``.mtp`` text in the ``PotMTP::Save`` layout
(potentials/potential_mtp.cpp:647-785) with an explicit ``scaling``; the
coefficients are plain uniform draws in the order radial (Z*Z*M*R), species
(Z), moments (S).
"""
from __future__ import annotations

import os
import re
from dataclasses import dataclass

import numpy as np

SEED_BASE = 20261201
REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
TEMPLATE_DIR = os.path.join(REPO, "tests", "golden", "templates")


def rng_for(workload_id: int, stream: int = 0) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([SEED_BASE + workload_id, stream]))


def uniform(rng, n, lo=0.0, hi=1.0):
    return lo + (hi - lo) * rng.random(n)


def gaussian(rng, n):
    u1 = rng.random(n)
    u2 = rng.random(n)
    return np.sqrt(-2.0 * np.log(1.0 - u1)) * np.cos(2.0 * np.pi * u2)


@dataclass
class Structure:
    cell: np.ndarray      # [3,3], rows are lattice vectors
    pos: np.ndarray       # [n,3] Cartesian
    types: np.ndarray     # [n] int32 species
    pbc: np.ndarray       # [3] int32

    @property
    def n(self):
        return len(self.types)


FCC_BASIS = np.array([[0, 0, 0], [0, .5, .5], [.5, 0, .5], [.5, .5, 0]])
BCC_BASIS = np.array([[0, 0, 0], [.5, .5, .5]])


def lattice(kind: str, reps, a: float) -> Structure:
    basis = FCC_BASIS if kind == "fcc" else BCC_BASIS
    reps = np.asarray(reps, int)
    grid = np.stack(np.meshgrid(np.arange(reps[0]), np.arange(reps[1]), np.arange(reps[2]),
                                indexing="ij"), -1).reshape(-1, 3)
    frac = (grid[:, None, :] + basis[None, :, :]).reshape(-1, 3) / reps
    cell = np.diag(reps * a).astype(np.float64)
    pos = frac @ cell
    return Structure(cell, pos, np.zeros(len(pos), np.int32), np.ones(3, np.int32))


def assign_species(rng, n: int, counts) -> np.ndarray:
    """Exact species counts, then a Fisher-Yates shuffle."""
    t = np.concatenate([np.full(c, s, np.int32) for s, c in enumerate(counts)])
    assert len(t) == n
    for i in range(n - 1, 0, -1):
        j = int(rng.random() * (i + 1))
        t[i], t[j] = t[j], t[i]
    return t


def fractions_to_counts(n: int, fractions) -> list[int]:
    c = [int(np.floor(f * n)) for f in fractions]
    c[0] += n - sum(c)
    return c


def strain(s: Structure, rng, amp: float) -> Structure:
    """Symmetric strain eps_ab ~ U[-amp, amp]: cell' = cell (I + eps), x' = x (I + eps)."""
    e = uniform(rng, 6, -amp, amp)
    eps = np.array([[e[0], e[3], e[4]], [e[3], e[1], e[5]], [e[4], e[5], e[2]]])
    F = np.eye(3) + eps
    return Structure(s.cell @ F, s.pos @ F, s.types, s.pbc)


def displace(s: Structure, rng, sigma: float) -> Structure:
    d = gaussian(rng, 3 * s.n).reshape(s.n, 3) * sigma
    return Structure(s.cell, s.pos + d, s.types, s.pbc)


def liquid(rng, n: int, density: float, dmin: float, nspecies: int) -> Structure:
    """Random sequential addition in a periodic cube at the given number density."""
    L = (n / density) ** (1.0 / 3.0)
    cell = np.eye(3) * L
    pos = np.zeros((0, 3))
    tries = 0
    while len(pos) < n:
        p = uniform(rng, 3) * L
        tries += 1
        if tries > 2000000:
            raise RuntimeError("random sequential addition did not converge")
        if len(pos):
            d = pos - p
            d -= L * np.round(d / L)
            if np.min(np.einsum("ij,ij->i", d, d)) < dmin * dmin:
                continue
        pos = np.vstack([pos, p])
    types = (uniform(rng, n) * nspecies).astype(np.int32)
    return Structure(cell, pos, types, np.ones(3, np.int32))


# ---------------------------------------------------------------- models --

def read_template(name: str) -> str:
    with open(os.path.join(TEMPLATE_DIR, name)) as f:
        return f.read()


def template_topology(text: str):
    """alpha_* tables of an .mtp text (coefficients are ignored)."""
    def grab(key):
        m = re.search(r"^" + key + r"\s*=\s*\{(.*?)\}\s*$", text, re.M | re.S)
        return m.group(1)

    def ival(key):
        return int(re.search(r"^\s*" + key + r"\s*=\s*(\S+)", text, re.M).group(1))

    basic = np.array([[int(v) for v in g.split(",")]
                      for g in re.findall(r"\{([-\d, ]+)\}", grab("alpha_index_basic"))],
                     np.int32).reshape(-1, 4)
    tgrp = grab("alpha_index_times") if ival("alpha_index_times_count") else ""
    times = np.array([[int(v) for v in g.split(",")] for g in re.findall(r"\{([-\d, ]+)\}", tgrp)],
                     np.int32).reshape(-1, 4)
    mp = np.array([int(v) for v in grab("alpha_moment_mapping").split(",")], np.int32)
    return dict(K=ival("alpha_moments_count"), basic=basic, times=times, map=mp,
                M=ival("radial_funcs_count"))


def fmt(x: float) -> str:
    return "%.17e" % x


BASIS_TYPES = ("RBChebyshev", "RBChebyCos", "RBChebyshevPoly4", "RBChebyshevPoly5",
               "RBChebyshevConfigurable")
CUTOFF_TYPES = ("quadratic", "normalized_quadratic", "cosine", "cosine_left", "cosine_unscaled",
                "cosine_squared", "sine_squared", "poly3", "poly4", "poly5", "smoothstep5",
                "smoothstep7")
SHIFT_TYPES = ("linear", "exponential", "exponential_left", "i2", "exponential_tanh")


def configurable(cutoff="cosine", shift="linear", one_minus=False, cutoff_b=-0.25, r1=None,
                 r2=None, lam=1.5, scale_lambda=0.8):
    """An RBChebyshevConfigurable description for basis_lines / write_mtp."""
    return dict(type="RBChebyshevConfigurable", cutoff=cutoff, shift=shift, one_minus=one_minus,
                cutoff_b=cutoff_b, r1=r1, r2=r2, lam=lam, scale_lambda=scale_lambda)


def basis_lines(kind, rmin: float, rmax: float, R: int, b: float = -1.0 / 3.0):
    """AnyBasis::SaveToStream (basis/basis.h:50-56), plus rb_b for the
    Poly4 / Poly5 bases (basis/basis.cpp:560-564, :733-737); kind may be a
    configurable() description (RBasis_ChebyshevConfigurable::SaveToStream,
    basis.cpp:913-919, with the cutoff and shift lines)."""
    cfg = kind if isinstance(kind, dict) else None
    name = cfg["type"] if cfg else kind
    out = ["radial_basis_type = " + name, "\tmin_dist = " + fmt(rmin),
           "\tmax_dist = " + fmt(rmax), "\tradial_basis_size = %d" % R]
    if name in ("RBChebyshevPoly4", "RBChebyshevPoly5"):
        out.append("\trb_b = " + fmt(b))
    if cfg:
        out.append("\tbasis_function_type = " +
                   ("one_minus_chebyshev" if cfg["one_minus"] else "chebyshev"))
        out.append("\tcutoff_type = " + cfg["cutoff"])
        if cfg["cutoff"] in ("poly3", "poly4", "poly5"):
            out.append("\tcutoff_b = " + fmt(cfg["cutoff_b"]))
        if cfg["cutoff"] == "smoothstep7":
            r1 = cfg["r1"] if cfg["r1"] is not None else rmin + 0.25 * (rmax - rmin)
            r2 = cfg["r2"] if cfg["r2"] is not None else rmin + 0.75 * (rmax - rmin)
            out += ["\tcutoff_r1 = " + fmt(r1), "\tcutoff_r2 = " + fmt(r2)]
        out.append("\tshift_type = " + cfg["shift"])
        if cfg["shift"] in ("exponential", "exponential_left", "exponential_tanh"):
            out.append("\tshift_lambda = " + fmt(cfg["lam"]))
        if cfg["shift"] == "exponential_tanh":
            out.append("\tshift_scale_lambda = " + fmt(cfg["scale_lambda"]))
    return out


def write_mtp(topo, Z, R, rmin, rmax, scaling, coeffs, basis="RBChebyshev", pair_bases=None,
              tag=None) -> str:
    """PotMTP::Save layout (potentials/potential_mtp.cpp:647-785).  basis
    names the shared radial basis; pair_bases, a list of Z*Z (kind, rmin,
    rmax[, b]) in pair order, writes a split file (radial_basis_split = 1)
    instead; tag is an optional potential_tag value."""
    M = topo["M"]
    nrad = Z * Z * M * R
    S = len(topo["map"])
    assert len(coeffs) == nrad + Z + S
    out = ["MTP", "version = 1.1.0", "potential_name = MTP1m", "scaling = " + fmt(scaling),
           "species_count = %d" % Z]
    if tag is not None:
        out.append("potential_tag = " + tag)
    if pair_bases is None:
        out += basis_lines(basis, rmin, rmax, R)
    else:
        assert len(pair_bases) == Z * Z
        out.append("radial_basis_split = 1")
        for q, pb in enumerate(pair_bases):
            out.append("pair %d %d" % (q // Z, q % Z))
            out += basis_lines(pb[0], pb[1], pb[2], R, *pb[3:])
    out += ["radial_funcs_count = %d" % M, "radial_coeffs"]
    q = 0
    for i in range(Z):
        for j in range(Z):
            out.append("\t%d-%d" % (i, j))
            for _ in range(M):
                out.append("\t\t{" + ", ".join(fmt(c) for c in coeffs[q:q + R]) + "}")
                q += R
    out.append("alpha_moments_count = %d" % topo["K"])
    out.append("alpha_index_basic_count = %d" % len(topo["basic"]))
    out.append("alpha_index_basic = {" + ", ".join("{%d, %d, %d, %d}" % tuple(b)
                                                    for b in topo["basic"]) + "}")
    out.append("alpha_index_times_count = %d" % len(topo["times"]))
    out.append("alpha_index_times = {" + ", ".join("{%d, %d, %d, %d}" % tuple(t)
                                                    for t in topo["times"]) + "}")
    out.append("alpha_scalar_moments = %d" % S)
    out.append("alpha_moment_mapping = {" + ", ".join(str(v) for v in topo["map"]) + "}")
    out.append("species_coeffs = {" + ", ".join(fmt(c) for c in coeffs[nrad:nrad + Z]) + "}")
    out.append("moment_coeffs = {" + ", ".join(fmt(c) for c in coeffs[nrad + Z:]) + "}")
    return "\n".join(out) + "\n"


def random_model(template: str, Z: int, R: int, rmin: float, rmax: float, lo: float, hi: float,
                 rng, scaling: float = 0.01, **kw) -> str:
    """A template's moment structure with U[lo, hi] coefficients; kw are
    write_mtp's basis, pair_bases and tag."""
    topo = template_topology(read_template(template))
    n = Z * Z * topo["M"] * R + Z + len(topo["map"])
    return write_mtp(topo, Z, R, rmin, rmax, scaling, uniform(rng, n, lo, hi), **kw)


MTPM_HEADS = ("mtp_m_li", "mtp_m_q2", "mtp_m_fs", "mtp_m_n1", "mtp_m_n2")
ACTIVATIONS = ("TANH", "RELU", "SIGMOID", "LINEAR")


def mtpm_coeff_count(head: str, q: int, h1: int = 0, h2: int = 0) -> int:
    """Head coefficient count (runtime/mtp/mlip.cpp:244-296)."""
    return {"mtp_m_li": 0, "mtp_m_q2": 5, "mtp_m_fs": 1, "mtp_m_n1": h1 * (q + 2),
            "mtp_m_n2": q * h1 + h1 + h1 * h2 + 2 * h2}[head]


def mtpm_model(linear_text: str, head: str, rng, q: int | None = None, h1: int = 0, h2: int = 0,
               activation: str = "TANH", form: str = "both", lo: float = -0.1,
               hi: float = 0.1, head_lo: float = -0.5, head_hi: float = 0.5) -> str:
    """An MTP-M potential (PotMTP_M::Save, potentials/potential_mtp_m.h:
    2256-2336) with the radial part and moment structure of a linear one:
    Z (q + 1) species coefficients, q S moment coefficients and the head's
    model_coeffs, all uniform random.  form says where the head is declared:
    "tag" (a structured potential_tag), "footer" (the "# mtp_*" lines) or
    "both", as Save writes it."""
    if q is None:
        q = {"mtp_m_li": 1, "mtp_m_q2": 2, "mtp_m_fs": 2}.get(head, 3)
    lines = linear_text.rstrip("\n").split("\n")
    Z = int(next(l for l in lines if l.startswith("species_count")).split("=")[1])
    S = int(next(l for l in lines if l.startswith("alpha_scalar_moments")).split("=")[1])
    body = [l for l in lines if not l.startswith(("species_coeffs", "moment_coeffs",
                                                  "potential_tag"))]
    mc = mtpm_coeff_count(head, q, h1, h2)
    if form in ("tag", "both"):
        nn = ""
        if head in ("mtp_m_n1", "mtp_m_n2"):
            layers = "[%d]" % h1 if head == "mtp_m_n1" else "[%d,%d]" % (h1, h2)
            nn = ',"nn":{"activation":"%s","hidden_layers":%s}' % (activation, layers)
        tag = ('{"model":"%s","model_coeffs_count":%d%s,"q":%d,'
               '"schema":"gpml.mtp.metadata","type":"MTP_M","version":1}' % (head, mc, nn, q))
        k = next(i for i, l in enumerate(body) if l.startswith("species_count"))
        body.insert(k + 1, "potential_tag = " + tag)
    body.append("species_coeffs = {" + ", ".join(fmt(c) for c in
                                                 uniform(rng, Z * (q + 1), lo, hi)) + "}")
    body.append("moment_coeffs = {" + ", ".join(fmt(c) for c in uniform(rng, q * S, lo, hi))
                + "}")
    body.append("model_coeffs = {" + ", ".join(fmt(c) for c in
                                               uniform(rng, mc, head_lo, head_hi)) + "}")
    if form in ("footer", "both"):
        body += ["# mtp_model = " + head, "# mtp_descriptor_count = %d" % q,
                 "# mtp_model_coeffs_count = %d" % mc]
        if head in ("mtp_m_n1", "mtp_m_n2"):
            body += ["# mtp_activation = " + activation, "# mtp_hidden1 = %d" % h1,
                     "# mtp_hidden2 = %d" % (h2 if head == "mtp_m_n2" else 0)]
    return "\n".join(body) + "\n"


# ------------------------------------------------------------ workloads --

def workload_inference(wid: int):
    """The E/F/S inference workloads (ids 1-3).  Returns (model_text, Structure)."""
    rng = rng_for(wid)
    if wid == 1:
        model = random_model("shapeev-10.mtp", 1, 8, 2.0, 5.0, -0.1, 0.1, rng)
        s = lattice("fcc", (3, 3, 3), 4.05)
        s = displace(s, rng, 0.1)
    elif wid == 2:
        model = random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, rng)
        s = lattice("fcc", (20, 20, 20), 3.56)
        s.types = assign_species(rng, s.n, fractions_to_counts(s.n, [0.75, 0.25]))
        s = strain(s, rng, 0.02)
        s = displace(s, rng, 0.12)
    elif wid == 3:
        model = random_model("shapeev-20.mtp", 4, 10, 2.0, 5.5, -0.05, 0.05, rng)
        s = lattice("fcc", (40, 40, 40), 3.6)
        s.types = assign_species(rng, s.n, fractions_to_counts(s.n, [0.25] * 4))
        s = displace(s, rng, 0.15)
    else:
        raise ValueError(wid)
    return model, s


def scaled_inference(wid: int, reps) -> tuple[str, Structure]:
    """Workload ``wid``'s model and recipe on a smaller supercell (parity sizes)."""
    rng = rng_for(wid, 7)
    if wid == 2:
        model = random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, rng)
        s = lattice("fcc", reps, 3.56)
        s.types = assign_species(rng, s.n, fractions_to_counts(s.n, [0.75, 0.25]))
        s = strain(s, rng, 0.02)
        s = displace(s, rng, 0.12)
    elif wid == 3:
        model = random_model("shapeev-20.mtp", 4, 10, 2.0, 5.5, -0.05, 0.05, rng)
        s = lattice("fcc", reps, 3.6)
        s.types = assign_species(rng, s.n, fractions_to_counts(s.n, [0.25] * 4))
        s = displace(s, rng, 0.15)
    else:
        raise ValueError(wid)
    return model, s


def training_structures(wid: int, count: int):
    """Training configurations of workloads 4 (FCC/BCC crystals) and 5 (liquids)."""
    rng = rng_for(wid, 1)
    out = []
    if wid == 4:
        shapes = [("fcc", (2, 2, 4)), ("fcc", (2, 3, 4)), ("fcc", (3, 3, 3)), ("fcc", (3, 3, 4)),
                  ("fcc", (4, 4, 4)), ("bcc", (4, 4, 4)), ("bcc", (4, 4, 5)), ("bcc", (4, 5, 5)),
                  ("bcc", (5, 5, 5)), ("bcc", (4, 4, 8))]
        for c in range(count):
            kind, reps = shapes[int(rng.random() * len(shapes))]
            a = 3.56 if kind == "fcc" else 2.87
            s = lattice(kind, reps, a)
            s.types = (uniform(rng, s.n) * 2).astype(np.int32)
            s = strain(s, rng, 0.03)
            s = displace(s, rng, 0.1 + 0.2 * rng.random())
            out.append(s)
    elif wid == 5:
        for c in range(count):
            n = 108 + int(rng.random() * 109)
            out.append(liquid(rng, n, 0.06, 1.5, 3))
    else:
        raise ValueError(wid)
    return out


def training_models(wid: int):
    """(reference model used for labels, starting model) of workloads 4 and 5."""
    rng = rng_for(wid, 2)
    if wid == 4:
        ref = random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, rng)
        start = random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, rng)
    elif wid == 5:
        ref = random_model("shapeev-20.mtp", 3, 10, 1.5, 6.0, -0.05, 0.05, rng)
        start = random_model("shapeev-20.mtp", 3, 10, 1.5, 6.0, -0.05, 0.05, rng)
    else:
        raise ValueError(wid)
    return ref, start


def noisy_labels(rng, n: int, E: float, F: np.ndarray, S: np.ndarray,
                 sigma_e_atom: float = 1e-3, sigma_f: float = 0.05):
    """Labels = reference prediction + Gaussian noise (1 meV/atom on E, 0.05 eV/A on F)."""
    e = E + n * sigma_e_atom * gaussian(rng, 1)[0]
    f = F + sigma_f * gaussian(rng, 3 * n).reshape(n, 3)
    return e, f, np.array(S, copy=True)
