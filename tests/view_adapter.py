"""The view a reference caller hands to MTPGpuDirect::initialize, made from
.mtp text for the tests.

MTPGpuEvaluator::initialize (potentials/mtp_gpu_adapter.cpp:420-468) fills
MTPGpuPotentialView from a loaded PotMTP: sizes, the flat tables, the
coefficient pointers (the MTP-M head's at :330-390), the species map, and one
MTPGpuRadialBasisView per ordered species pair for split models and for
shared bases other than RBChebyshev / RBChebyCos (radial_basis_for,
:110-212).  This module does the same from the text that
mtpx_format_model_text writes, so the test can load a model through the
view and compare it with the oracle's evaluation of the text.
"""
from __future__ import annotations

import re

import numpy as np

from mtpx import capi


def _num(s):
    return float(s)


def _blocks(text):
    """(key -> value) of the top-level "key = value" lines, and the radial
    basis blocks as lists of (key, value)."""
    top, bases, cur = {}, [], None
    for line in text.splitlines():
        if line.startswith("pair "):
            continue
        if line.startswith("radial_basis_type = "):
            cur = {"radial_basis_type": line.split("=", 1)[1].strip()}
            bases.append(cur)
            continue
        if line.startswith("\t") and cur is not None and "=" in line and not line.startswith("\t\t"):
            k, v = line.strip().split("=", 1)
            cur[k.strip()] = v.strip()
            continue
        if not line.startswith("\t"):
            cur = None
            if "=" in line:
                k, v = line.split("=", 1)
                top[k.strip()] = v.strip()
    return top, bases


def _ints(s):
    return np.array([int(v) for v in re.findall(r"-?\d+", s)], np.int32)


def _basis_view(b):
    """radial_basis_for (potentials/mtp_gpu_adapter.cpp:110-212)."""
    kind = b["radial_basis_type"]
    out = dict(radial_basis=capi.RB_KINDS[kind], min_dist=_num(b["min_dist"]),
               max_dist=_num(b["max_dist"]), scaling=_num(b.get("scaling", "0.01")))
    if kind in ("RBChebyshevPoly4", "RBChebyshevPoly5"):
        out["cutoff_parameter"] = _num(b["rb_b"])
    if kind == "RBChebyshevConfigurable":
        out["one_minus_chebyshev"] = int(b["basis_function_type"] == "one_minus_chebyshev")
        out["cutoff"] = capi.CUTOFFS[b["cutoff_type"]]
        out["transform"] = capi.SHIFTS[b["shift_type"]]
        out["cutoff_parameter"] = _num(b.get("cutoff_b", "0"))
        out["cutoff_r1"] = _num(b.get("cutoff_r1", "0"))
        out["cutoff_r2"] = _num(b.get("cutoff_r2", "0"))
        out["transform_parameter"] = _num(b.get("shift_lambda", "0"))
        out["transform_scale_parameter"] = _num(b.get("shift_scale_lambda", "0"))
    return out


def view_of_text(text: str, spmap=None, max_type=None, force_pairs=False):
    """(ModelView, canonical text) of a model.  spmap defaults to the
    adapter's identity over the species (mtp_gpu_adapter.cpp:424-430);
    force_pairs passes Z^2 pair descriptors even where the adapter would
    pass the scalar fields."""
    canon = capi.format_model_text(text)
    top, bases = _blocks(canon)
    info, coef = capi.parse_model_text(canon)
    head = capi.parse_model_head(canon)
    Z, M, R, K, B, T, S = (info[k] for k in "ZMRKBTS")
    scaling = _num(top["scaling"])
    for b in bases:
        b.setdefault("scaling", top["scaling"])
    split = int(top.get("radial_basis_split", "0")) != 0
    first = _basis_view(bases[0])
    pairs = None
    if split:
        pairs = [_basis_view(b) for b in bases]
    elif force_pairs or first["radial_basis"] not in (0, 1):
        pairs = [dict(first) for _ in range(Z * Z)]
    cutoff = max(b["max_dist"] for b in (pairs or [first]))
    nrad = Z * Z * M * R
    f = dict(species_count=Z, alpha_moments_count=K, alpha_index_basic_count=B,
             alpha_index_times_count=T, alpha_scalar_moments=S, radial_func_count=M, rb_size=R,
             min_dist=first["min_dist"], max_dist=first["max_dist"], cutoff=cutoff,
             scaling=scaling, radial_basis=first["radial_basis"],
             radial_coeffs=coef[:nrad], radial_coeffs_count=nrad,
             species_coeffs=coef[nrad:nrad + Z],
             alpha_index_basic=_ints(top["alpha_index_basic"]),
             alpha_index_times=_ints(top["alpha_index_times"]) if T else None,
             alpha_moment_mapping=_ints(top["alpha_moment_mapping"]))
    basic = f["alpha_index_basic"].reshape(B, 4)
    f["max_mu"] = int(basic[:, 0].max())
    f["max_alpha_index_basic"] = int(basic[:, 1:].sum(1).max())
    if head["head"] == "linear":
        f["model"] = capi.VIEW_MODELS["linear"]
        f["moment_coeffs"] = coef[nrad + Z:nrad + Z + S]
    else:
        q, mc = head["q"], head["model_coeffs_count"]
        o = nrad + Z
        f["model"] = capi.VIEW_MODELS[head["head"]]
        f["descriptor_count"] = q
        f["descriptor_species_coeffs"] = coef[o:o + q * Z]
        f["descriptor_moment_coeffs"] = coef[o + q * Z:o + q * Z + q * S]
        f["model_coeffs"] = coef[o + q * Z + q * S:o + q * Z + q * S + mc] if mc else None
        f["model_coeffs_count"] = mc
        f["model_activation"] = capi.VIEW_ACTIVATIONS[head["activation"]]
        f["model_hidden1"] = head["hidden1"]
        f["model_hidden2"] = head["hidden2"]
    if spmap is None:
        spmap = np.arange(Z, dtype=np.int32)
    f["spmap"] = np.asarray(spmap, np.int32)
    f["max_type"] = int(max_type if max_type is not None else len(spmap))
    return capi.make_view(f, pairs), canon


def without_tag(text: str) -> str:
    """The text without its potential_tag line (a view carries no tag)."""
    return "\n".join(l for l in text.splitlines() if not l.startswith("potential_tag"))
