"""Models loaded through the view (mtpx_load_model = MTPGpuDirect::initialize
over MTPGpuPotentialView, runtime/mtp/gpu-direct/mtp_gpu_direct.h:215-289),
on the device, against the oracle's evaluation of the text the view was made
from.

- E/F/S at 1e-10 relative for a ChebyCos basis, a split model, a
  configurable basis, an MTP-M head and a level-16 model.
- The same model loaded from text and from its view gives the same
  coefficients and bit-identical E/F/S.
- A non-identity species map with 1-based LAMMPS types (make_lammps_pair_view,
  mtp_gpu_direct.h:291-330): max_type Z+1, type 0 unmapped (-1), types 1..Z
  mapped in reverse, through mtpx_build_neighbors, mtpx_set_structures and
  mtpx_compute_sites (whose type -> species step the reference takes at
  mtp_gpu_direct.cu:580, 1430, 1581).  Results equal the oracle's on the
  structure with the mapped species.
"""
import copy

import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from mtpx import synth as S
from test_gpm import MODELS
from test_model_io import model_text
from test_mtpm import head_text, structure
from test_sites_gpu import ghost_system
from view_adapter import view_of_text

TOL = 1e-10
pytestmark = pytest.mark.gpu

CASES = {
    "chebycos": lambda: model_text("chebycos"),
    "split": lambda: model_text("split"),
    "configurable": lambda: model_text("configurable"),
    "split-configurable": MODELS["split-configurable"],
    "mtp_m_n2": lambda: head_text("mtp_m_n2", 4, 3, "SIGMOID"),
    "mtp_m_q2": lambda: head_text("mtp_m_q2"),
    "level16": MODELS["level16"],
}


def _oracle(text, s, types=None):
    m = O.Model(text)
    types = s.types if types is None else types
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, types, m.cutoff)
    return m, pos, O.efs(m, nb)


@pytest.mark.parametrize("kind", list(CASES))
def test_view_model_matches_oracle(ctx, kind):
    text = CASES[kind]()
    s = structure(seed=43)
    m, pos, (E, F, St, se) = _oracle(text, s)
    view, _ = view_of_text(text)
    ctx.load_model_view(view)
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, m.cutoff)
    for det in (False, True):
        Eg, Fg, Sg, seg = ctx.efs(deterministic=det)
        assert rel_err(Eg, E) < TOL
        assert rel_err(Fg, F) < TOL
        assert rel_err(Sg, St) < TOL
        assert rel_err(seg, se) < TOL


@pytest.mark.parametrize("kind", ["split-configurable", "mtp_m_n2", "level16"])
def test_view_and_text_load_the_same_model(ctx, kind):
    text = CASES[kind]()
    s = structure(seed=44)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    ctx.load_model_text(text)
    coef_t = ctx.get_coeffs()
    cut = O.Model(text).cutoff
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, cut)
    ref = ctx.efs(deterministic=True)
    view, _ = view_of_text(text)
    ctx.load_model_view(view)
    assert np.array_equal(ctx.get_coeffs().view(np.uint64), coef_t.view(np.uint64))
    ctx.build_neighbors(s.cell, s.pbc, pos, s.types, cut)
    got = ctx.efs(deterministic=True)
    for a, b in zip(got, ref):
        assert np.array_equal(np.asarray(a).view(np.uint64), np.asarray(b).view(np.uint64))


def _lammps_map(Z):
    """1-based LAMMPS types: type 0 unused, type t -> species Z - t."""
    return np.array([-1] + [Z - t for t in range(1, Z + 1)], np.int32)


def test_species_map_through_every_entry_point(ctx):
    text = CASES["split-configurable"]()
    Z = 2
    spmap = _lammps_map(Z)
    s = structure(seed=45)
    species = s.types.astype(np.int32)
    lammps = (Z - species).astype(np.int32)  # spmap[lammps] == species
    assert np.array_equal(spmap[lammps], species)
    m, pos, (E, F, St, se) = _oracle(text, s)
    view, _ = view_of_text(text, spmap=spmap)
    ctx.load_model_view(view)
    # a single structure built from LAMMPS types
    ctx.build_neighbors(s.cell, s.pbc, pos, lammps, m.cutoff)
    nb = ctx.get_neighbors()
    assert np.array_equal(nb["center_types"], species)  # lists hold species
    Eg, Fg, Sg, _ = ctx.efs()
    assert rel_err(Eg, E) < TOL and rel_err(Fg, F) < TOL and rel_err(Sg, St) < TOL
    # a batch of two structures
    sl = copy.copy(s)
    sl.types = lammps
    ctx.set_structures([sl, sl], m.cutoff)
    Eb, Fb, Sb, _ = ctx.compute_batch()
    assert rel_err(Eb, np.array([E, E])) < TOL
    assert rel_err(Fb, np.concatenate([F, F])) < TOL
    # a ghost-atom site request in LAMMPS types
    g = ghost_system(m, s)
    out = ctx.compute_sites(g["offsets"], g["neighbors"], (Z - g["types"]).astype(np.int32),
                            x=g["pts"], nlocal=g["n"], accumulate=False, deterministic=True)
    assert rel_err(out["energy"], E) < TOL
    # types outside [0, max_type) are refused; type 0 (species -1) is refused
    # outside site requests
    with pytest.raises(capi.MtpxError, match="species-map range"):
        ctx.build_neighbors(s.cell, s.pbc, pos, np.full(s.n, Z + 1, np.int32), m.cutoff)
    with pytest.raises(capi.MtpxError, match="maps to species -1"):
        ctx.build_neighbors(s.cell, s.pbc, pos, np.zeros(s.n, np.int32), m.cutoff)


def test_unmapped_type_is_skipped_in_site_requests(ctx):
    """Atoms of LAMMPS type 0 (species -1) drop out of a site request, as
    the reference's species map returning -1 does: the result equals the
    request with those atoms' type set negative under the identity map."""
    text = CASES["chebycos"]()
    Z = 2
    s = structure(seed=46)
    m = O.Model(text)
    g = ghost_system(m, s)
    species = g["types"].copy()
    lammps = (Z - species).astype(np.int32)
    drop = (np.arange(len(lammps)) % 7) == 3
    lammps[drop] = 0
    species_neg = species.copy()
    species_neg[drop] = -1
    ctx.load_model_text(text)
    ref = ctx.compute_sites(g["offsets"], g["neighbors"], species_neg, x=g["pts"],
                            nlocal=g["n"], accumulate=False, deterministic=True)
    ctx.set_species_map(_lammps_map(Z))
    got = ctx.compute_sites(g["offsets"], g["neighbors"], lammps, x=g["pts"], nlocal=g["n"],
                            accumulate=False, deterministic=True)
    assert got["energy"] == ref["energy"]
    assert np.array_equal(got["force"], ref["force"])
    ctx.set_species_map(None)
    with pytest.raises(capi.MtpxError):
        ctx.set_species_map(np.array([0, 2], np.int32))
