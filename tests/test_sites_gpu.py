"""CSR site requests with ghost atoms (mtpx_compute_sites) against the oracle.

The request is the one the LAMMPS pair style mlip/gpudirect sends
(LAMMPS/USER-MLIP/pair_MLIP_gpu_direct.cpp:577-603; MTPGpuComputeRequest /
MTPGpuBatchRequest, runtime/mtp/gpu-direct/mtp_gpu_direct.h:359-517) with the
semantics of MLIPCore::compute (runtime/mtp/mlip.cpp:907-1191): owned atoms
plus ghost atoms (the periodic images within the cutoff), full lists over
both, forces on ghosts folded back onto their owners afterwards -- the
folding oracle/ref_drivers/mlip_ref.cpp does around the reference core.

Tolerance 1e-10 relative (largest absolute difference over the largest
magnitude) against the oracle's periodic E/F/S (PotMTP::getEFS); the
per-atom virial against -1/2 D r^T per entry end (symmetrised), formed from
the oracle's per-site derivatives."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import synth as S

TOL = 1e-10
pytestmark = pytest.mark.gpu


def ghost_system(model, s, list_cutoff=None):
    """Owned atoms + periodic images as ghosts, and brute-force full lists
    over them (strict r < cutoff, r > 0) -- the input LAMMPS hands over."""
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, model.cutoff)
    pts, orig = nb.points()
    rc = model.cutoff if list_cutoff is None else list_cutoff
    n = s.n
    off = [0]
    nbr = []
    for i in range(n):
        d = pts - pts[i]
        rr = np.einsum("ij,ij->i", d, d)
        sel = np.nonzero((rr < rc * rc) & (np.arange(len(pts)) != i))[0]
        nbr.extend(sel.tolist())
        off.append(len(nbr))
    types = s.types[orig].astype(np.int32)
    return dict(pos=pos, nb=nb, pts=pts, orig=orig, types=types, offsets=np.array(off, np.int32),
                neighbors=np.array(nbr, np.int32), n=n)


def fold(values, orig, n):
    out = np.zeros((n,) + values.shape[1:])
    np.add.at(out, orig, values)
    return out


def half_virial(D, r):
    return np.stack([-0.5 * D[:, 0] * r[:, 0], -0.5 * D[:, 1] * r[:, 1], -0.5 * D[:, 2] * r[:, 2],
                     -0.25 * (D[:, 1] * r[:, 0] + D[:, 0] * r[:, 1]),
                     -0.25 * (D[:, 2] * r[:, 0] + D[:, 0] * r[:, 2]),
                     -0.25 * (D[:, 2] * r[:, 1] + D[:, 1] * r[:, 2])], axis=1)


def oracle_site_virial(model, nb):
    """Per-atom virial folded onto owners: each entry's -1/2 D r^T to the
    centre and to the neighbour's owner."""
    out = np.zeros((nb.n, 6))
    for i in range(nb.n):
        sl = slice(nb.offsets[i], nb.offsets[i + 1])
        _, D = O.site_efs(model, nb, i)
        h = half_virial(D, nb.vec[sl])
        out[i] += h.sum(axis=0)
        np.add.at(out, nb.idx[sl], h)
    return out


def virial6(St):
    sym = 0.5 * (St + St.T)
    return np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])


@pytest.fixture(scope="module")
def case():
    text, s = S.scaled_inference(2, (3, 3, 3))
    m = O.Model(text)
    g = ghost_system(m, s)
    E, F, St, se = O.efs(m, g["nb"])
    return dict(text=text, s=s, m=m, g=g, E=E, F=F, St=St, se=se,
                sv=oracle_site_virial(m, g["nb"]))


@pytest.mark.parametrize("deterministic", [False, True])
def test_ghost_request_matches_periodic_oracle(ctx, case, deterministic):
    g, n = case["g"], case["g"]["n"]
    ctx.load_model_text(case["text"])
    start = S.rng_for(41).random((len(g["pts"]), 3))
    out = ctx.compute_sites(g["offsets"], g["neighbors"], g["types"], x=g["pts"], nlocal=n,
                            force=start, accumulate=True, deterministic=deterministic)
    f_ghost = out["force"] - start  # accumulate_force: added onto the given forces
    assert np.abs(f_ghost[n:]).max() > 0  # ghosts carry reactions before folding
    assert rel_err(out["energy"], case["E"]) < TOL
    assert rel_err(out["site_energy"], case["se"]) < TOL
    assert rel_err(fold(f_ghost, g["orig"], n), case["F"]) < TOL
    assert rel_err(out["virial6"], virial6(case["St"])) < TOL
    assert rel_err(fold(out["site_virial"], g["orig"], n), case["sv"]) < TOL
    # the per-atom virials (ghosts included) add up to the global virial
    assert rel_err(out["site_virial"].sum(axis=0), out["virial6"]) < 1e-12


def test_overwrite_vectors_mask_and_repeatability(ctx, case):
    g, n = case["g"], case["g"]["n"]
    ctx.load_model_text(case["text"])
    base = ctx.compute_sites(g["offsets"], g["neighbors"], g["types"], x=g["pts"], nlocal=n,
                             accumulate=False, deterministic=True)
    # neighbour vectors instead of positions; special-bond bits above the mask
    vec = g["pts"][g["neighbors"]] - np.repeat(g["pts"][:n], np.diff(g["offsets"]), axis=0)
    tagged = g["neighbors"] | (np.arange(len(g["neighbors"])) % 4 << 29).astype(np.int32)
    got = ctx.compute_sites(g["offsets"], tagged, g["types"], vectors=vec, nlocal=n,
                            mask=(1 << 29) - 1, force=np.full((len(g["pts"]), 3), 7.0),
                            accumulate=False, deterministic=True)
    assert rel_err(got["force"], base["force"]) < 1e-13
    assert rel_err(got["energy"], base["energy"]) < 1e-13
    again = ctx.compute_sites(g["offsets"], tagged, g["types"], vectors=vec, nlocal=n,
                              mask=(1 << 29) - 1, accumulate=False, deterministic=True)
    for k in ("force", "site_virial", "site_energy", "virial6"):
        assert np.array_equal(np.asarray(got[k]).view(np.uint64),
                              np.asarray(again[k]).view(np.uint64)), k


def test_negative_types_skip_atoms(ctx, case):
    """A species map entry of -1 (mlip.cpp:945, 957): the atom is neither a
    centre nor a neighbour, so the result equals the structure without it."""
    g, s, m = case["g"], case["s"], case["m"]
    n, k = g["n"], 5
    types = g["types"].copy()
    types[g["orig"] == k] = -1
    ctx.load_model_text(case["text"])
    out = ctx.compute_sites(g["offsets"], g["neighbors"], types, x=g["pts"], nlocal=n,
                            accumulate=False)
    keep = np.arange(n) != k
    sr = S.Structure(s.cell, O.wrap(s.cell, s.pbc, s.pos)[keep], s.types[keep], s.pbc)
    nbr = O.Neighbors.build(sr.cell, sr.pbc, sr.pos, sr.types, m.cutoff)
    E, F, St, se = O.efs(m, nbr)
    f = fold(out["force"], g["orig"], n)
    assert rel_err(out["energy"], E) < TOL
    assert rel_err(f[keep], F) < TOL and np.all(f[k] == 0)
    assert out["site_energy"][k] == 0 and rel_err(out["site_energy"][keep], se) < TOL
    assert rel_err(out["virial6"], virial6(St)) < TOL


def test_reuse_topology_with_skin(ctx, case):
    """Lists built with a skin are kept (reuse_topology, neighbor->ago != 0
    in the pair style); moved positions are re-evaluated on them and entries
    beyond the cutoff are skipped."""
    s, m = case["s"], case["m"]
    g = ghost_system(m, s, list_cutoff=m.cutoff + 0.6)
    n = g["n"]
    ctx.load_model_text(case["text"])
    first = ctx.compute_sites(g["offsets"], g["neighbors"], g["types"], x=g["pts"], nlocal=n,
                              accumulate=False)
    assert rel_err(first["energy"], case["E"]) < TOL
    shift = 0.05 * (S.rng_for(42).random((n, 3)) - 0.5)
    pts2 = g["pts"] + shift[g["orig"]]  # ghosts move with their owners
    second = ctx.compute_sites(g["offsets"], g["neighbors"], g["types"], x=pts2, nlocal=n,
                               accumulate=False, reuse=True)
    moved = S.Structure(s.cell, g["pos"] + shift, s.types, s.pbc)
    nb2 = O.Neighbors.build(moved.cell, moved.pbc, O.wrap(moved.cell, moved.pbc, moved.pos),
                            moved.types, m.cutoff)
    E2, F2, St2, _ = O.efs(m, nb2)
    assert rel_err(second["energy"], E2) < TOL
    assert rel_err(fold(second["force"], g["orig"], n), F2) < TOL
    assert rel_err(second["virial6"], virial6(St2)) < TOL


def test_centre_subset_and_order(ctx, case):
    """centers[] lists the centre atoms in any order (LAMMPS ilist); owned
    atoms that are not centres get no site energy."""
    g, n, m = case["g"], case["g"]["n"], case["m"]
    order = np.random.default_rng(3).permutation(n)[: n // 2]
    off = [0]
    nbr = []
    for i in order:
        nbr.extend(g["neighbors"][g["offsets"][i]:g["offsets"][i + 1]].tolist())
        off.append(len(nbr))
    ctx.load_model_text(case["text"])
    out = ctx.compute_sites(np.array(off), np.array(nbr), g["types"], x=g["pts"], centers=order,
                            nlocal=n, accumulate=False)
    assert rel_err(out["energy"], case["se"][order].sum()) < TOL
    assert rel_err(out["site_energy"][order], case["se"][order]) < TOL
    rest = np.setdiff1d(np.arange(n), order)
    assert np.all(out["site_energy"][rest] == 0)


def test_empty_request(ctx, case):
    ctx.load_model_text(case["text"])
    out = ctx.compute_sites(np.array([0]), np.zeros(0), np.zeros(0), x=np.zeros((0, 3)))
    assert out["energy"] == 0 and out["force"].shape == (0, 3)
    out = ctx.compute_sites(np.array([0, 0]), np.zeros(0), np.array([0]), x=np.zeros((1, 3)))
    coef = ctx.get_coeffs()
    nrad = ctx.info["Z"] ** 2 * ctx.info["M"] * ctx.info["R"]
    assert out["energy"] == coef[nrad] and np.all(out["force"] == 0)


def test_add_efs_accumulates(ctx, case):
    """PotMTP::add_efs (potential_mtp.cpp:1904-1907): getEFS adds onto the
    outputs instead of overwriting them."""
    nb = case["g"]["nb"]
    ctx.load_model_text(case["text"])
    ctx.set_neighbors(nb.offsets, nb.idx, nb.types, nb.vec, nb.dist, nb.center_types)
    E, F, St, se = ctx.efs(deterministic=True)
    rng = S.rng_for(43)
    init = (1.5, rng.random(F.shape), rng.random((3, 3)), rng.random(se.shape))
    ctx.set_add_efs(True)
    try:
        E2, F2, S2, se2 = ctx.efs(deterministic=True, init=init)
    finally:
        ctx.set_add_efs(False)
    assert E2 == init[0] + E
    assert np.array_equal(F2, init[1] + F) and np.array_equal(S2, init[2] + St)
    assert np.array_equal(se2, init[3] + se)
    E3, F3, _, _ = ctx.efs(deterministic=True, init=init)
    assert E3 == E and np.array_equal(F3, F)
