"""Pin the CPU oracle to the reference.

* Golden vectors (tests/golden/*.npz, written by make_golden.py from the
  reference binaries compiled from the IMR-MLP sources): neighbour lists bit
  for bit, E/F/virial to 1e-12.
* The reference binaries themselves (oracle/_ref, when built in this
  container) on further seeded inputs.
* The reference's recorded template inventory (sources.json "shapeev/10").
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import synth as S

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")


def _groups(npz):
    names = sorted({k.split("/")[0] for k in npz.files})
    return names


NBH = np.load(os.path.join(GOLDEN, "nbh_golden.npz"))
EFS = np.load(os.path.join(GOLDEN, "efs_golden.npz"))


def _same_lists(nb, ref):
    assert np.array_equal(nb.offsets, ref["offsets"])
    assert np.array_equal(nb.idx, ref["idx"])
    assert np.array_equal(nb.types, ref["types"])
    assert np.array_equal(nb.center_types, ref["center_types"])
    assert np.array_equal(nb.vec.view(np.uint64), np.asarray(ref["vec"]).view(np.uint64))
    assert np.array_equal(nb.dist.view(np.uint64), np.asarray(ref["dist"]).view(np.uint64))


@pytest.mark.parametrize("name", _groups(NBH))
def test_oracle_lists_match_reference_golden(name):
    g = {k.split("/in_")[1]: NBH[k] for k in NBH.files if k.startswith(name + "/in_")}
    ref = {k.split("/ref_")[1]: NBH[k] for k in NBH.files if k.startswith(name + "/ref_")}
    nb = O.Neighbors.build(g["cell"], g["pbc"], g["pos"], g["types"], float(g["cutoff"]))
    _same_lists(nb, ref)


@pytest.mark.parametrize("name", _groups(EFS))
def test_oracle_efs_matches_reference_golden(name):
    g = {k.split("/", 1)[1]: EFS[k] for k in EFS.files if k.startswith(name + "/")}
    m = O.Model(str(g["model"]))
    nb = O.Neighbors.build(g["cell"], g["pbc"], g["pos"], g["types"], m.cutoff)
    E, F, St, se = O.efs(m, nb)
    sym = 0.5 * (St + St.T)
    v6 = np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])
    assert rel_err(E, g["ref_E"]) < 1e-12
    assert rel_err(se, g["ref_site"]) < 1e-12
    assert rel_err(F, g["ref_F"]) < 1e-12
    assert rel_err(v6, g["ref_virial6"]) < 1e-12


needs_ref = pytest.mark.skipif(not (O.ref_available("nbh_ref") and O.ref_available("mlip_ref")),
                               reason="reference binaries not built (make -C oracle ref)")


@needs_ref
def test_oracle_lists_match_reference_binary_random(workdir):
    rng = S.rng_for(600)
    for k in range(12):
        kind = "fcc" if k % 2 == 0 else "bcc"
        s = S.lattice(kind, (2, 2, 2 + k % 3), 3.6 if kind == "fcc" else 2.9)
        s = S.displace(S.strain(s, rng, 0.1), rng, 0.25)
        cell = s.cell.copy()
        cell[2] += (rng.random() - 0.5) * cell[0] + (rng.random() - 0.5) * cell[1]
        s.cell = cell
        s.types = (S.uniform(rng, s.n) * 3).astype(np.int32)
        rc = 3.0 + 3.0 * rng.random()
        pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, rc)
        _same_lists(nb, O.ref_neighbors(s.cell, s.pbc, pos, s.types, rc, workdir))


@needs_ref
def test_oracle_lists_match_reference_binary_liquid(workdir):
    for s in S.training_structures(5, 2):
        pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, 6.0)
        _same_lists(nb, O.ref_neighbors(s.cell, s.pbc, pos, s.types, 6.0, workdir))


@needs_ref
def test_oracle_efs_matches_reference_binary(workdir):
    for wid, reps in [(2, (3, 3, 3)), (3, (3, 3, 2))]:
        text, s = S.scaled_inference(wid, reps)
        m = O.Model(text)
        pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
        E, F, St, se = O.efs(m, nb)
        Er, ser, Fr, vr = O.ref_mlip_efs(text, nb, s.types, m.cutoff, workdir, m.Z)
        sym = 0.5 * (St + St.T)
        v6 = np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])
        assert rel_err(E, Er) < 1e-12 and rel_err(F, Fr) < 1e-12 and rel_err(v6, vr) < 1e-12
        assert rel_err(se, ser) < 1e-12


@needs_ref
def test_duplicate_mapping_energy_matches_reference_binary(workdir):
    """The duplicate-mapping model (alpha_moment_mapping {0, 4, 5, 6, 4}):
    energies and site energies agree with the reference core to 1e-12.
    Forces are not compared with it: runtime/mtp/mlip.cpp:1101 assigns the
    adjoint seed of a scalar's moment (=) where PotMTP adds it
    (potential_mtp.cpp:2976, +=), so that core's forces for this model are
    not minus its own energy gradient; the oracle's are
    (test_oracle_math.test_duplicate_scalar_mapping_accumulates)."""
    from test_oracle_math import _dup_case
    text, s = _dup_case()
    m = O.Model(text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, se = O.efs(m, nb)
    Er, ser, Fr, vr = O.ref_mlip_efs(text, nb, s.types, m.cutoff, workdir, m.Z)
    assert rel_err(E, Er) < 1e-12 and rel_err(se, ser) < 1e-12
    # the reference core's forces miss the first duplicate's coefficient
    assert rel_err(F, Fr) > 1e-6


def test_level10_template_inventory():
    """sources.json records shapeev/10 as 41 moments, 25 basic, 42 products,
    16 scalars; the carved template must reproduce it."""
    m = O.Model(S.random_model("shapeev-10.mtp", 1, 8, 2.0, 5.0, -0.1, 0.1, S.rng_for(1)))
    assert (m.K, m.B, m.T, m.S, m.M) == (41, 25, 42, 16, 3)


def test_template_inventories():
    for name, inv in {"shapeev-16.mtp": (299, 130, 741, 92), "shapeev-20.mtp": (1035, 295, 4665, 288),
                      "shapeev-20-t.mtp": (1042, 295, 4526, 288),
                      "shapeev-02.mtp": (1, 1, 0, 1), "shapeev-06.mtp": (8, 5, 5, 5)}.items():
        m = O.Model(S.read_template(name))
        assert (m.K, m.B, m.T, m.S) == inv, name
