"""Linear fit on the device against the oracle's restatement of
CalcEFSCmpt_R / CalcSiteBasisDers (potentials/potential_mtp.cpp:2675-2707,
3163-3280), AddLinearFast (train/train_mtp.cpp:1289-1395), the Gram of
TrainLinearFast (:2426-2427) and Orthogonalize (:3849-3930).

Tolerances: components, rows and the normal equations 1e-10 relative
(largest absolute difference over the largest magnitude)."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from mtpx import synth as S

pytestmark = pytest.mark.gpu


def _crystals(count, seed, drop=False):
    ref_text, start_text = S.training_models(4)
    mref = O.Model(ref_text)
    rng = S.rng_for(900 + seed)
    structs, nbs, labels = [], [], []
    for k, s in enumerate(S.training_structures(4, count)):
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, 5.0)
        E, F, St, _ = O.efs(mref, nb)
        e, f, st = S.noisy_labels(rng, s.n, E, F, St)
        lb = O.Labels(s.n, energy=e, forces=f, stress=st, fitness=0.5 + rng.random())
        if drop:
            if k % 4 == 1:
                lb.forces = None
            if k % 4 == 2:
                lb.stress = None
            if k % 4 == 3:
                lb.energy = None
            if k % 3 == 0:
                af = 0.5 + rng.random(s.n)
                af[::5] = 0.0  # atoms excluded from the force rows
                lb.atomic_fitness = af
        structs.append(s)
        nbs.append(nb)
        labels.append(lb)
    return start_text, structs, nbs, labels


def _upload(ctx, text, structs, labels, settings, cutoff=5.0):
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, cutoff)
    has = np.array([[lb.energy is not None, lb.forces is not None, lb.stress is not None]
                    for lb in labels], np.int32)
    tf = np.concatenate([lb.forces if lb.forces is not None else np.zeros((lb.n, 3))
                         for lb in labels])
    fit = np.array([lb.fitness for lb in labels])
    af = np.concatenate([lb.atomic_fitness if lb.atomic_fitness is not None else np.ones(lb.n)
                         for lb in labels])
    st = capi.LossSettings.make(*[getattr(settings, f[0]) for f in settings._fields_])
    active, wE, wF, wS = capi.loss_weights(st, off, has, tf, fit, af)
    tE = np.array([lb.energy if lb.energy is not None else 0.0 for lb in labels])
    tS = np.array([lb.stress if lb.stress is not None else np.zeros((3, 3)) for lb in labels])
    ctx.set_labels(active, tE, wE, tf, wF, tS, wS)
    return off


@pytest.fixture(scope="module")
def crystal_set():
    return _crystals(6, 1, drop=True)


SETTINGS = {"linear": O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=0.001),
            "per-atom": O.LossSettings.make(weight_eng=1.0, weight_force=0.01,
                                            weight_stress=0.001, eng_pow=2.0, force_pow=1.0,
                                            stress_pow=0.0),
            "force-norm": O.LossSettings.make(force_norm_f=1.0, force_norm_p=1.5)}


def test_components_match_oracle(ctx, crystal_set):
    text, structs, nbs, labels = crystal_set
    off = _upload(ctx, text, structs, labels, SETTINGS["linear"])
    m = O.Model(text)
    ec, fc, sc = ctx.efs_components()
    for c, nb in enumerate(nbs):
        eo, fo, so = O.efs_components(m, nb)
        assert rel_err(ec[c], eo) < 1e-10
        assert rel_err(fc[off[c]:off[c + 1]], fo) < 1e-10
        assert rel_err(sc[c], so) < 1e-10


def test_components_reproduce_efs(ctx, crystal_set):
    """sum_q x_q components_q equals the device E/F/S."""
    text, structs, nbs, labels = crystal_set
    _upload(ctx, text, structs, labels, SETTINGS["linear"])
    ec, fc, sc = ctx.efs_components()
    x = ctx.get_coeffs()
    info = ctx.info
    lin = x[info["Z"] * info["Z"] * info["M"] * info["R"]:]
    E, F, St, _ = ctx.compute_batch()
    assert rel_err(ec @ lin, E) < 1e-10
    assert rel_err(fc @ lin, F) < 1e-10
    assert rel_err(sc @ lin, St) < 1e-10


@pytest.mark.parametrize("name", list(SETTINGS))
def test_linear_rows_match_oracle(ctx, crystal_set, name):
    text, structs, nbs, labels = crystal_set
    st = SETTINGS[name]
    _upload(ctx, text, structs, labels, st)
    m = O.Model(text)
    A, y = ctx.linear_rows()
    Ao = np.concatenate([O.linear_rows(m, nb, st, lb)[0] for nb, lb in zip(nbs, labels)])
    yo = np.concatenate([O.linear_rows(m, nb, st, lb)[1] for nb, lb in zip(nbs, labels)])
    assert A.shape == Ao.shape
    assert rel_err(A, Ao) < 1e-10 and rel_err(y, yo) < 1e-10


@pytest.mark.parametrize("name", list(SETTINGS))
def test_linear_system_matches_oracle(ctx, crystal_set, name):
    text, structs, nbs, labels = crystal_set
    st = SETTINGS[name]
    _upload(ctx, text, structs, labels, st)
    m = O.Model(text)
    G, b = ctx.linear_system()
    Go, bo = O.linear_system_batch(m, nbs, labels, st, threads=8)
    assert rel_err(G, Go) < 1e-10 and rel_err(b, bo) < 1e-10
    assert np.array_equal(G, G.T)


def test_components_independent_of_grouping(ctx, crystal_set, monkeypatch):
    """Structures are processed in groups bounded by a budget for the sites'
    Jacobian values (MTPX_LIN_GROUP_MB): a 1 MB budget puts every structure
    in a group of its own; the components are bitwise those of one group
    (each row has one writer, which sums in site order)."""
    text, structs, nbs, labels = crystal_set
    _upload(ctx, text, structs, labels, SETTINGS["linear"])
    monkeypatch.setenv("MTPX_LIN_GROUP_MB", "1")
    small = ctx.efs_components()
    monkeypatch.setenv("MTPX_LIN_GROUP_MB", "4096")
    big = ctx.efs_components()
    again = ctx.efs_components()
    for a, b, c in zip(small, big, again):
        assert np.array_equal(a, b) and np.array_equal(b, c)


def test_components_of_large_structures(ctx, monkeypatch):
    """Structures of every tile size class, up to 1,372 atoms (beyond what
    one LDS tile holds, so their rows accumulate in the output itself):
    components 1e-10 against the oracle; every structure through the
    output-row path (MTPX_LIN_TILE_ROWS=0) gives the same components to
    rounding (the two atomic units order the adds of one instruction to the
    same row, periodic images of one atom, differently) and is repeatable
    bit for bit, as the default path is."""
    ref_text, text = S.training_models(4)
    m = O.Model(text)
    rng = S.rng_for(91)
    structs, nbs = [], []
    for kind, reps in [("fcc", (2, 2, 2)), ("bcc", (4, 4, 5)), ("fcc", (4, 4, 5)),
                       ("fcc", (5, 5, 5)), ("bcc", (7, 7, 7)), ("fcc", (7, 7, 7))]:
        s = S.displace(S.lattice(kind, reps, 3.56 if kind == "fcc" else 2.86), rng, 0.1)
        s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        structs.append(s)
        nbs.append(O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, 5.0))
    assert max(s.n for s in structs) > 1000
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, 5.0)
    ec, fc, sc = ctx.efs_components()
    for c, nb in enumerate(nbs):
        eo, fo, so = O.efs_components(m, nb)
        assert rel_err(ec[c], eo) < 1e-10
        assert rel_err(fc[off[c]:off[c + 1]], fo) < 1e-10
        assert rel_err(sc[c], so) < 1e-10
    again = ctx.efs_components()
    monkeypatch.setenv("MTPX_LIN_TILE_ROWS", "0")
    rows = ctx.efs_components()
    rows2 = ctx.efs_components()
    for a, b, c, d in zip((ec, fc, sc), again, rows, rows2):
        assert np.array_equal(a, b) and np.array_equal(c, d)
        assert np.abs(a - c).max() <= 1e-13 * np.abs(a).max()


def test_gram_of_the_device_rows(ctx, crystal_set):
    """The matrix-core Gram equals the textbook sum over the returned rows."""
    text, structs, nbs, labels = crystal_set
    _upload(ctx, text, structs, labels, SETTINGS["per-atom"])
    A, y = ctx.linear_rows()
    G, b = ctx.linear_system()
    Gt, bt = O.gram(A, y)
    assert rel_err(G, Gt) < 1e-12 and rel_err(b, bt) < 1e-12


@pytest.mark.parametrize("name", ["shapeev-20.mtp", "pot4b.mtp"])
def test_gram_of_wide_systems(ctx, name):
    """Wider normal equations (p = 290 and 758: several tile groups and
    shorter LDS row blocks) against the oracle's assembly and the textbook
    sum of the device's own rows."""
    rng = S.rng_for(91)
    if name == "pot4b.mtp":
        text = S.read_template(name)
    else:
        text = S.random_model(name, 2, 8, 1.9, 5.0, -0.1, 0.1, rng)
    m = O.Model(text)
    structs, nbs, labels = [], [], []
    for k in range(2):
        s = S.displace(S.lattice("bcc", (2, 2, 2 + k), 2.87), rng, 0.1)
        s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, m.cutoff)
        E, F, St, _ = O.efs(m, nb)
        e, f, st = S.noisy_labels(rng, s.n, E, F, St)
        structs.append(s)
        nbs.append(nb)
        labels.append(O.Labels(s.n, energy=e, forces=f, stress=st))
    st = SETTINGS["linear"]
    _upload(ctx, text, structs, labels, st, cutoff=m.cutoff)
    G, b = ctx.linear_system()
    assert G.shape == (m.Z + m.S, m.Z + m.S)
    A, y = ctx.linear_rows()
    Gt, bt = O.gram(A, y)
    assert rel_err(G, Gt) < 1e-12 and rel_err(b, bt) < 1e-12
    Go, bo = O.linear_system_batch(m, nbs, labels, st, threads=8)
    assert rel_err(G, Go) < 1e-10 and rel_err(b, bo) < 1e-10


def test_fixed_species_coefficients(ctx, crystal_set):
    """fix_species_coeffs: rows without the species columns and energy
    targets less the species part, against the oracle; the rows follow a
    change of the species coefficients; switching back restores p = Z + S."""
    text, structs, nbs, labels = crystal_set
    st = SETTINGS["per-atom"]
    _upload(ctx, text, structs, labels, st)
    m = O.Model(text)
    try:
        ctx.set_fix_species_coeffs(True)
        A, y = ctx.linear_rows()
        Ao = np.concatenate([O.linear_rows(m, nb, st, lb, fix_species=True)[0]
                             for nb, lb in zip(nbs, labels)])
        yo = np.concatenate([O.linear_rows(m, nb, st, lb, fix_species=True)[1]
                             for nb, lb in zip(nbs, labels)])
        assert A.shape == (Ao.shape[0], m.S)
        assert rel_err(A, Ao) < 1e-10 and rel_err(y, yo) < 1e-10
        G, b = ctx.linear_system()
        Go, bo = O.linear_system_batch(m, nbs, labels, st, threads=8, fix_species=True)
        assert rel_err(G, Go) < 1e-10 and rel_err(b, bo) < 1e-10
        # new species coefficients: new energy targets, same matrix
        c = ctx.get_coeffs()
        c[m.nradial:m.nradial + m.Z] += np.array([0.3, -0.2])
        ctx.set_coeffs(c)
        m.coeffs = c
        G2, b2 = ctx.linear_system()
        Go2, bo2 = O.linear_system_batch(m, nbs, labels, st, threads=8, fix_species=True)
        assert rel_err(b2, bo2) < 1e-10 and rel_err(G2, G) < 1e-12
        assert rel_err(b2, b) > 1e-6
    finally:
        ctx.set_fix_species_coeffs(False)
    G, b = ctx.linear_system()
    assert G.shape == (m.Z + m.S, m.Z + m.S)


def test_orthogonalize_matches_oracle(ctx):
    text, _ = S.training_models(4)
    m = O.Model(text)
    ctx.load_model_text(text)
    ctx.orthogonalize()
    m.orthogonalize()
    assert rel_err(ctx.get_coeffs(), m.coeffs) < 1e-14


def test_linear_after_orthogonalize(ctx, crystal_set):
    """The TrainLinearFast order: orthogonalise, then assemble."""
    text, structs, nbs, labels = crystal_set
    st = SETTINGS["linear"]
    _upload(ctx, text, structs, labels, st)
    ctx.orthogonalize()
    m = O.Model(text)
    m.orthogonalize()
    G, b = ctx.linear_system()
    Go, bo = O.linear_system_batch(m, nbs, labels, st, threads=8)
    assert rel_err(G, Go) < 1e-10 and rel_err(b, bo) < 1e-10


def test_level10_and_runtime_profile_models(ctx):
    """Level-10 and level-20 (compile-time profiles; the level-20 site kernel
    lives in the second object of lin_kernel.hip) and a model on the runtime
    profile."""
    rng = S.rng_for(77)
    for name, R in [("shapeev-10.mtp", 8), ("shapeev-20.mtp", 10), ("shapeev-16.mtp", 6)]:
        text = S.random_model(name, 2, R, 1.9, 5.0, -0.1, 0.1, rng)
        m = O.Model(text)
        s = S.displace(S.lattice("fcc", (3, 3, 3), 3.56), rng, 0.1)
        s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, 5.0)
        ctx.load_model_text(text)
        ctx.set_structures([s], 5.0)
        ec, fc, sc = ctx.efs_components()
        eo, fo, so = O.efs_components(m, nb)
        assert rel_err(ec[0], eo) < 1e-10 and rel_err(fc, fo) < 1e-10
        assert rel_err(sc[0], so) < 1e-10


def test_components_with_repeated_atoms(ctx):
    """Cells narrower than twice the cutoff put several images of one atom in
    a list, so lanes of one batch add to the same tile row.  Small and large
    cells in one batch, the level-16 model (the compiled walk), against the
    oracle."""
    text, _ = S.training_models(4)
    m = O.Model(text)
    rng = S.rng_for(91)
    structs = []
    for reps, a in [((2, 2, 2), 3.56), ((1, 1, 2), 3.56), ((3, 3, 3), 3.6), ((1, 1, 1), 3.5)]:
        s = S.displace(S.lattice("fcc", reps, a), rng, 0.1)
        s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        structs.append(s)
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, 5.0)
    ec, fc, sc = ctx.efs_components()
    repeats = 0
    for c, s in enumerate(structs):
        nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, m.cutoff)
        for i in range(nb.n):
            row = nb.idx[nb.offsets[i]:nb.offsets[i + 1]]
            repeats += len(row) - len(set(row.tolist()))
        eo, fo, so = O.efs_components(m, nb)
        assert rel_err(ec[c], eo) < 1e-10
        assert rel_err(fc[off[c]:off[c + 1]], fo) < 1e-10
        assert rel_err(sc[c], so) < 1e-10
    assert repeats > 0  # the small cells do repeat atoms within a list
    # lanes adding to one row in one instruction are applied in a fixed order
    again = ctx.efs_components()
    for x, y in zip((ec, fc, sc), again):
        assert np.array_equal(x.view(np.uint64), y.view(np.uint64))


def test_components_with_isolated_atoms(ctx):
    """Atoms with empty neighbour lists in the middle of a structure (a slab
    with atoms out in its vacuum): the sites after them keep their own
    entries.  Level-16 model (the compiled walk), against the oracle."""
    text, _ = S.training_models(4)
    m = O.Model(text)
    rng = S.rng_for(93)
    slab = S.displace(S.lattice("fcc", (2, 2, 2), 3.56), rng, 0.05)
    cell = slab.cell.copy()
    cell[2, 2] = 30.0
    far = np.array([[1.0, 2.0, 15.0], [3.0, 1.0, 22.5]])
    pos = np.concatenate([slab.pos[:10], far[:1], slab.pos[10:21], far[1:], slab.pos[21:]])
    s = S.Structure(cell, pos, (S.uniform(rng, len(pos)) * 2).astype(np.int32),
                    np.ones(3, np.int32))
    s.pos = O.wrap(s.cell, s.pbc, s.pos)
    big = S.displace(S.lattice("fcc", (3, 3, 3), 3.6), rng, 0.1)
    big.types = (S.uniform(rng, big.n) * 2).astype(np.int32)
    big.pos = O.wrap(big.cell, big.pbc, big.pos)
    structs = [s, big]
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, 5.0)
    ec, fc, sc = ctx.efs_components()
    empty = 0
    for c, st in enumerate(structs):
        nb = O.Neighbors.build(st.cell, st.pbc, st.pos, st.types, m.cutoff)
        empty += int(np.sum(np.diff(nb.offsets) == 0))
        eo, fo, so = O.efs_components(m, nb)
        assert rel_err(ec[c], eo) < 1e-10
        assert rel_err(fc[off[c]:off[c + 1]], fo) < 1e-10
        assert rel_err(sc[c], so) < 1e-10
    assert empty == 2


def test_empty_batch_linear_system(ctx):
    text, _ = S.training_models(4)
    ctx.load_model_text(text)
    ctx.set_structures([], 5.0)
    ctx.set_labels(np.zeros((0, 3), np.int32))
    G, b = ctx.linear_system()
    assert not G.any() and not b.any()


def test_orthogonalize_known_answer(ctx):
    """mtpx_orthogonalize on the hand-worked three-channel case (see
    test_oracle_math.ORTHO_MTP): the reference's projection by the norm of
    the channel being projected, not textbook Gram-Schmidt."""
    from test_oracle_math import ORTHO_EXPECTED, ORTHO_MTP
    ctx.load_model_text(ORTHO_MTP)
    ctx.orthogonalize()
    got = ctx.get_coeffs()[:6].reshape(3, 2)
    assert np.abs(got - ORTHO_EXPECTED).max() < 1e-9


def test_duplicate_scalar_mapping_rows(ctx):
    """Duplicate mapping entries give identical design columns."""
    text = S.random_model("dup-scalar.mtp", 2, 6, 1.8, 4.6, -0.5, 0.5, S.rng_for(700))
    m = O.Model(text)
    rng = S.rng_for(704)
    s = S.displace(S.strain(S.lattice("bcc", (2, 2, 3), 2.87), rng, 0.03), rng, 0.15)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    s.pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, m.cutoff)
    ctx.load_model_text(text)
    ctx.set_structures([s], m.cutoff)
    ec, fc, sc = ctx.efs_components()
    eo, fo, so = O.efs_components(m, nb)
    assert rel_err(ec[0], eo) < 1e-10 and rel_err(fc, fo) < 1e-10 and rel_err(sc[0], so) < 1e-10
    assert np.array_equal(fc[..., m.Z + 1], fc[..., m.Z + 4])
