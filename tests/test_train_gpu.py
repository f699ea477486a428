"""Training path on the device against the oracle's restatement of
Trainer_MTP::AddLossGard / AccumulateGard and PotMTP's gradient
(train/train_mtp.cpp:3039-3094, 3839-3996; potentials/potential_mtp.cpp:
3348-3550, 6568-6742, 6896-6923).

Tolerances: E/F/S 1e-10 relative, loss and gradient 1e-9 relative (largest
absolute difference over the largest magnitude)."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from mtpx import synth as S

pytestmark = pytest.mark.gpu


def _dataset(wid, count, seed, drop=False):
    """Structures, oracle lists, labels (reference model + noise)."""
    ref_text, start_text = S.training_models(wid)
    cutoff = 5.0 if wid == 4 else 6.0
    mref = O.Model(ref_text)
    rng = S.rng_for(700 + seed)
    structs, nbs, labels = [], [], []
    for k, s in enumerate(S.training_structures(wid, count)):
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, cutoff)
        E, F, St, _ = O.efs(mref, nb)
        e, f, st = S.noisy_labels(rng, s.n, E, F, St)
        lb = O.Labels(s.n, energy=e, forces=f, stress=st)
        if drop:  # vary which labels each structure carries
            if k % 4 == 1:
                lb.forces = None
            if k % 4 == 2:
                lb.stress = None
            if k % 4 == 3:
                lb.energy = None
                lb.fitness = 0.5
            if k % 3 == 0:
                lb.atomic_fitness = 0.5 + rng.random(s.n)
        structs.append(s)
        nbs.append(nb)
        labels.append(lb)
    return start_text, cutoff, structs, nbs, labels


def _upload(ctx, text, cutoff, structs, labels, settings):
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, cutoff)
    nc = len(structs)
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


SETTINGS = {
    "default": O.LossSettings.make(),
    "per-atom": O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=0.001,
                                    eng_pow=2.0, force_pow=1.0, stress_pow=0.0),
    "force-norm": O.LossSettings.make(force_norm_f=1.0, force_norm_p=1.5, force_norm_d=0.1),
}


@pytest.fixture(scope="module")
def lvl16_set():
    return _dataset(4, 6, 1, drop=True)


@pytest.fixture(scope="module")
def lvl20_set():
    return _dataset(5, 3, 2)


def test_compute_batch_matches_oracle(ctx, lvl16_set):
    text, cutoff, structs, nbs, labels = lvl16_set
    m = O.Model(text)
    off = _upload(ctx, text, cutoff, structs, labels, SETTINGS["default"])
    E, F, St, se = ctx.compute_batch()
    for c, nb in enumerate(nbs):
        Eo, Fo, So, seo = O.efs(m, nb)
        assert rel_err(E[c], Eo) < 1e-10
        assert rel_err(F[off[c]:off[c + 1]], Fo) < 1e-10
        assert rel_err(St[c], So) < 1e-10
        assert rel_err(se[off[c]:off[c + 1]], seo) < 1e-10


@pytest.mark.parametrize("name", list(SETTINGS))
def test_loss_grad_matches_oracle_lvl16(ctx, lvl16_set, name):
    text, cutoff, structs, nbs, labels = lvl16_set
    st = SETTINGS[name]
    _upload(ctx, text, cutoff, structs, labels, st)
    m = O.Model(text)
    f_o, g_o = O.loss_grad_batch(m, nbs, labels, st, penalty_weight=1e-3, reg_l2=1e-4,
                                 reg_l1=1e-5, threads=8)
    f, g, met = ctx.loss_grad(penalty_weight=1e-3, reg_l2=1e-4, reg_l1=1e-5)
    assert rel_err(f, f_o) < 1e-9
    assert rel_err(g, g_o) < 1e-9
    # metrics against the per-structure oracle
    mo = np.zeros(6)
    for nb, lb in zip(nbs, labels):
        _, _, mt = O.add_loss_grad(m, nb, st, lb)
        mo += mt
    assert rel_err(met[1:4], mo[0:3]) < 1e-9
    assert rel_err(met[4:7], mo[3:6]) < 1e-9
    assert abs(met[0] - mo[0:3].sum()) <= 1e-9 * abs(mo[0:3].sum())


def test_loss_grad_matches_oracle_lvl20_liquid(ctx, lvl20_set):
    text, cutoff, structs, nbs, labels = lvl20_set
    st = SETTINGS["default"]
    _upload(ctx, text, cutoff, structs, labels, st)
    m = O.Model(text)
    f_o, g_o = O.loss_grad_batch(m, nbs, labels, st, penalty_weight=1e-6, reg_l2=1e-10,
                                 threads=8)
    f, g, _ = ctx.loss_grad(penalty_weight=1e-6, reg_l2=1e-10)
    assert rel_err(f, f_o) < 1e-9
    assert rel_err(g, g_o) < 1e-9
    # every coefficient block is exercised
    nr = m.Z * m.Z * m.M * m.R
    for blk in (g[:nr], g[nr:nr + m.Z], g[nr + m.Z:]):
        assert np.abs(blk).max() > 0


def test_isolated_atoms_in_a_batch(ctx):
    """A slab with two atoms out in its vacuum (empty neighbour lists in the
    middle of a structure) beside a crystal: E/F/S and the loss gradient
    against the oracle."""
    ref_text, start_text = S.training_models(4)
    mref = O.Model(ref_text)
    rng = S.rng_for(95)
    slab = S.displace(S.lattice("fcc", (2, 2, 2), 3.56), rng, 0.05)
    cell = slab.cell.copy()
    cell[2, 2] = 30.0
    far = np.array([[1.0, 2.0, 15.0], [3.0, 1.0, 22.5]])
    pos = np.concatenate([slab.pos[:10], far[:1], slab.pos[10:21], far[1:], slab.pos[21:]])
    s = S.Structure(cell, pos, (S.uniform(rng, len(pos)) * 2).astype(np.int32),
                    np.ones(3, np.int32))
    big = S.displace(S.lattice("fcc", (3, 3, 3), 3.6), rng, 0.1)
    big.types = (S.uniform(rng, big.n) * 2).astype(np.int32)
    structs, nbs, labels = [], [], []
    for st in (s, big):
        st.pos = O.wrap(st.cell, st.pbc, st.pos)
        nb = O.Neighbors.build(st.cell, st.pbc, st.pos, st.types, 5.0)
        E, F, St, _ = O.efs(mref, nb)
        e, f, sv = S.noisy_labels(rng, st.n, E, F, St)
        structs.append(st)
        nbs.append(nb)
        labels.append(O.Labels(st.n, energy=e, forces=f, stress=sv))
    assert sum(int(np.sum(np.diff(nb.offsets) == 0)) for nb in nbs) == 2
    settings = SETTINGS["default"]
    off = _upload(ctx, start_text, 5.0, structs, labels, settings)
    m = O.Model(start_text)
    E, F, St, se = ctx.compute_batch()
    for c, nb in enumerate(nbs):
        Eo, Fo, So, seo = O.efs(m, nb)
        assert rel_err(E[c], Eo) < 1e-10
        assert rel_err(F[off[c]:off[c + 1]], Fo) < 1e-10
        assert rel_err(St[c], So) < 1e-10
    f_o, g_o = O.loss_grad_batch(m, nbs, labels, settings, penalty_weight=1e-3, reg_l2=1e-4,
                                 threads=8)
    f, g, _ = ctx.loss_grad(penalty_weight=1e-3, reg_l2=1e-4)
    assert rel_err(f, f_o) < 1e-9
    assert rel_err(g, g_o) < 1e-9


def test_gradient_of_explicit_adjoints(ctx, lvl16_set):
    """AccumulateEFSCombinationGard with arbitrary adjoints, summed over
    structures, accumulating into a given vector."""
    text, cutoff, structs, nbs, labels = lvl16_set
    off = _upload(ctx, text, cutoff, structs, labels, SETTINGS["default"])
    m = O.Model(text)
    rng = S.rng_for(811)
    nc, N = len(structs), int(off[-1])
    dE = rng.random(nc) - 0.5
    dF = rng.random((N, 3)) - 0.5
    dS = rng.random((nc, 3, 3)) - 0.5
    g_o = np.zeros(m.ncoef)
    for c, nb in enumerate(nbs):
        O.accumulate_efs_combination_grad(m, nb, dE[c], dF[off[c]:off[c + 1]], dS[c], g_o)
    base = rng.random(m.ncoef)
    g = ctx.accumulate_gradient(dE, dF, dS, gradient=base)
    assert rel_err(g - base, g_o) < 1e-9


def test_energy_only_gradient(ctx, lvl16_set):
    """Zero force and stress adjoints: the AccumulateFPGard(se_weight) path."""
    text, cutoff, structs, nbs, labels = lvl16_set
    off = _upload(ctx, text, cutoff, structs, labels, SETTINGS["default"])
    m = O.Model(text)
    dE = np.linspace(0.3, 1.1, len(structs))
    g_o = np.zeros(m.ncoef)
    for c, nb in enumerate(nbs):
        for i in range(nb.n):
            O.accumulate_fp_grad(m, nb, i, dE[c], None, g_o)
    g = ctx.accumulate_gradient(dE, None, None)
    assert rel_err(g, g_o) < 1e-9


def test_prepare_loss_then_gradient(ctx, lvl16_set):
    """compute_batch + prepare_loss + accumulate_gradient equal loss_grad
    without the mean and penalty."""
    text, cutoff, structs, nbs, labels = lvl16_set
    _upload(ctx, text, cutoff, structs, labels, SETTINGS["per-atom"])
    # deterministic forces: the two evaluations see bitwise the same E/F/S
    ctx.compute_batch(deterministic=True)
    met = ctx.prepare_loss()
    g = ctx.accumulate_gradient()
    f2, g2, met2 = ctx.loss_grad(deterministic=True)
    nc = len(structs)
    assert met[0] / nc == pytest.approx(f2, rel=1e-14)
    assert np.array_equal(met, met2)
    assert rel_err(g / nc, g2) < 1e-14


def test_gradient_is_bitwise_repeatable(ctx, lvl16_set):
    text, cutoff, structs, nbs, labels = lvl16_set
    _upload(ctx, text, cutoff, structs, labels, SETTINGS["default"])
    a = ctx.loss_grad(deterministic=True)
    b = ctx.loss_grad(deterministic=True)
    assert a[0] == b[0] and np.array_equal(a[1], b[1])


def test_penalty_matches_oracle(ctx):
    text, _ = S.training_models(5)
    m = O.Model(text)
    ctx.load_model_text(text)
    for w, l2, l1 in [(1e-3, 0.0, 0.0), (0.0, 1e-2, 0.0), (0.0, 0.0, 1e-3), (1e-6, 1e-10, 1e-7)]:
        lo, go = O.penalty_grad(m, w, l2, l1)
        lg, gg = ctx.penalty(w, l2, l1)
        assert rel_err(lg, lo) < 1e-12 and rel_err(gg, go) < 1e-12


def test_coefficient_update_between_iterations(ctx, lvl16_set):
    """An L-BFGS step changes the coefficients: the next loss_grad uses them."""
    text, cutoff, structs, nbs, labels = lvl16_set
    st = SETTINGS["default"]
    _upload(ctx, text, cutoff, structs, labels, st)
    m = O.Model(text)
    f0, g0, _ = ctx.loss_grad()
    x = ctx.get_coeffs() - 1e-3 * g0 / np.abs(g0).max()
    ctx.set_coeffs(x)
    m.coeffs = x
    f1, g1, _ = ctx.loss_grad()
    f_o, g_o = O.loss_grad_batch(m, nbs, labels, st, penalty_weight=0.0, reg_l2=0.0, threads=8)
    assert f1 != f0
    assert rel_err(f1, f_o) < 1e-9 and rel_err(g1, g_o) < 1e-9


def test_empty_batch_and_empty_structure(ctx):
    text, _ = S.training_models(4)
    ctx.load_model_text(text)
    ctx.set_structures([], 5.0)
    ctx.set_labels(np.zeros((0, 3), np.int32))
    f, g, met = ctx.loss_grad()
    assert f == 0.0 and not g.any() and not met.any()
    # a structure without atoms between two others
    s = S.displace(S.lattice("fcc", (2, 2, 2), 3.56), S.rng_for(5), 0.1)
    empty = S.Structure(np.eye(3) * 10, np.zeros((0, 3)), np.zeros(0, np.int32),
                        np.ones(3, np.int32))
    off = ctx.set_structures([s, empty, s], 5.0)
    assert off.tolist() == [0, 32, 32, 64]
    E, F, St, _ = ctx.compute_batch()
    assert E[1] == 0.0 and not St[1].any()
    assert E[0] == pytest.approx(E[2], rel=1e-14)


def test_loss_grad_duplicate_scalar_mapping(ctx):
    """A repeated alpha_moment_mapping entry: both scalars count in the
    energy and in the adjoint seed, and each gets its own gradient entry."""
    text = S.random_model("dup-scalar.mtp", 2, 6, 1.8, 4.6, -0.5, 0.5, S.rng_for(700))
    ref = S.random_model("dup-scalar.mtp", 2, 6, 1.8, 4.6, -0.5, 0.5, S.rng_for(702))
    m, mref = O.Model(text), O.Model(ref)
    rng = S.rng_for(703)
    structs, nbs, labels = [], [], []
    for k in range(4):
        s = S.displace(S.strain(S.lattice("bcc", (2, 2, 2 + k % 2), 2.87), rng, 0.03), rng, 0.15)
        s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, mref.cutoff)
        E, F, St, _ = O.efs(mref, nb)
        e, f, st = S.noisy_labels(rng, s.n, E, F, St)
        structs.append(s)
        nbs.append(nb)
        labels.append(O.Labels(s.n, energy=e, forces=f, stress=st))
    st = SETTINGS["default"]
    _upload(ctx, text, mref.cutoff, structs, labels, st)
    f_o, g_o = O.loss_grad_batch(m, nbs, labels, st, penalty_weight=1e-3, reg_l2=1e-4, threads=4)
    f, g, _ = ctx.loss_grad(penalty_weight=1e-3, reg_l2=1e-4)
    assert rel_err(f, f_o) < 1e-9
    assert rel_err(g, g_o) < 1e-9
    # the two scalars mapped to moment 4 see the same moment: equal energy
    # derivatives (dL/dE m_4 + q_4) up to the L2 term of their own coefficient
    base = m.nradial + m.Z
    x = m.coeffs
    assert abs((g[base + 1] - 2e-4 * x[base + 1]) - (g[base + 4] - 2e-4 * x[base + 4])) \
        < 1e-12 * np.abs(g).max()
