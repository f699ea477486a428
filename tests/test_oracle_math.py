"""Pin the oracle with what the mathematics fixes: closed forms, finite
differences, invariances and linearity.  Each check is chosen so that a
plausible slip (a dropped term, a sign, a swapped index, a transposed
operand) fails it."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import synth as S


def _efs_of(model, s, pos=None):
    pos = O.wrap(s.cell, s.pbc, s.pos if pos is None else pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, model.cutoff)
    return O.efs(model, nb)


# ---------------------------------------------------------------- radial --

def test_chebyshev_closed_form_and_derivative():
    """RBChebyshev: Q_k(r) = s (r - r_c)^2 T_k(xi), T_k = cos(k acos xi)."""
    m = O.Model(S.random_model("shapeev-16.mtp", 1, 10, 1.9, 5.0, -1, 1, S.rng_for(7)))
    for r in np.linspace(1.95, 4.99, 23):
        v, d = m.rb_calc_der(r)
        xi = (2 * r - (1.9 + 5.0)) / (5.0 - 1.9)
        T = np.cos(np.arange(10) * np.arccos(xi))
        assert np.allclose(v, 0.01 * (r - 5.0) ** 2 * T, rtol=1e-12, atol=1e-15)
        h = 1e-6
        fd = (m.rb_calc_der(r + h)[0] - m.rb_calc_der(r - h)[0]) / (2 * h)
        assert np.allclose(d, fd, rtol=1e-7, atol=1e-10)


# ---------------------------------------------------- closed-form energy --

TWO_MOMENT = """MTP
version = 1.1.0
potential_name = MTP1m
scaling = 1.0e-2
species_count = 1
radial_basis_type = RBChebyshev
\tmin_dist = 2.0
\tmax_dist = 5.0
\tradial_basis_size = 3
radial_funcs_count = 1
radial_coeffs
\t0-0
\t\t{0.7, -0.3, 0.2}
alpha_moments_count = 3
alpha_index_basic_count = 2
alpha_index_basic = {{0, 0, 0, 0}, {0, 1, 0, 0}}
alpha_index_times_count = 1
alpha_index_times = {{1, 1, 1, 2}}
alpha_scalar_moments = 2
alpha_moment_mapping = {0, 2}
species_coeffs = {-1.25}
moment_coeffs = {0.4, 2.5}
"""


def test_two_moment_closed_form():
    """E = sum_i [eps + xi0 sum_j f(r_ij) + xi1 (sum_j f(r_ij) x_ij / r_ij)^2]
    (the closed form of unitest/ut_mtp_cuda.cpp:110-133)."""
    m = O.Model(TWO_MOMENT)
    rng = S.rng_for(8)
    s = S.displace(S.lattice("fcc", (2, 2, 2), 3.9), rng, 0.2)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, 5.0)
    E, F, St, se = O.efs(m, nb)
    c = np.array([0.7, -0.3, 0.2])
    Eref = 0.0
    for i in range(nb.n):
        sl = slice(nb.offsets[i], nb.offsets[i + 1])
        r = nb.dist[sl]
        xi = (2 * r - 7.0) / 3.0
        T = np.stack([np.ones_like(xi), xi, 2 * xi * xi - 1])
        f = 0.01 * (r - 5.0) ** 2 * (c @ T)
        Eref += -1.25 + 0.4 * f.sum() + 2.5 * (np.sum(f * nb.vec[sl, 0] / r)) ** 2
    assert rel_err(E, Eref) < 1e-13


# ------------------------------------------------------ forces, virial --

@pytest.fixture(scope="module")
def small_case():
    text, s = S.scaled_inference(2, (2, 2, 2))
    s = S.displace(s, S.rng_for(9), 0.05)
    return O.Model(text), s


def test_forces_are_minus_energy_gradient(small_case):
    m, s = small_case
    E, F, St, se = _efs_of(m, s)
    h = 1e-5
    rng = np.random.default_rng(0)
    for i in rng.choice(s.n, 6, replace=False):
        for a in range(3):
            p1 = s.pos.copy()
            p1[i, a] += h
            p2 = s.pos.copy()
            p2[i, a] -= h
            fd = -(_efs_of(m, s, p1)[0] - _efs_of(m, s, p2)[0]) / (2 * h)
            assert abs(F[i, a] - fd) < 1e-7 * max(1.0, np.abs(F).max())


def test_net_force_vanishes_and_site_energies_sum(small_case):
    m, s = small_case
    E, F, St, se = _efs_of(m, s)
    assert np.abs(F.sum(axis=0)).max() < 1e-12 * np.abs(F).max() * s.n
    assert abs(E - se.sum()) < 1e-12 * np.abs(se).sum()


def test_virial_is_strain_derivative(small_case):
    """S_ab = -dE/d eps_ba under cell' = cell (I + eps), x' = x (I + eps)."""
    m, s = small_case
    E, F, St, se = _efs_of(m, s)
    h = 1e-6
    for a in range(3):
        for b in range(3):
            eps = np.zeros((3, 3))
            eps[a, b] = h
            Fp = np.eye(3) + eps
            Fm = np.eye(3) - eps
            sp = S.Structure(s.cell @ Fp, s.pos @ Fp, s.types, s.pbc)
            sm = S.Structure(s.cell @ Fm, s.pos @ Fm, s.types, s.pbc)
            dE = (_efs_of(m, sp)[0] - _efs_of(m, sm)[0]) / (2 * h)
            assert abs(St[b, a] + dE) < 1e-6 * max(1.0, np.abs(St).max())
    assert np.abs(St - St.T).max() < 1e-10 * np.abs(St).max()


def test_rotation_invariance(small_case):
    m, s = small_case
    E, F, St, se = _efs_of(m, s)
    th = 0.7
    R = np.array([[np.cos(th), -np.sin(th), 0], [np.sin(th), np.cos(th), 0], [0, 0, 1]])
    R = R @ np.array([[1, 0, 0], [0, np.cos(0.4), -np.sin(0.4)], [0, np.sin(0.4), np.cos(0.4)]])
    sr = S.Structure(s.cell @ R.T, O.wrap(s.cell, s.pbc, s.pos) @ R.T, s.types, s.pbc)
    Er, Fr, Sr, _ = _efs_of(m, sr)
    assert rel_err(Er, E) < 1e-12
    assert rel_err(Fr, F @ R.T) < 1e-10
    assert rel_err(Sr, R @ St @ R.T) < 1e-10


def test_atom_permutation_invariance(small_case):
    m, s = small_case
    E, F, St, se = _efs_of(m, s)
    perm = np.random.default_rng(1).permutation(s.n)
    sp = S.Structure(s.cell, s.pos[perm], s.types[perm], s.pbc)
    Ep, Fp, Sp, sep = _efs_of(m, sp)
    assert rel_err(Ep, E) < 1e-12
    assert rel_err(Fp, F[perm]) < 1e-11
    assert rel_err(sep, se[perm]) < 1e-12


# -------------------------------------------------------------- training --

def _config(wid=4):
    ref_text, start_text = S.training_models(4)
    s = S.training_structures(4, 1)[0]
    s = S.Structure(s.cell, s.pos, s.types, s.pbc)
    mref = O.Model(ref_text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, mref.cutoff)
    E, F, St, _ = O.efs(mref, nb)
    e, f, st = S.noisy_labels(S.rng_for(wid, 3), s.n, E, F, St)
    return O.Model(start_text), nb, O.Labels(s.n, e, f, st)


@pytest.mark.parametrize("weights", [(1.0, 0.01, 1e-3), (1.0, 0.0, 0.0), (0.0, 0.05, 0.0),
                                     (0.0, 0.0, 0.1)])
def test_loss_gradient_matches_coefficient_fd(weights):
    """AddLossGard's gradient against central differences of its loss in every
    coefficient class (radial, species, moment)."""
    m, nb, lab = _config()
    st = O.LossSettings.make(weight_eng=weights[0], weight_force=weights[1],
                             weight_stress=weights[2])
    x0 = m.coeffs
    loss, g, _ = O.add_loss_grad(m, nb, st, lab)
    rng = np.random.default_rng(2)
    idx = np.concatenate([rng.choice(m.nradial, 12, replace=False),
                          m.nradial + np.arange(m.Z),
                          m.nradial + m.Z + rng.choice(m.S, 10, replace=False)])
    for k in idx:
        h = 1e-6 * max(1.0, abs(x0[k]))
        xp = x0.copy()
        xp[k] += h
        m.coeffs = xp
        lp = O.add_loss_grad(m, nb, st, lab)[0]
        xm = x0.copy()
        xm[k] -= h
        m.coeffs = xm
        lm = O.add_loss_grad(m, nb, st, lab)[0]
        m.coeffs = x0
        fd = (lp - lm) / (2 * h)
        assert abs(g[k] - fd) < 2e-6 * max(abs(fd), 1e-3 * np.abs(g).max()), (k, g[k], fd)


def test_loss_closed_form():
    """L = W_F sum |dF|^2 + W_S sum dS_ab^2 + W_E dE^2 with W_X = w_X / N^p_X."""
    m, nb, lab = _config()
    st = O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=1e-3)
    loss, g, met = O.add_loss_grad(m, nb, st, lab)
    E, F, St, _ = O.efs(m, nb)
    n = lab.n
    ref = (0.01 * np.sum((F - lab.forces) ** 2) + 1e-3 / n * np.sum((St - lab.stress) ** 2)
           + 1.0 / n * (E - lab.energy) ** 2)
    assert rel_err(loss, ref) < 1e-12
    assert rel_err(met[:3].sum(), loss) < 1e-12


def test_penalty_gradient_fd():
    m, nb, lab = _config()
    x0 = m.coeffs.copy()
    x0[: m.nradial] *= 3.0  # away from the unit-norm minimum
    m.coeffs = x0
    p, g = O.penalty_grad(m, 1e-3, 1e-4, 0.0)
    for k in list(range(0, m.nradial, 7)) + list(range(m.nradial + m.Z, m.ncoef, 9)):
        h = 1e-6
        xp = x0.copy()
        xp[k] += h
        m.coeffs = xp
        pp = O.penalty_grad(m, 1e-3, 1e-4, 0.0)[0]
        xm = x0.copy()
        xm[k] -= h
        m.coeffs = xm
        pm = O.penalty_grad(m, 1e-3, 1e-4, 0.0)[0]
        m.coeffs = x0
        assert abs(g[k] - (pp - pm) / (2 * h)) < 1e-6 * max(1e-6, abs(g[k]))


def test_batch_loss_is_mean_plus_penalty():
    m, nb, lab = _config()
    st = O.LossSettings.make()
    f, g = O.loss_grad_batch(m, [nb, nb], [lab, lab], st, penalty_weight=1e-6, reg_l2=1e-10,
                             threads=2)
    l1, g1, _ = O.add_loss_grad(m, nb, st, lab)
    p, pg = O.penalty_grad(m, 1e-6, 1e-10, 0.0)
    assert rel_err(f, l1 + p) < 1e-12
    assert rel_err(g, g1 + pg) < 1e-12


# ------------------------------------------------------------ linear fit --

def test_design_rows_reproduce_efs():
    """E, F, S are linear in [species | moment] coefficients: the rows of
    CalcEFSCmpt_R contracted with them give getEFS."""
    text, s = S.scaled_inference(2, (2, 2, 3))
    m = O.Model(text)
    pos = O.wrap(s.cell, s.pbc, s.pos)
    nb = O.Neighbors.build(s.cell, s.pbc, pos, s.types, m.cutoff)
    E, F, St, _ = O.efs(m, nb)
    ec, fc, sc = O.efs_components(m, nb)
    lin = m.coeffs[m.nradial:]
    assert rel_err(ec @ lin, E) < 1e-12
    assert rel_err(fc @ lin, F) < 1e-11
    assert rel_err(sc @ lin, St) < 1e-11
    assert np.allclose(ec[: m.Z], np.bincount(s.types, minlength=m.Z))


def test_linear_rows_weights_and_gram():
    m, nb, lab = _config()
    st = O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=1e-3)
    A, y = O.linear_rows(m, nb, st, lab)
    n = lab.n
    assert A.shape == (3 * n + 9 + 1, m.Z + m.S)
    lin = m.coeffs[m.nradial:]
    E, F, St, _ = O.efs(m, nb)
    pred = A @ lin
    w = np.concatenate([np.full(3 * n, np.sqrt(0.01)), np.full(9, np.sqrt(1e-3 / n)),
                        [np.sqrt(1.0 / n)]])
    assert rel_err(pred, w * np.concatenate([F.ravel(), St.ravel(), [E]])) < 1e-11
    assert rel_err(y, w * np.concatenate([lab.forces.ravel(), lab.stress.ravel(),
                                          [lab.energy]])) < 1e-14
    G, b = O.gram(A, y)
    assert rel_err(G, A.T @ A) < 1e-13 and rel_err(b, A.T @ y) < 1e-13
    # the least-squares residual of the Gram system is the loss with those weights
    Gb, bb = O.linear_system_batch(m, [nb], [lab], st, threads=1)
    assert rel_err(Gb, G) < 1e-15 and rel_err(bb, b) < 1e-15
    loss = O.add_loss_grad(m, nb, st, lab)[0]
    assert rel_err(lin @ G @ lin - 2 * lin @ b + y @ y, loss) < 1e-8


def test_orthogonalize_normalises_first_channel():
    """Orthogonalize (potential_mtp.cpp:3849-3930): channel 0 is divided by
    sqrt(sum c^2 + 1e-10 per term); later channels are projected with the norm
    of the channel being projected (the reference's formula)."""
    text, _ = S.scaled_inference(2, (2, 2, 2))
    m = O.Model(text)
    c = m.coeffs
    M, R, Z = m.M, m.R, m.Z
    rad = c[: m.nradial].reshape(Z * Z, M, R)
    m.orthogonalize()
    out = m.coeffs[: m.nradial].reshape(Z * Z, M, R)
    c0 = rad[:, 0, :]
    assert np.allclose(out[:, 0, :], c0 / np.sqrt(np.sum(c0 ** 2) + 1e-10 * c0.size), rtol=1e-13)
    for k in range(M):
        assert abs(np.sum(out[:, k, :] ** 2) - 1) < 1e-6
    assert np.array_equal(m.coeffs[m.nradial:], c[m.nradial:])
