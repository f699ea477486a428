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


def test_linear_rows_with_fixed_species_coefficients():
    """fix_species_coeffs (train_mtp.cpp:1300-1302, 1381-1392): for any
    moment coefficients theta, the reduced rows give the same residuals as
    the full rows with the species coefficients held at the model's values,
    and the loss at the model's own coefficients is unchanged."""
    m, nb, lab = _config()
    st = O.LossSettings.make(weight_eng=1.0, weight_force=0.01, weight_stress=1e-3)
    A, y = O.linear_rows(m, nb, st, lab)
    Af, yf = O.linear_rows(m, nb, st, lab, fix_species=True)
    assert Af.shape == (A.shape[0], m.S)
    csp = m.coeffs[m.nradial:m.nradial + m.Z]
    assert np.abs(csp).max() > 0
    rng = np.random.default_rng(5)
    for theta in (m.coeffs[m.nradial + m.Z:], rng.standard_normal(m.S)):
        full = A @ np.concatenate([csp, theta]) - y
        red = Af @ theta - yf
        assert rel_err(red, full) < 1e-12
    # only the energy row's target moves, by sqrt(w) sum_s n_s c_s
    n_s = np.bincount(nb.center_types, minlength=m.Z)
    dy = y - yf
    assert np.abs(dy[:-1]).max() == 0.0
    assert rel_err(dy[-1], np.sqrt(1.0 / lab.n) * (n_s @ csp)) < 1e-13
    G, b = O.linear_system_batch(m, [nb], [lab], st, threads=1, fix_species=True)
    Gt, bt = O.gram(Af, yf)
    assert rel_err(G, Gt) < 1e-15 and rel_err(b, bt) < 1e-15


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


# A three-function, two-term radial basis whose Orthogonalize result was
# worked out by hand.  Channels c0 = (3, 4), c1 = (2, 0), c2 = (0, 5) (one
# species pair).  potential_mtp.cpp:3849-3930 projects channel k on an
# earlier channel k2 with scal / |c_k|^2 -- the squared norm of the channel
# being projected, recomputed before each projection -- not |c_k2|^2:
#   c0 -> (3, 4) / 5                                     = (0.6, 0.8)
#   c1: |c1|^2 = 4, scal = 2 * 0.6 = 1.2, c1 -= 0.3 c0    = (1.82, -0.24)
#       |c1|^2 = 3.37                                    -> c1 / sqrt(3.37)
#   c2: |c2|^2 = 25, scal = 5 * 0.8 = 4, c2 -= 0.16 c0    = (-0.096, 4.872)
#       |c2|^2 = 23.7456, scal = c2 . c1 = -1.344 / sqrt(3.37),
#       c2 -= c1 scal / 23.7456 = c2 - (1.82, -0.24) (-1.344) / (3.37 * 23.7456)
#          = (-0.0654326627833672, 4.86796914234506), |c2|^2 = 23.7014050041826
# The 1e-10 added per term to the final norms moves these by ~1e-10.
# Textbook Gram-Schmidt (divide by |c_k2|^2 = 1) gives c1 = (0.8, -0.6) and
# c2 = (0, 0) instead.
ORTHO_MTP = """MTP
version = 1.1.0
potential_name = MTP1m
scaling = 1.0
species_count = 1
potential_tag = 
radial_basis_type = RBChebyshev
\tmin_dist = 2.0
\tmax_dist = 5.0
\tradial_basis_size = 2
\tradial_funcs_count = 3
\tradial_coeffs
\t\t0-0
\t\t\t{3, 4}
\t\t\t{2, 0}
\t\t\t{0, 5}
alpha_moments_count = 3
alpha_index_basic_count = 3
alpha_index_basic = {{0, 0, 0, 0}, {1, 0, 0, 0}, {2, 0, 0, 0}}
alpha_index_times_count = 0
alpha_index_times = {}
alpha_scalar_moments = 3
alpha_moment_mapping = {0, 1, 2}
species_coeffs = {0.5}
moment_coeffs = {1, 2, 3}
"""
ORTHO_EXPECTED = np.array([[0.6, 0.8],
                           [0.9914171734791749, -0.1307363305686824],
                           [-0.013440256236068761, 0.9999096756769127]])
ORTHO_TEXTBOOK = np.array([[0.6, 0.8], [0.8, -0.6], [0.0, 0.0]])


def _textbook_gram_schmidt(c):
    """Classical Gram-Schmidt with unit-norm earlier channels (the planted
    alternative the known answer must reject)."""
    out = []
    for v in c:
        v = v.astype(float).copy()
        for u in out:
            v -= u * (v @ u) / (u @ u) if (u @ u) > 0 else 0.0
        nv = np.sqrt(v @ v + 1e-10 * v.size)
        out.append(v / nv)
    return np.array(out)


def test_orthogonalize_known_answer():
    m = O.Model(ORTHO_MTP)
    assert (m.Z, m.M, m.R) == (1, 3, 2)
    m.orthogonalize()
    got = m.coeffs[: m.nradial].reshape(3, 2)
    assert np.abs(got - ORTHO_EXPECTED).max() < 1e-9
    # the known answer rejects textbook Gram-Schmidt
    tb = _textbook_gram_schmidt(np.array([[3, 4], [2, 0], [0, 5]]))
    assert np.abs(tb - ORTHO_TEXTBOOK).max() < 1e-6
    assert np.abs(tb - ORTHO_EXPECTED).max() > 0.1


def test_orthogonalize_first_projection_closed_form():
    """After one projection c1' = c1 - c0 (c1.c0) / |c1|^2 with |c0| = 1, so
    c1'.c0 = s (1 - 1 / |c1|^2) with s = c1.c0: nonzero unless |c1| = 1
    (textbook Gram-Schmidt leaves 0)."""
    rng = S.rng_for(31)
    for trial in range(5):
        M, R = 2, 4
        v0 = rng.random(R) - 0.5
        v1 = 2.0 * (rng.random(R) - 0.5)
        text = ORTHO_MTP.replace("\tradial_basis_size = 2", "\tradial_basis_size = 4")
        text = text.replace("\tradial_funcs_count = 3", "\tradial_funcs_count = 2")
        body = "\t\t\t{%s}\n\t\t\t{%s}\n" % (", ".join(repr(float(x)) for x in v0),
                                                  ", ".join(repr(float(x)) for x in v1))
        start = text.index("\t\t\t{3, 4}")
        end = text.index("alpha_moments_count")
        text = text[:start] + body + text[end:]
        text = text.replace("{{0, 0, 0, 0}, {1, 0, 0, 0}, {2, 0, 0, 0}}",
                            "{{0, 0, 0, 0}, {1, 0, 0, 0}, {1, 0, 0, 0}}")
        m = O.Model(text)
        assert (m.M, m.R) == (M, R)
        m.orthogonalize()
        out = m.coeffs[: m.nradial].reshape(M, R)
        c0 = v0 / np.sqrt(v0 @ v0 + 1e-10 * R)
        sc = v1 @ c0
        v1p = v1 - c0 * sc / (v1 @ v1)
        assert abs(v1p @ c0 - sc * (1 - (c0 @ c0) / (v1 @ v1))) < 1e-13
        assert np.abs(out[1] - v1p / np.sqrt(v1p @ v1p + 1e-10 * R)).max() < 1e-12
        assert abs(out[1] @ out[0]) > 1e-3 * abs(sc)


# --------------------------------------------------- loss weight factors --

def _loss_parts(m, nb, lab, **kw):
    st = O.LossSettings.make(**kw)
    loss, g, met = O.add_loss_grad(m, nb, st, lab)
    return loss, met


def test_force_normalisation_scales_every_term():
    """fit:force_wgt_d/f/p (train_mtp.cpp:3868-3880): with the label forces
    scaled so that mean_i |F*_i|^2 = 4, d = 0.1, f = 0.025, p = 2 the factor is
    0.1 / (0.1 + (0.025 * 4)^2) = 10/11, and it multiplies the energy, force
    and stress terms alike (never the predicted forces' norm)."""
    m, nb, lab = _config()
    F = lab.forces
    lab.forces = F * np.sqrt(4.0 / np.mean(np.sum(F * F, axis=1)))
    assert abs(np.mean(np.sum(lab.forces ** 2, axis=1)) - 4.0) < 1e-12
    for w in [(1.0, 0.0, 0.0), (0.0, 0.05, 0.0), (0.0, 0.0, 0.1), (1.0, 0.01, 1e-3)]:
        kw = dict(weight_eng=w[0], weight_force=w[1], weight_stress=w[2], force_norm_d=0.1,
                  force_norm_p=2.0)
        base, mb = _loss_parts(m, nb, lab, force_norm_f=0.0, **kw)
        norm, mn = _loss_parts(m, nb, lab, force_norm_f=0.025, **kw)
        assert abs(norm - base * 10.0 / 11.0) < 1e-13 * abs(base), w
        # metrics: [loss_e, loss_f, loss_s] scale, the squared errors do not
        assert np.allclose(mn[0:3], mb[0:3] * 10.0 / 11.0, rtol=1e-13, atol=0)
        assert np.array_equal(mn[3:6], mb[3:6])
    # the factor depends on the labels only: the same predicted forces with a
    # label set of half the norm give d / (d + (f * 1)^2) = 0.1 / 0.100625
    lab.forces = lab.forces * 0.5
    kw = dict(weight_eng=1.0, weight_force=0.0, weight_stress=0.0, force_norm_d=0.1,
              force_norm_p=2.0)
    base, _ = _loss_parts(m, nb, lab, force_norm_f=0.0, **kw)
    norm, _ = _loss_parts(m, nb, lab, force_norm_f=0.025, **kw)
    assert abs(norm - base * 0.1 / 0.100625) < 1e-13 * abs(base)


def test_fitness_scales_energy_only_and_atomic_fitness_forces_per_atom():
    """Atoms::fitness multiplies the energy weight only (train_mtp.cpp:2552-2556);
    atomic_fitness_i multiplies the force weight of atom i only (:3888-3893)."""
    m, nb, lab = _config()
    n = lab.n
    E, F, St, _ = O.efs(m, nb)
    for w in [(1.0, 0.0, 0.0), (0.0, 0.05, 0.0), (0.0, 0.0, 0.1)]:
        kw = dict(weight_eng=w[0], weight_force=w[1], weight_stress=w[2])
        base, _ = _loss_parts(m, nb, lab, **kw)
        lab.fitness = 3.0
        fit, _ = _loss_parts(m, nb, lab, **kw)
        lab.fitness = 1.0
        assert abs(fit - (3.0 if w[0] > 0 else 1.0) * base) < 1e-13 * abs(base), w
    # atomic fitness: an indicator of atom k leaves W_F |F_k - F*_k|^2
    kw = dict(weight_eng=0.0, weight_force=0.05, weight_stress=0.0)
    total = _loss_parts(m, nb, lab, **kw)[0]
    parts = []
    for k in [0, 3, n - 1]:
        a = np.zeros(n)
        a[k] = 1.0
        lab.atomic_fitness = a
        parts.append(_loss_parts(m, nb, lab, **kw)[0])
        assert abs(parts[-1] - 0.05 * np.sum((F[k] - lab.forces[k]) ** 2)) < 1e-15 + 1e-13 * parts[-1]
    lab.atomic_fitness = np.full(n, 2.5)
    assert abs(_loss_parts(m, nb, lab, **kw)[0] - 2.5 * total) < 1e-13 * total
    # energy and stress terms ignore atomic fitness
    kw = dict(weight_eng=1.0, weight_force=0.0, weight_stress=0.1)
    with_af = _loss_parts(m, nb, lab, **kw)[0]
    lab.atomic_fitness = None
    assert abs(with_af - _loss_parts(m, nb, lab, **kw)[0]) < 1e-13 * abs(with_af)


def test_energy_and_stress_powers():
    """W_X = w_X / N^p_X with the configured powers (train_mtp.cpp:2552-2568)."""
    m, nb, lab = _config()
    n = lab.n
    for key, pw in [("eng_pow", 0.0), ("eng_pow", 2.0), ("stress_pow", 0.5), ("force_pow", 1.5)]:
        kw = dict(weight_eng=1.0 if key == "eng_pow" else 0.0,
                  weight_force=0.05 if key == "force_pow" else 0.0,
                  weight_stress=0.1 if key == "stress_pow" else 0.0)
        default = {"eng_pow": 1.0, "stress_pow": 1.0, "force_pow": 0.0}[key]
        base, _ = _loss_parts(m, nb, lab, **kw)
        kw[key] = pw
        got, _ = _loss_parts(m, nb, lab, **kw)
        assert abs(got - base * n ** (default - pw)) < 1e-12 * abs(got), key


# --------------------------------------------- duplicate scalar mapping --

def _dup_case():
    text = S.random_model("dup-scalar.mtp", 2, 6, 1.8, 4.6, -0.5, 0.5, S.rng_for(700))
    rng = S.rng_for(701)
    s = S.displace(S.strain(S.lattice("bcc", (2, 2, 3), 2.87), rng, 0.03), rng, 0.15)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    return text, s


def test_duplicate_scalar_mapping_accumulates():
    """alpha_moment_mapping {0, 4, 5, 6, 4} (the moment graph of
    runtime/mtp/cpu/tests/test_mtp_cpu.cpp:30-33, with rules whose two
    operands are the same moment): the energy counts moment 4 with
    xi_1 + xi_4, and so must the adjoint seed (potential_mtp.cpp:2976, +=).
    Forces are minus the energy gradient."""
    text, s = _dup_case()
    m = O.Model(text)
    assert list(m.tables()[2]) == [0, 4, 5, 6, 4]
    E, F, St, se = _efs_of(m, s)
    # energy: replacing the duplicate by a single entry with the summed
    # coefficient leaves every output unchanged
    x = m.coeffs.copy()
    base = m.nradial + m.Z
    single = text.replace("alpha_scalar_moments = 5", "alpha_scalar_moments = 4")
    single = single.replace("alpha_moment_mapping = {0, 4, 5, 6, 4}",
                            "alpha_moment_mapping = {0, 4, 5, 6}")
    mc = x[base:]
    lines = single.splitlines()
    for i, l in enumerate(lines):
        if l.startswith("moment_coeffs"):
            merged = [mc[0], mc[1] + mc[4], mc[2], mc[3]]
            lines[i] = "moment_coeffs = {%s}" % ", ".join(repr(float(v)) for v in merged)
    m1 = O.Model("\n".join(lines) + "\n")
    E1, F1, S1, se1 = _efs_of(m1, s)
    assert rel_err(E, E1) < 1e-13 and rel_err(F, F1) < 1e-12 and rel_err(St, S1) < 1e-12
    h = 1e-5
    for i in range(0, s.n, 5):
        for a in range(3):
            p1 = s.pos.copy()
            p1[i, a] += h
            p2 = s.pos.copy()
            p2[i, a] -= h
            fd = -(_efs_of(m, s, p1)[0] - _efs_of(m, s, p2)[0]) / (2 * h)
            assert abs(F[i, a] - fd) < 1e-7 * max(1.0, np.abs(F).max())
