"""The L-BFGS solver of the C ABI (mtpx_lbfgs_minimize, host code) against
the reference's vendored LBFGSpp -- LBFGSSolver<double, LineSearchLewisOverton>
compiled from deplibs/LBFGSpp/include into oracle/_ref/liblbfgs_ref.so -- on
the same objectives, plus what the mathematics fixes.

The two differ only in the order of the sums inside dot products and norms
(Eigen's packet reductions), so a two-dimensional problem, where both sum
the same two terms, is compared bit for bit; larger problems compare the
objective values of the first evaluations to 1e-9 relative and the final
points to what the stopping tolerance allows."""
import numpy as np
import pytest

import oracle as O
from mtpx import capi

needs_ref = pytest.mark.skipif(not O.ref_available("liblbfgs_ref.so"),
                               reason="oracle/_ref/liblbfgs_ref.so not built")


def rosenbrock(x):
    f = np.sum(100.0 * (x[1:] - x[:-1] ** 2) ** 2 + (1.0 - x[:-1]) ** 2)
    g = np.zeros_like(x)
    g[:-1] += -400.0 * x[:-1] * (x[1:] - x[:-1] ** 2) - 2.0 * (1.0 - x[:-1])
    g[1:] += 200.0 * (x[1:] - x[:-1] ** 2)
    return f, g


def quartic(n, seed):
    """0.5 x'Ax - b'x + 0.25 sum x^4 with A SPD: one minimum, A x - b + x^3 = 0."""
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((n, n))
    A = A @ A.T / n + np.eye(n)
    b = rng.standard_normal(n)

    def fg(x):
        return 0.5 * x @ A @ x - b @ x + 0.25 * np.sum(x ** 4), A @ x - b + x ** 3
    return fg, rng.standard_normal(n)


def recorded(fg, hist):
    def w(x):
        r = fg(x)
        hist.append(r[0])
        return r
    return w


def both(fg, x0, **kw):
    hr, hp = [], []
    r = O.ref_lbfgs(recorded(fg, hr), x0, O.RefLbfgsParams.default(**kw))
    p = capi.lbfgs_minimize(recorded(fg, hp), x0, capi.LbfgsParams.default(**kw))
    return r, p, np.array(hr), np.array(hp)


def test_defaults_are_lbfgsparam():
    p = capi.LbfgsParams.default()
    r = O.RefLbfgsParams.default()
    for name, _ in capi.LbfgsParams._fields_:
        assert getattr(p, name) == getattr(r, name), name


def test_rosenbrock_converges():
    """Known answer: the Rosenbrock minimum (1, 1) to the gradient tolerance
    (|g| <= max(epsilon, epsilon_rel |x|))."""
    rc, x, it, f, ev, msg = capi.lbfgs_minimize(rosenbrock, np.array([-1.2, 1.0]))
    assert rc == capi.OK and msg == ""
    assert np.linalg.norm(rosenbrock(x)[1]) <= 1e-5 * max(1.0, np.linalg.norm(x))
    assert np.abs(x - 1.0).max() < 1e-5 and f < 1e-10
    assert ev >= it


@needs_ref
def test_rosenbrock_2d_bitwise():
    r, p, hr, hp = both(rosenbrock, np.array([-1.2, 1.0]))
    assert r[0] and p[0] == capi.OK
    assert (r[2], r[4]) == (p[2], p[4])
    assert np.array_equal(hr, hp)
    assert np.array_equal(r[1], p[1]) and r[3] == p[3]


@needs_ref
@pytest.mark.parametrize("m", [3, 6, 12])
def test_rosenbrock_10d(m):
    x0 = np.array([-1.2 if i % 2 == 0 else 1.0 for i in range(10)])
    r, p, hr, hp = both(rosenbrock, x0, m=m)
    assert r[0] and p[0] == capi.OK
    k = min(20, len(hr), len(hp))
    assert np.all(np.abs(hr[:k] - hp[:k]) <= 1e-9 * np.abs(hr[:k]))
    assert np.abs(r[1] - p[1]).max() < 1e-4   # both at the minimum to the tolerance
    assert abs(r[2] - p[2]) <= 2


@needs_ref
@pytest.mark.parametrize("n,seed", [(5, 1), (40, 2), (200, 3)])
def test_quartic(n, seed):
    fg, x0 = quartic(n, seed)
    r, p, hr, hp = both(fg, x0)
    assert (r[2], r[4]) == (p[2], p[4])
    assert np.all(np.abs(hr - hp) <= 1e-12 * np.abs(hr))
    assert np.abs(r[1] - p[1]).max() < 1e-10
    # the stationarity condition the minimum satisfies
    assert np.linalg.norm(fg(p[1])[1]) <= 1e-5 * max(1.0, np.linalg.norm(p[1]))


@needs_ref
@pytest.mark.parametrize("kw", [dict(max_iterations=3), dict(past=2, delta=1e-3),
                                dict(epsgmax=1e-2), dict(initial_step=0.5),
                                dict(first_initial_step=0.01), dict(max_step_move=0.05),
                                dict(epsilon_rel=1e-2)])
def test_stopping_rules_and_steps(kw):
    x0 = np.array([-1.2, 1.0])
    r, p, hr, hp = both(rosenbrock, x0, **kw)
    assert r[0] and p[0] == capi.OK
    assert (r[2], r[4]) == (p[2], p[4])
    assert np.array_equal(hr, hp) and np.array_equal(r[1], p[1])


@needs_ref
def test_scaled_objective_overwriting_the_iterate():
    """Trainer_MTP::operator()'s form: coefficients x / s, gradient times s,
    and x / s left in the solver's iterate."""
    fg0, x0 = quartic(2, 5)
    s = np.array([10.0, 0.25])

    def fg(x):
        c = x / s
        f, g = fg0(c)
        return f, g * s, c
    r, p, hr, hp = both(fg, x0 * s, max_iterations=8)
    assert (r[2], r[4]) == (p[2], p[4])
    assert np.array_equal(hr, hp) and np.array_equal(r[1], p[1])


@needs_ref
def test_failures_carry_the_solvers_messages():
    # one evaluation per line search is too few for Rosenbrock's first step
    r, p, _, _ = both(rosenbrock, np.array([-1.2, 1.0]), max_linesearch=1)
    assert not r[0] and p[0] == -9
    assert p[5] == r[5] == "exceed max linesearch"

    def nan_after_start(x):
        f, g = rosenbrock(x)
        return (f if np.array_equal(x, [-1.2, 1.0]) else np.nan), g
    r, p, _, _ = both(nan_after_start, np.array([-1.2, 1.0]))
    assert not r[0] and p[0] == -9 and p[5] == r[5] == "inf or nan"


@needs_ref
@pytest.mark.parametrize("kw", [dict(m=0), dict(epsilon=-1.0), dict(past=-1),
                                dict(max_linesearch=0), dict(max_step=1e-30),
                                dict(f_dec_coeff=1.0), dict(s_curv_coeff=1e-5)])
def test_parameter_checks(kw):
    r, p, _, _ = both(rosenbrock, np.array([-1.2, 1.0]), **kw)
    assert not r[0] and p[0] == capi.ERRORS_BY_NAME["MTPX_E_INVALID"]
    assert p[5] == r[5]


def test_objective_status_stops_the_solver():
    def bad(x):
        raise ValueError("no")
    rc, x, it, f, ev, msg = capi.lbfgs_minimize(bad, np.array([1.0, 2.0]))
    assert rc == capi.ERRORS_BY_NAME["MTPX_E_INVALID"] and "status" in msg
