"""mtpx_train_lbfgs (Trainer_MTP::TrainNonLinearLBFGS, train/train_mtp.cpp:
4256-4339) on the device against the same iteration driven from the host:
the reference's LBFGSpp (oracle/_ref/liblbfgs_ref.so) when it is built, and
the product's own host solver (pinned against it on the CPU) otherwise, both
over the oracle's loss and gradient in Trainer_MTP::operator()'s form --
coefficients x / scaling, gradient times scaling, x / scaling left in the
solver's iterate.

The device objective agrees with the oracle to about 1e-14 relative, so the
trajectories stay together over a few iterations: objective values of every
evaluation to 1e-9 relative, final coefficients to 1e-7."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from mtpx import capi
from test_train_gpu import SETTINGS, _dataset, _upload

pytestmark = pytest.mark.gpu

PEN = dict(penalty_weight=1e-3, reg_l2=1e-4, reg_l1=0.0)


def trainer_scaling(x):
    """Trainer_MTP::TrainLBFGS's per-coefficient scaling (train_mtp.cpp:4391-4403)."""
    a = np.abs(x)
    s = 1.0 / np.where(a == 0, 1.0, a)
    s = np.where(a > 1e4, 1e-4, s)
    s = np.where(a < 1e-1, 10.0, s)
    s = np.where(a < 1e-2, 100.0, s)
    return np.where(a < 1e-6, 1e6, s)


@pytest.fixture(scope="module")
def small_set():
    return _dataset(4, 3, 5)


def host_run(model, nbs, labels, settings, x0, scale, params, unscale, use_ref):
    """(ok, message, x, iterations, f, objective history) of the host solver."""
    hist = []

    def fg(x):
        c = x / scale
        model.coeffs = c
        f, g = O.loss_grad_batch(model, nbs, labels, settings, threads=8, **PEN)
        hist.append(f)
        return (f, g * scale, c) if unscale else (f, g * scale)
    if use_ref:
        ok, x, it, f, ev, msg = O.ref_lbfgs(fg, x0, O.RefLbfgsParams.default(**params))
    else:
        rc, x, it, f, ev, msg = capi.lbfgs_minimize(fg, x0, capi.LbfgsParams.default(**params))
        ok = rc == capi.OK
    return ok, msg, x, it, f, np.array(hist)


@pytest.mark.parametrize("scaling", ["ones", "trainer"])
@pytest.mark.parametrize("unscale", [1, 0])
@pytest.mark.parametrize("use_ref", [True, False])
def test_train_lbfgs_follows_the_host_solver(ctx, small_set, scaling, unscale, use_ref):
    """Same evaluations, same outcome.  With the trainer's scaling and the
    trainer's in-place division (unscale 1) the line search starts from
    x / scaling rather than x, and the reference's solver may stop with
    "exceed max linesearch": the device run must stop the same way, at the
    same evaluation."""
    if use_ref and not O.ref_available("liblbfgs_ref.so"):
        pytest.skip("oracle/_ref/liblbfgs_ref.so not built")
    text, cutoff, structs, nbs, labels = small_set
    st = SETTINGS["default"]
    _upload(ctx, text, cutoff, structs, labels, st)
    c0 = ctx.get_coeffs()
    scale = np.ones_like(c0) if scaling == "ones" else trainer_scaling(c0)
    params = dict(max_iterations=3, unscale_iterate=unscale)
    rc, msg, it, loss, hist, ev, x = ctx.train_lbfgs(
        capi.LbfgsParams.default(**params), scaling=scale, deterministic=True,
        raise_on_error=False, **PEN)
    m = O.Model(text)
    ok, msg_r, xr, itr, fr, hr = host_run(m, nbs, labels, st, c0 * scale, scale, params, unscale,
                                          use_ref)
    assert (rc == capi.OK) == ok and msg == msg_r
    assert ev == len(hr) and len(hist) == ev
    assert np.all(np.abs(hist - hr) <= 1e-9 * np.abs(hr))
    if scaling == "ones" or not unscale:
        assert ok, msg   # the consistent form descends from a sound start
    if not ok:
        assert rc == capi.ERRORS_BY_NAME["MTPX_E_SOLVER"]
        return
    assert it == itr
    assert rel_err(loss, fr) < 1e-9
    assert rel_err(x, xr) < 1e-7
    # the context keeps the coefficients of the last evaluation
    last = x if unscale else x / scale
    assert np.array_equal(ctx.get_coeffs(), last)
    # the loss went down from the start
    assert hist[-1] < hist[0]


def test_train_lbfgs_explicit_start_and_errors(ctx, small_set):
    text, cutoff, structs, nbs, labels = small_set
    _upload(ctx, text, cutoff, structs, labels, SETTINGS["default"])
    c0 = ctx.get_coeffs()
    # an explicit starting point equal to the default one gives the same run
    a = ctx.train_lbfgs(capi.LbfgsParams.default(max_iterations=2), deterministic=True, **PEN)
    ctx.set_coeffs(c0)
    b = ctx.train_lbfgs(capi.LbfgsParams.default(max_iterations=2), x=c0, deterministic=True,
                        **PEN)
    assert a[:2] == b[:2] and np.array_equal(a[2], b[2]) and np.array_equal(a[4], b[4])
    # a failed line search reports the solver's text and keeps the context usable
    ctx.set_coeffs(c0)
    with pytest.raises(capi.MtpxError) as e:
        ctx.train_lbfgs(capi.LbfgsParams.default(max_linesearch=1, first_initial_step=1e3),
                        deterministic=True, **PEN)
    assert "exceed max linesearch" in str(e.value)
    f, g, _ = ctx.loss_grad(deterministic=True, **PEN)
    assert np.isfinite(f)
    with pytest.raises(capi.MtpxError):
        ctx.train_lbfgs(capi.LbfgsParams.default(m=0))
    with pytest.raises(capi.MtpxError):
        ctx.train_lbfgs(scaling=np.zeros(c0.size))
