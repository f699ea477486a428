"""Split and non-Chebyshev radial bases on the device against the oracle
(itself pinned to the reference core in test_model_io): E/F/S at 1e-10,
loss and gradient at 1e-9, linear-fit components at 1e-10; the context's
PotMTP::Save text after a coefficient update."""
import numpy as np
import pytest

import oracle as O
from helpers import assert_efs_close, oracle_case, rel_err, upload_oracle_lists
from mtpx import capi
from mtpx import synth as S
from test_model_io import BASES, model_text

pytestmark = pytest.mark.gpu


def _bcc(seed, reps=(3, 3, 3)):
    rng = S.rng_for(seed)
    s = S.displace(S.strain(S.lattice("bcc", reps, 2.87), rng, 0.03), rng, 0.15)
    s.types = (S.uniform(rng, s.n) * 2).astype(np.int32)
    return s


@pytest.mark.parametrize("kind", list(BASES))
def test_efs_matches_oracle(ctx, kind):
    text = model_text(kind)
    ref = oracle_case(text, _bcc(730))
    ctx.load_model_text(text)
    upload_oracle_lists(ctx, ref["nb"])
    assert_efs_close(ctx.efs(), ref, 1e-10)
    assert_efs_close(ctx.efs(deterministic=True), ref, 1e-10)
    # lists built on the device with the model's (largest) cutoff
    m = ref["model"]
    ctx.build_neighbors(_bcc(730).cell, _bcc(730).pbc, ref["pos"], _bcc(730).types, m.cutoff)
    assert_efs_close(ctx.efs(), ref, 1e-10)


@pytest.mark.parametrize("kind", ["split", "chebycos", "poly5", "configurable"])
def test_level16_structure_with_general_bases(ctx, kind):
    """The level-16 moment graph on a general basis runs the run-time
    profile kernels (not the compile-time level-16 ones)."""
    text = model_text(kind, template="shapeev-16.mtp", seed=731)
    ref = oracle_case(text, _bcc(732, (3, 3, 4)))
    ctx.load_model_text(text)
    upload_oracle_lists(ctx, ref["nb"])
    assert_efs_close(ctx.efs(), ref, 1e-10)


@pytest.mark.parametrize("kind", ["split", "chebycos", "poly4", "configurable", "split-configurable"])
def test_loss_grad_matches_oracle(ctx, kind):
    text = model_text(kind, seed=733)
    ref_text = model_text(kind, seed=734)
    m, mref = O.Model(text), O.Model(ref_text)
    rng = S.rng_for(735)
    structs, nbs, labels = [], [], []
    for k in range(3):
        s = _bcc(736 + k, (2, 2, 2 + k))
        s.pos = O.wrap(s.cell, s.pbc, s.pos)
        nb = O.Neighbors.build(s.cell, s.pbc, s.pos, s.types, mref.cutoff)
        E, F, St, _ = O.efs(mref, nb)
        e, f, sv = S.noisy_labels(rng, s.n, E, F, St)
        structs.append(s)
        nbs.append(nb)
        labels.append(O.Labels(s.n, energy=e, forces=f, stress=sv))
    st = O.LossSettings.make()
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, m.cutoff)
    has = np.ones((len(structs), 3), np.int32)
    tf = np.concatenate([lb.forces for lb in labels])
    active, wE, wF, wS = capi.loss_weights(capi.LossSettings.make(), off, has, tf)
    ctx.set_labels(active, np.array([lb.energy for lb in labels]), wE, tf, wF,
                   np.array([lb.stress for lb in labels]), wS)
    f_o, g_o = O.loss_grad_batch(m, nbs, labels, st, penalty_weight=1e-4, reg_l2=1e-6, threads=4)
    f, g, _ = ctx.loss_grad(penalty_weight=1e-4, reg_l2=1e-6)
    assert rel_err(f, f_o) < 1e-9 and rel_err(g, g_o) < 1e-9
    ec, fc, sc = ctx.efs_components()
    for c, nb in enumerate(nbs):
        eo, fo, so = O.efs_components(m, nb)
        assert rel_err(ec[c], eo) < 1e-10 and rel_err(sc[c], so) < 1e-10
        assert rel_err(fc[off[c]:off[c + 1]], fo) < 1e-10


def test_save_after_coefficient_update(ctx):
    text = model_text("split")
    ctx.load_model_text(text)
    x = ctx.get_coeffs() * 1.5
    ctx.set_coeffs(x)
    saved = ctx.save_model_text()
    m = O.Model(text)
    m.coeffs = x
    assert saved == m.save_text()
    assert capi.format_model_text(saved) == saved
