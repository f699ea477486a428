"""MTP-M potentials on the device (the head of Executor::evaluate_site,
runtime/mtp/cpu/mtp_cpu.cpp:291-442, fused into the E/F/S kernel) against
the oracle, itself pinned to the reference executor in test_mtpm: E/F/S and
site energies at 1e-11 relative in both force modes, energies only, batches
of structures, ghost-atom site requests and calc_efs; coefficient updates;
heads wider than a wave (descriptors, hidden units > 64); the refusals of
the training and linear-fit entry points."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from helpers import assert_efs_close, oracle_case, rel_err, upload_oracle_lists
from mtpx import capi
from mtpx import synth as S
from test_mtpm import CASES, case_id, head_text, structure

pytestmark = pytest.mark.gpu
TOL = 1e-11


@pytest.mark.parametrize("case", CASES, ids=case_id)
def test_efs_matches_oracle(ctx, case):
    head, h1, h2, act = case
    text = head_text(head, h1, h2, act)
    ref = oracle_case(text, structure())
    ctx.load_model_text(text)
    got = ctx.model_head()
    assert (got["head"], got["hidden1"], got["hidden2"]) == (head, h1, h2)
    upload_oracle_lists(ctx, ref["nb"])
    assert_efs_close(ctx.efs(), ref, TOL)
    assert_efs_close(ctx.efs(deterministic=True), ref, TOL)
    E, se = ctx.energy()
    assert rel_err(E[0], ref["E"]) < TOL and rel_err(se, ref["se"]) < TOL


@pytest.mark.parametrize("case", [CASES[1], CASES[5], CASES[8]], ids=case_id)
def test_level16_graph_and_device_lists(ctx, case):
    """The level-16 moment graph (its compile-time kernel profile) with a
    head, lists built on the device."""
    head, h1, h2, act = case
    base = S.random_model("shapeev-16.mtp", 2, 8, 1.9, 5.0, -0.05, 0.05, S.rng_for(50))
    text = head_text(head, h1, h2, act, base=base, seed=51)
    s = structure(52, (3, 3, 3))
    ref = oracle_case(text, s)
    ctx.load_model_text(text)
    ctx.build_neighbors(s.cell, s.pbc, ref["pos"], s.types, ref["model"].cutoff)
    assert_efs_close(ctx.efs(), ref, TOL)
    assert_efs_close(ctx.efs(deterministic=True), ref, TOL)


@pytest.mark.parametrize("head,q,h1,h2,act", [("mtp_m_n1", 70, 80, 0, "SIGMOID"),
                                              ("mtp_m_n2", 67, 70, 66, "TANH")])
def test_heads_wider_than_a_wave(ctx, head, q, h1, h2, act):
    """Descriptors and hidden units beyond 64 lanes take the strided loops."""
    text = S.mtpm_model(S.random_model("shapeev-10.mtp", 2, 6, 2.0, 5.0, -0.1, 0.1,
                                       S.rng_for(54)), head, S.rng_for(55), q=q, h1=h1, h2=h2,
                        activation=act, head_lo=-0.1, head_hi=0.1)
    ref = oracle_case(text, structure(56))
    ctx.load_model_text(text)
    assert ctx.model_head()["q"] == q
    upload_oracle_lists(ctx, ref["nb"])
    assert_efs_close(ctx.efs(), ref, TOL)


def test_coefficient_update_and_save(ctx):
    text = head_text("mtp_m_n2", 4, 3, "SIGMOID")
    m = O.Model(text)
    s = structure(57)
    ref = oracle_case(text, s)
    ctx.load_model_text(text)
    upload_oracle_lists(ctx, ref["nb"])
    x = ctx.get_coeffs()
    assert np.array_equal(x, m.coeffs)
    x2 = x * (1.0 + 0.1 * S.uniform(S.rng_for(58), x.size, -1.0, 1.0))
    ctx.set_coeffs(x2)
    m.coeffs = x2
    E, F, St, se = O.efs(m, ref["nb"])
    assert_efs_close(ctx.efs(), dict(E=E, F=F, S=St, se=se), TOL)
    saved = ctx.save_model_text()
    assert np.array_equal(O.Model(saved).coeffs, x2)
    assert capi.parse_model_head(saved) == ctx.model_head()


def test_batch_of_structures(ctx):
    text = head_text("mtp_m_fs", seed=59)
    m = O.Model(text)
    structs = [structure(60 + k, (2, 2, 2 + k)) for k in range(3)]
    ctx.load_model_text(text)
    off = ctx.set_structures(structs, m.cutoff)
    for det in (False, True):
        E, F, St, se = ctx.compute_batch(deterministic=det)
        for c, s in enumerate(structs):
            ref = oracle_case(text, s)
            assert rel_err(E[c], ref["E"]) < TOL and rel_err(St[c], ref["S"]) < TOL
            assert rel_err(F[off[c]:off[c + 1]], ref["F"]) < TOL
            assert rel_err(se[off[c]:off[c + 1]], ref["se"]) < TOL


def test_ghost_site_request(ctx):
    """mtpx_compute_sites over owned atoms plus periodic images as ghosts
    (the request of the LAMMPS pair style)."""
    from test_sites_gpu import fold, ghost_system
    text = head_text("mtp_m_n1", 4, 0, "TANH", seed=61)
    m = O.Model(text)
    s = structure(62)
    g = ghost_system(m, s)
    ref = oracle_case(text, s)
    ctx.load_model_text(text)
    out = ctx.compute_sites(g["offsets"], g["neighbors"], g["types"], x=g["pts"], nlocal=g["n"])
    assert rel_err(out["energy"], ref["E"]) < TOL
    assert rel_err(out["site_energy"], ref["se"]) < TOL
    assert rel_err(fold(out["force"], g["orig"], g["n"]), ref["F"]) < TOL
    St = ref["S"]
    sym = 0.5 * (St + St.T)
    v6 = np.array([sym[0, 0], sym[1, 1], sym[2, 2], sym[0, 1], sym[0, 2], sym[1, 2]])
    assert rel_err(out["virial6"], v6) < TOL


def test_calc_efs_front_end(tmp_path):
    from test_calc_efs_gpu import EXE, _read_cfg, _write_cfg
    if not os.path.exists(EXE):
        pytest.fail("mtpx_calc_efs is not built")
    text = head_text("mtp_m_q2", seed=63)
    mtp = tmp_path / "pot.mtp"
    mtp.write_text(text)
    structs = [structure(64), structure(65, (2, 2, 3))]
    cfg = tmp_path / "in.cfg"
    _write_cfg(cfg, structs)
    out = tmp_path / "out.cfg"
    r = subprocess.run([EXE, "--pot", str(mtp), "--in", str(cfg), "--out", str(out), "--lossless"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    for s, got in zip(structs, _read_cfg(out)):
        ref = oracle_case(text, s)
        c = got["cols"]
        assert rel_err(got["energy"], ref["E"]) < 1e-10
        assert rel_err(np.stack([c["fx"], c["fy"], c["fz"]], 1), ref["F"]) < 1e-10
        assert rel_err(c["site_en"], ref["se"]) < 1e-10


def test_training_entry_points_refuse_heads(ctx):
    text = head_text("mtp_m_q2", seed=66)
    m = O.Model(text)
    structs = [structure(67)]
    ctx.load_model_text(text)
    ctx.set_structures(structs, m.cutoff)
    code = capi.ERRORS_BY_NAME["MTPX_E_MODEL"]
    calls = [lambda: ctx.loss_grad(), lambda: ctx.efs_components(), lambda: ctx.linear_rows(),
             lambda: ctx.linear_system(), lambda: ctx.train_lbfgs(),
             lambda: ctx.penalty(1e-3, 0.0, 0.0), lambda: ctx.accumulate_gradient()]
    for call in calls:
        with pytest.raises(capi.MtpxError) as e:
            call()
        assert e.value.code == code, e.value
    # evaluation still works afterwards
    E, F, St, se = ctx.compute_batch()
    ref = oracle_case(text, structs[0])
    assert rel_err(E[0], ref["E"]) < TOL
